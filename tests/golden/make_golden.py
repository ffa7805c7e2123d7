"""Write tests/golden/sdpa_snapshots.npz from the reference's own test data.

Run once in a container that has the reference checkout (it is not needed at
test time):

    python tests/golden/make_golden.py /root/reference

Inputs are regenerated exactly as the reference's fixtures do
(tests/conftest.py:253-280 there: torch.manual_seed(1|2|3) then randn of
(batch=4, queries=12 / keys=16, d_model=64), mask = randn(4,12,16) > 0.5 after
seed 5).  Expected outputs are the arrays of the reference's snapshot files
tests/_snapshots/test_scaled_dot_product_attention.npz and
test_4d_scaled_dot_product_attention.npz (data, copied as-is).  Nothing of
the reference's code is imported or run.
"""
import sys
from pathlib import Path

import numpy as np
import torch


def main(ref_root: str) -> None:
    snap = Path(ref_root) / "tests" / "_snapshots"
    exp3 = np.load(snap / "test_scaled_dot_product_attention.npz")["array"]
    exp4 = np.load(snap / "test_4d_scaled_dot_product_attention.npz")["array"]
    torch.manual_seed(1)
    q = torch.randn(4, 12, 64)
    torch.manual_seed(2)
    k = torch.randn(4, 16, 64)
    torch.manual_seed(3)
    v = torch.randn(4, 16, 64)
    torch.manual_seed(5)
    mask = torch.randn(4, 12, 16) > 0.5
    out = Path(__file__).with_name("sdpa_snapshots.npz")
    np.savez_compressed(out, q=q.numpy(), k=k.numpy(), v=v.numpy(), mask=mask.numpy(),
                        expected_3d=exp3, expected_4d=exp4)
    print(f"wrote {out}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
