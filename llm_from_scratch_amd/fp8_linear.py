"""FP8Linear: drop-in for the nn.Linear sites of the decode path.

The reference model builds its projections with nn.Linear(bias=True)
(model/attention/GQA.py:34-37, model/architecture/mlp.py:56-58, the MoE
experts via MLP, model/architecture/moe.py:179-182, and lm_head,
model/transformer.py:160).  FP8Linear holds the weight quantised once to
e4m3fn with 128x128 block scales (weight_quant) and runs
    y = fp8_gemm(act_quant(x, 128), W_q, W_s) + bias
with the bias added in the fp32 accumulator before the single rounding to
bf16.  in_features must be a multiple of 128.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
from torch import nn

from . import kernels


class FP8Linear(nn.Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = True, device=None):
        super().__init__()
        assert in_features % 128 == 0, "FP8Linear needs in_features % 128 == 0"
        self.in_features = in_features
        self.out_features = out_features
        dev = torch.device(device) if device is not None else torch.device("cuda")
        self.register_buffer("weight", torch.zeros(out_features, in_features, dtype=kernels.FP8, device=dev))
        self.register_buffer("weight_scale", torch.ones(math.ceil(out_features / 128), in_features // 128,
                                                        dtype=torch.float32, device=dev))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float32, device=dev))
        else:
            self.bias = None

    @torch.no_grad()
    def load_weight(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> "FP8Linear":
        """Quantise a [out, in] weight (any float dtype, rounded to bf16 first)
        with 128x128 block scales."""
        w = weight.to(device=self.weight.device, dtype=torch.bfloat16).contiguous()
        assert w.shape == (self.out_features, self.in_features)
        q, s = kernels.weight_quant(w, 128)
        self.weight.copy_(q)
        self.weight_scale.copy_(s)
        if self.bias is not None and bias is not None:
            self.bias.copy_(bias.to(torch.float32))
        return self

    @classmethod
    def from_linear(cls, linear: nn.Linear, device=None) -> "FP8Linear":
        m = cls(linear.in_features, linear.out_features, linear.bias is not None,
                device=device or linear.weight.device)
        return m.load_weight(linear.weight, linear.bias)

    def dequantized_weight(self) -> torch.Tensor:
        return kernels.weight_dequant(self.weight, self.weight_scale, 128)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x.to(torch.bfloat16).contiguous()
        if self.fused_act(x.numel() // self.in_features):
            # act_quant inside the GEMM's workgroups: the same codes, scales and bits
            return kernels.fp8_gemm_act(x, self.weight, self.weight_scale, self.bias)
        xq, xs = kernels.act_quant(x, 128)
        return self.gemm(xq, xs)

    def fused_act(self, rows: int) -> bool:
        """Whether forward on `rows` input rows quantises them inside the
        GEMM (the one-shot shapes that fp8_gemm runs in one split)."""
        M, N, K = rows, self.out_features, self.in_features
        return (kernels.fp8_gemm_act_supported(M, N, K) and not kernels.use_skinny_gemm(M, N, K)
                and kernels.default_gemm_splits(M, N, K) == 1)

    def gemm(self, xq: torch.Tensor, xs: torch.Tensor) -> torch.Tensor:
        """The linear on an input already quantised by act_quant (codes and
        1x128 scales), e.g. by a fused norm."""
        return kernels.fp8_gemm(xq, xs, self.weight, self.weight_scale, self.bias)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}, fp8=e4m3fn/128x128"
