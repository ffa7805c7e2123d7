"""CPU oracle for the block-wise FP8 and paged-KV hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
package: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or as
the timed CPU baseline), never as the thing measured on the GPU.

Modules
  fp8       -- e4m3fn codec, act_quant, 128x128 weight quant, weight_dequant,
               block-scaled fp8_gemm (numpy, float32/float64)
  paged_kv  -- store_kvcache, paged-attention decode, SDPA, slot mapping

Every function cites the reference file:line it restates.  Parity status of
each function (what pins it) is written in its docstring.
"""
