"""Softmax / DFL oracle: PyTorch CPU (test infrastructure only).

  softmax(x, dim, half_to_float) -- torch.softmax on CPU in x's dtype;
      half_to_float is the fp32 softmax of the fp16 input (verify_softmax.py:48-53
      uses the same expectation for aten::_softmax(..., True)).  Reference
      kernels: softmax.cpp:6-173 (generic), softmax.cpp:175-271 (DFL view).
  softmax_rounded(x, dim) -- fp32 softmax rounded once to x's dtype: the
      correctly rounded reference the <= 1e-3 relative bar is measured
      against (CPU's own fp16 softmax over a non-last dim sits up to ~1.9 fp16
      ulp from it; the reference's test compares with CPU at 1e-3 absolute,
      verify_softmax.py:57).
  dfl_expect(x, out_dtype) -- fused DFL: fp32 softmax over the 16 bins of each
      side of [N,64,A], dot with arange(16), one cast (whole_blocked.py:137 with
      the DFL 1x1 conv of weights arange(16), model_optimization.py:20-31).
  dfl_expect_unfused(x) -- the reference's two-step chain: fp16 probabilities,
      then the fp32-accumulated arange(16) dot rounded to fp16.

Pinning (tests/test_oracle_reductions.py): float64 numpy softmax within 1e-6
relative for fp32 and the fp16 rounding bound for fp16; NaN/inf masks derived
from the IEEE rules by hand; sum-to-one and expectation range invariants; a
one-hot DFL case whose expectation is the hot bin.
"""
from __future__ import annotations

import torch


def softmax(x: torch.Tensor, dim: int, half_to_float: bool = False) -> torch.Tensor:
    if half_to_float:
        return torch.softmax(x.float(), dim)
    return torch.softmax(x, dim)


def softmax_rounded(x: torch.Tensor, dim: int) -> torch.Tensor:
    return torch.softmax(x.float(), dim).to(x.dtype)


def dfl_expect(x: torch.Tensor, out_dtype=torch.float16) -> torch.Tensor:
    n, c, a = x.shape
    p = torch.softmax(x.float().view(n, c // 16, 16, a), 2)
    w = torch.arange(16, dtype=torch.float32).view(1, 1, 16, 1)
    return (p * w).sum(2).to(out_dtype)


def dfl_expect_unfused(x: torch.Tensor) -> torch.Tensor:
    n, c, a = x.shape
    p = torch.softmax(x.view(n, c // 16, 16, a).transpose(1, 2), 1)  # fp16 [N,16,4,A]
    w = torch.arange(16, dtype=torch.float32).view(1, 16, 1, 1)
    return (p.float() * w).sum(1).to(torch.float16)
