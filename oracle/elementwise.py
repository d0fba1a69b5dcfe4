"""Elementwise oracle: the reference's PyTorch CPU implementation of each op.

The reference's own tests check every device op against stock PyTorch CPU on
the same seeded inputs (verify_ops.py:74, verify_strided_binary.py:18-57,
verify_all.py:76-81); these functions are those CPU op sequences.

Pinning (tests/test_oracle_elementwise.py):
  binary_*      -- (binary, binary_scalar, binary_scalar_rounded)
                   bit-exact against float64 numpy evaluation rounded once to
                   fp16 (exact sums/products; division double rounding is
                   innocuous at 53 >= 2*11+2), i.e. the correctly rounded result.
  sigmoid/silu  -- within 1 fp16 ulp of a float64 evaluation; NaN/inf cases.
  silu_add      -- within 1 ulp of float64 y + x/(1+e^-x) rounded once.
  affine_silu   -- fp16 intermediates equal the pinned mul/add; final SiLU
                   within 1 ulp of float64.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

OPS = {0: "sub", 1: "mul", 2: "div", 3: "add"}


def binary(op: int, x: torch.Tensor, y: torch.Tensor, alpha: float = 1.0) -> torch.Tensor:
    """x op y on CPU in x's dtype (ops.cpp:464-497 semantics: broadcast via
    infer_size, alpha scales the second operand of add/sub).

    For alpha != 1 this is PyTorch CPU's vectorized rule restated: alpha is
    rounded to the tensor dtype, x + alpha*y is evaluated in fp32 and cast once
    (CPU's scalar tail loop at each parallel-chunk end evaluates differently;
    the restatement follows the vectorized loop that covers the rest)."""
    name = OPS[op]
    if name in ("add", "sub") and alpha != 1.0:
        a = torch.tensor(alpha, dtype=x.dtype).float()
        xf, yf = x.float(), y.float()
        r = xf + a * yf if name == "add" else xf - a * yf
        return r.to(x.dtype)
    if name in ("add", "sub"):
        return getattr(torch, name)(x, y)
    return getattr(torch, name)(x, y)


def binary_scalar(op: int, x: torch.Tensor, scalar: float, scalar_first: bool = False,
                  alpha: float = 1.0) -> torch.Tensor:
    """Tensor op Python number on CPU.  PyTorch CPU rounds the number to the
    tensor dtype for add/sub/rsub and keeps it at fp32 for mul/div (the
    reference rounds it to the tensor dtype for every op, ops.cpp:466-467)."""
    name = OPS[op]
    if scalar_first:
        if name == "sub":
            return torch.rsub(x, scalar, alpha=alpha)
        if name == "add":
            return torch.add(x, scalar, alpha=1.0) if alpha == 1.0 else \
                (x.float() * torch.tensor(alpha, dtype=x.dtype).float()
                 + torch.tensor(scalar, dtype=x.dtype).float()).to(x.dtype)
        if name == "mul":
            return torch.mul(x, scalar)
        return (torch.tensor(scalar, dtype=torch.float32) / x.float()).to(x.dtype)
    if name in ("add", "sub"):
        return getattr(torch, name)(x, scalar, alpha=alpha)
    return getattr(torch, name)(x, scalar)


def binary_scalar_rounded(op: int, x: torch.Tensor, scalar: float, scalar_first: bool = False,
                          alpha: float = 1.0) -> torch.Tensor:
    """Tensor op Python number by the reference's rule: the 0-d CPU operand is
    converted to the tensor dtype first (ops.cpp:466-467), then the
    tensor-tensor op runs (ops.cpp:468-497).  That is binary() against a
    broadcast tensor holding the rounded scalar."""
    s = torch.full_like(x, scalar)
    return binary(op, s, x, alpha) if scalar_first else binary(op, x, s, alpha)


def sigmoid(x: torch.Tensor) -> torch.Tensor:
    """torch.sigmoid on CPU (fp32 opmath, one cast; backend.cpp:226-244 is the
    reference device counterpart, which rounds in fp16 four times)."""
    return torch.sigmoid(x)


def silu(x: torch.Tensor) -> torch.Tensor:
    """F.silu on CPU: x / (1 + exp(-x)) in fp32, one cast (elementwise.cpp:71-86)."""
    return F.silu(x)


def silu_add(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Fused C2f residual y + SiLU(x), single rounding: (silu(x32) + y32) -> x.dtype."""
    return (F.silu(x.float()) + y.float()).to(x.dtype)


def silu_add_unfused(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """The op-by-op chain the reference runs: silu_ then add (two roundings)."""
    return torch.add(y, F.silu(x))


def affine_silu(x: torch.Tensor, s: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Op-by-op half chain F.silu(torch.add(torch.mul(x, s), b)) -- what the
    reference's unfused ATen sequence computes (ops.cpp:464-497 twice, then
    silu_)."""
    return F.silu(torch.add(torch.mul(x, s), b))


def affine_silu_fp32(x: torch.Tensor, s: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Single-rounding variant, reported beside the primary oracle."""
    return F.silu(x.float() * s.float() + b.float()).to(x.dtype)
