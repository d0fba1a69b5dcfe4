"""Numerical contracts shared by all tests (test infrastructure only).

* ``ulp_distance``: fp16 bits -> ordered integer o(b) = b if sign = 0 else
  -(b & 0x7fff), so +0 and -0 coincide; ulp = |o(a) - o(r)|.  NaN must meet
  NaN (payload free), infinities must match exactly.
* ``rel_error``: |a - r| / max(|r|, 2^-14); the floor is fp16's smallest
  normal, so subnormal outputs are judged absolutely.

Pinned by tests/test_oracle_numerics.py against hand-computed fp16 encodings.
"""
from __future__ import annotations

import numpy as np
import torch

FP16_MIN_NORMAL = 2.0 ** -14


def bits16(t: torch.Tensor) -> np.ndarray:
    """Raw fp16 bits as int64 (CPU)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().astype(np.int64) & 0xFFFF


def ordered16(b: np.ndarray) -> np.ndarray:
    b = b.astype(np.int64)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def ulp_report(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    """Compare two fp16 tensors; returns max ulp over finite pairs, NaN/inf agreement
    and the count of exactly equal encodings (+0/-0 counted equal)."""
    assert actual.dtype == torch.float16 and expected.dtype == torch.float16
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    a = bits16(actual).reshape(-1)
    r = bits16(expected).reshape(-1)
    a_nan = ((a & 0x7C00) == 0x7C00) & ((a & 0x3FF) != 0)
    r_nan = ((r & 0x7C00) == 0x7C00) & ((r & 0x3FF) != 0)
    a_inf = (a & 0x7FFF) == 0x7C00
    r_inf = (r & 0x7FFF) == 0x7C00
    nan_ok = bool(np.array_equal(a_nan, r_nan))
    inf_ok = bool(np.array_equal(a_inf & ~r_nan, r_inf & ~a_nan) and
                  np.array_equal(a[a_inf & r_inf], r[a_inf & r_inf]))
    finite = ~(a_nan | r_nan | a_inf | r_inf)
    d = np.abs(ordered16(a[finite]) - ordered16(r[finite]))
    return dict(max_ulp=int(d.max()) if d.size else 0, nan_match=nan_ok, inf_match=inf_ok,
                exact=int((d == 0).sum()), finite=int(finite.sum()), count=int(a.size))


def assert_ulp(actual: torch.Tensor, expected: torch.Tensor, max_ulp: int, what: str = "") -> dict:
    rep = ulp_report(actual, expected)
    assert rep["nan_match"], f"{what}: NaN positions differ"
    assert rep["inf_match"], f"{what}: infinities differ"
    assert rep["max_ulp"] <= max_ulp, f"{what}: {rep['max_ulp']} ulp > {max_ulp} ({rep})"
    return rep


def rel_error(actual: torch.Tensor, expected: torch.Tensor) -> tuple[float, float]:
    """(max floored relative error, max abs error) over positions finite in expected."""
    a = actual.detach().cpu().double()
    r = expected.detach().cpu().double()
    m = torch.isfinite(r)
    if not bool(m.any()):
        return 0.0, 0.0
    diff = (a[m] - r[m]).abs()
    rel = diff / r[m].abs().clamp_min(FP16_MIN_NORMAL)
    return float(rel.max()), float(diff.max())


def assert_rel(actual: torch.Tensor, expected: torch.Tensor, tol: float, what: str = "") -> float:
    a = actual.detach().cpu()
    r = expected.detach().cpu()
    assert torch.equal(torch.isnan(a), torch.isnan(r)), f"{what}: NaN mask differs"
    assert torch.equal(torch.isposinf(a), torch.isposinf(r)), f"{what}: +inf mask differs"
    assert torch.equal(torch.isneginf(a), torch.isneginf(r)), f"{what}: -inf mask differs"
    rel, _ = rel_error(a, r)
    assert rel <= tol, f"{what}: relative error {rel} > {tol}"
    return rel


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    a = a.detach().cpu().contiguous()
    b = b.detach().cpu().contiguous()
    return (a.dtype == b.dtype and a.shape == b.shape and
            torch.equal(a.reshape(-1).view(torch.uint8), b.reshape(-1).view(torch.uint8)))


def ulp16_spacing(r: torch.Tensor) -> torch.Tensor:
    """Spacing of fp16 numbers at |r| (2^-24 in the subnormal range), float64."""
    a = r.detach().cpu().double().abs()
    e = torch.floor(torch.log2(a.clamp_min(2.0 ** -24)))
    return torch.pow(2.0, (e - 10).clamp_min(-24))


def ulp32_spacing(r: torch.Tensor) -> torch.Tensor:
    a = r.detach().cpu().double().abs()
    e = torch.floor(torch.log2(a.clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 23)


def assert_fused_cancel(actual: torch.Tensor, expected: torch.Tensor, term: torch.Tensor,
                        max_ulp: int = 2, term_ulp32: int = 4, what: str = "") -> dict:
    """Bound for a fused r = y + f(x) evaluated in fp32 and rounded once:
    |a - r| <= max_ulp fp16 ulps of r  OR  <= term_ulp32 fp32 ulps of |f(x)|.
    The second arm covers cancellation (y ~ -f(x)), where two correct fp32
    evaluations of f that differ by one fp32 ulp land many fp16 ulps apart
    in the small result."""
    rep = ulp_report(actual, expected)
    assert rep["nan_match"] and rep["inf_match"], f"{what}: non-finite mismatch"
    a = actual.detach().cpu().double()
    r = expected.detach().cpu().double()
    m = torch.isfinite(r)
    err = (a - r).abs()[m]
    ulp_arm = err <= max_ulp * ulp16_spacing(r)[m]
    ok = ulp_arm | (err <= term_ulp32 * ulp32_spacing(term)[m])
    assert bool(ok.all()), f"{what}: {int((~ok).sum())} elements outside the fused bound ({rep})"
    # elements that pass only through the cancellation arm, and how far they are
    only = (~ulp_arm).numpy()
    rep["cancel_only"] = int(only.sum())
    if rep["cancel_only"]:
        fa = ordered16(bits16(actual).reshape(-1)[m.reshape(-1).numpy()])
        fr = ordered16(bits16(expected).reshape(-1)[m.reshape(-1).numpy()])
        rep["cancel_max_ulp"] = int(np.abs(fa - fr)[only].max())
    else:
        rep["cancel_max_ulp"] = 0
    return rep
