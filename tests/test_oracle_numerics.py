"""Known answers for the numerical-contract helpers every parity test uses
(oracle/numerics.py): the fp16 ulp distance, the floored relative error, the
fp16/fp32 spacings and both arms of the fused-cancellation bound.  Each case
is a hand-computed encoding or value, so a wrong sign, floor or exponent in a
helper fails here."""
import math

import pytest
import torch

from oracle.numerics import (FP16_MIN_NORMAL, assert_fused_cancel, assert_rel, assert_ulp, bits_equal,
                             rel_error, ulp16_spacing, ulp32_spacing, ulp_report)


def h(*bits):
    return torch.tensor(bits, dtype=torch.int16).view(torch.float16)


def test_ulp_distance_known_encodings():
    # 1.0 = 0x3C00, next up 0x3C01, next down 0x3BFF: one ulp either side
    assert ulp_report(h(0x3C01), h(0x3C00))["max_ulp"] == 1
    assert ulp_report(h(0x3BFF), h(0x3C00))["max_ulp"] == 1
    # +0 and -0 coincide; the smallest subnormals either side of zero are 2 apart
    assert ulp_report(h(0x0000), h(0x8000 - 65536))["max_ulp"] == 0
    assert ulp_report(h(0x0001), h(0x8001 - 65536))["max_ulp"] == 2
    # across the sign: -1.0 (0xBC00) to +1.0 is 2 * 0x3C00 ulps
    assert ulp_report(h(0xBC00 - 65536), h(0x3C00))["max_ulp"] == 2 * 0x3C00
    # max finite to +inf are not compared as finite; inf must match exactly
    rep = ulp_report(h(0x7C00), h(0x7BFF))
    assert not rep["inf_match"]
    assert ulp_report(h(0x7C00), h(0x7C00))["inf_match"]
    # NaN meets NaN whatever the payload, never a number
    assert ulp_report(h(0x7E00), h(0x7C01))["nan_match"]
    assert not ulp_report(h(0x7E00), h(0x3C00))["nan_match"]


def test_assert_ulp_bar():
    assert_ulp(h(0x3C02), h(0x3C00), 2)
    with pytest.raises(AssertionError):
        assert_ulp(h(0x3C03), h(0x3C00), 2)


def test_rel_error_floor_at_fp16_min_normal():
    assert FP16_MIN_NORMAL == 2.0 ** -14
    # above the floor: relative to |r|
    d = torch.float64
    rel, ab = rel_error(torch.tensor([1.001], dtype=d), torch.tensor([1.0], dtype=d))
    assert rel == pytest.approx(1e-3, rel=1e-6) and ab == pytest.approx(1e-3, rel=1e-6)
    # below the floor: relative to 2^-14, so a subnormal result is judged absolutely
    r = torch.tensor([2.0 ** -24], dtype=d)
    rel, _ = rel_error(torch.tensor([2.0 ** -24 + 2.0 ** -20], dtype=d), r)
    assert rel == pytest.approx(2.0 ** -20 / 2.0 ** -14)
    # sign of the error does not matter; non-finite references are skipped
    rel, _ = rel_error(torch.tensor([0.999, 5.0], dtype=d), torch.tensor([1.0, float("inf")], dtype=d))
    assert rel == pytest.approx(1e-3, rel=1e-6)
    assert rel_error(torch.tensor([1.0]), torch.tensor([float("nan")])) == (0.0, 0.0)


def test_assert_rel_masks_and_bar():
    assert_rel(torch.tensor([1.0009, float("nan")]), torch.tensor([1.0, float("nan")]), 1e-3)
    with pytest.raises(AssertionError, match="relative"):
        assert_rel(torch.tensor([1.0011]), torch.tensor([1.0]), 1e-3)
    with pytest.raises(AssertionError, match="NaN mask"):
        assert_rel(torch.tensor([1.0]), torch.tensor([float("nan")]), 1e-3)


def test_spacings():
    # fp16: 2^(e-10) for normals, 2^-24 for subnormals
    r = torch.tensor([1.0, 1.5, 2.0, 1000.0, 2.0 ** -14, 2.0 ** -20, 0.0])
    expect = [2.0 ** -10, 2.0 ** -10, 2.0 ** -9, 0.5, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24]
    assert ulp16_spacing(r).tolist() == expect
    # the spacing is the gap to the next fp16 number for normals
    for v in (1.0, 3.0, 1000.0):
        nxt = torch.tensor([v], dtype=torch.float16).view(torch.int16) + 1
        assert nxt.view(torch.float16).double().item() - v == ulp16_spacing(torch.tensor([v])).item()
    # fp32: 2^(e-23)
    assert ulp32_spacing(torch.tensor([1.0, 3.0])).tolist() == [2.0 ** -23, 2.0 ** -22]
    assert math.isclose(ulp32_spacing(torch.tensor([1e-40])).item(), 2.0 ** -149)


def test_fused_cancel_both_arms():
    # arm 1: within max_ulp fp16 ulps of r
    r = torch.tensor([1.0], dtype=torch.float16)
    assert_fused_cancel(h(0x3C02), r, torch.tensor([1.0]), max_ulp=2)
    with pytest.raises(AssertionError):
        assert_fused_cancel(h(0x3C03), r, torch.tensor([1.0]), max_ulp=2, term_ulp32=0)
    # arm 2: cancellation.  r = y + f with |f| = 3 and y = -3 + tiny: a result
    # 1 fp16 ulp-of-tiny * 10 away is accepted when within 4 fp32 ulps of |f|
    tiny = torch.tensor([2.0 ** -14], dtype=torch.float16)
    off = torch.tensor([2.0 ** -14 + 2.0 ** -20], dtype=torch.float16)      # many fp16 ulps of r away
    assert (off.double() - tiny.double()).abs().item() <= 4 * 2.0 ** -22   # <= 4 fp32 ulps of 3.0
    assert_fused_cancel(off, tiny, torch.tensor([3.0]), max_ulp=2, term_ulp32=4)
    with pytest.raises(AssertionError):
        assert_fused_cancel(off, tiny, torch.tensor([3.0]), max_ulp=2, term_ulp32=0)


def test_bits_equal_is_bytewise():
    assert bits_equal(h(0x7E01), h(0x7E01))
    assert not bits_equal(h(0x7E01), h(0x7E02))   # NaN payloads count
    assert not bits_equal(h(0x0000), h(0x8000 - 65536))  # so do zero signs
    assert not bits_equal(torch.zeros(2), torch.zeros(2, dtype=torch.float64))
