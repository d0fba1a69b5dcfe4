"""Pins the data-movement oracle (CPU only)."""
import itertools

import numpy as np
import pytest

import torch
import torch.nn.functional as F

from oracle import movement as mv
from oracle.numerics import bits_equal
from tests.helpers import random_bits16, to_blocked


def test_cat_matches_torch_cat_bits():
    for dim in range(4):
        parts = []
        for i, size in enumerate((1, 2, 5)):
            shape = [3, 3, 4, 4]
            shape[dim] = size
            parts.append(random_bits16(tuple(shape), 10 + i))
        # torch.cat on int16 views is the library reference for bit movement
        expect = torch.cat([p.view(torch.int16) for p in parts], dim).view(torch.float16)
        assert bits_equal(mv.cat(parts, dim), expect)
    e = torch.empty(0, dtype=torch.float16)
    x = random_bits16((3, 4), 3)
    assert bits_equal(mv.cat([e, x, e], 1), x)
    assert mv.cat([e, e], 0).shape == (0,)


def test_upsample_matches_interpolate_and_loops():
    x = torch.randn(2, 3, 5, 7).half()
    ref = F.interpolate(x.float(), scale_factor=2, mode="nearest").half()
    assert bits_equal(mv.upsample2x_nchw(x), ref)
    xb = random_bits16((2, 3, 4, 5, 16), 4)
    y = mv.upsample2x_blocked(xb)
    assert y.shape == (2, 3, 8, 10, 16)
    yi, xi = y.view(torch.int16), xb.view(torch.int16)
    for n, c, h, w in itertools.product(range(2), range(3), range(8), range(10)):
        assert torch.equal(yi[n, c, h, w], xi[n, c, h // 2, w // 2])
    # a transposed-axis mistake would break the non-square case above; nearest
    # of the NCHW view of blocked data agrees too
    nchw = xb.view(torch.int16).permute(0, 1, 4, 2, 3).reshape(2, 48, 4, 5).float()
    ref = F.interpolate(nchw, scale_factor=2, mode="nearest")
    got = y.view(torch.int16).permute(0, 1, 4, 2, 3).reshape(2, 48, 8, 10).float()
    assert torch.equal(got, ref)


def test_pack_unpack_brute_force():
    for c in (3, 16, 17, 40):
        x = random_bits16((2, c, 3, 5), c)
        y = mv.pack_blocked(x)
        c1 = (c + 15) // 16
        assert y.shape == (2, c1, 3, 5, 16)
        yi, xi = y.view(torch.int16), x.view(torch.int16)
        for n, cb, h, w, k in itertools.product(range(2), range(c1), range(3), range(5), range(16)):
            ch = cb * 16 + k
            assert yi[n, cb, h, w, k] == (xi[n, ch, h, w] if ch < c else 0)
        assert bits_equal(mv.unpack_blocked(y, c), x)


def test_upsample_cat_composition():
    a = random_bits16((2, 2, 3, 4, 16), 5)
    b = random_bits16((2, 1, 6, 8, 16), 6)
    got = mv.upsample_cat_blocked([a, b], [True, False])
    assert got.shape == (2, 3, 6, 8, 16)
    assert bits_equal(got[:, :2], mv.upsample2x_blocked(a))
    assert bits_equal(got[:, 2:], b)


def brute_maxpool(x: np.ndarray, k: int) -> np.ndarray:
    """Window max by hand: first strictly greater value in row-major window
    order, NaN if the window holds a NaN."""
    n, c, h, w = x.shape
    r = k // 2
    out = np.empty_like(x)
    for i in np.ndindex(n, c, h, w):
        b, ch, yy, xx = i
        best, nan = None, False
        for dy in range(-r, r + 1):
            for dx in range(-r, r + 1):
                sy, sx = yy + dy, xx + dx
                if 0 <= sy < h and 0 <= sx < w:
                    v = x[b, ch, sy, sx]
                    if np.isnan(v):
                        nan = True
                    elif best is None or v > best:
                        best = v
        out[i] = np.float16("nan") if nan else best
    return out


@pytest.mark.parametrize("k", [1, 3, 5, 7])
def test_maxpool_against_brute_force(k):
    g = torch.Generator().manual_seed(k)
    x = torch.randn(2, 3, 6, 7, generator=g).half()
    # ties between +0 and -0 in both orders, infinities, a NaN
    x[0, 0, 2, 2], x[0, 0, 2, 3] = -0.0, 0.0
    x[0, 0, 0:6, 0:7] = torch.where(x[0, 0] > 0, -x[0, 0], x[0, 0])  # plane 0 all <= 0
    x[0, 0, 3, 1], x[0, 0, 1, 4] = 0.0, -0.0
    x[0, 1, 1, 1] = float("inf")
    x[1, 2, 4, 4] = float("-inf")
    x[1, 1, 2, 5] = float("nan")
    got = mv.maxpool_nchw(x, k)
    want = torch.from_numpy(brute_maxpool(x.numpy(), k))
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan)
    assert bits_equal(got[~nan], want[~nan])
    blocked = to_blocked(torch.cat((x, x.flip(1), x, x.flip(2), x, x), 1)[:, :16])
    assert bits_equal(mv.maxpool_blocked(blocked, k),
                      to_blocked(mv.maxpool_nchw(torch.cat((x, x.flip(1), x, x.flip(2), x, x), 1)[:, :16], k)))


def test_sppf_chain_identities():
    """sppf_blocked: slot 0 is x; with no +0/-0 ties the r-th chained k-pool is
    one (r*(k-1)+1)-wide pool (max over a window of windows, -inf padding never
    wins), which a slot pooling x instead of its predecessor would fail; a NaN
    spreads by k//2 pixels per repeat."""
    g = torch.Generator().manual_seed(5)
    x = to_blocked(torch.randn(2, 32, 9, 11, generator=g).half())
    for k in (3, 5):
        y = mv.sppf_blocked(x, k, 3)
        assert y.shape == (2, 8, 9, 11, 16)
        assert bits_equal(y[:, :2], x)
        for r in (1, 2, 3):
            assert bits_equal(y[:, 2 * r:2 * r + 2], mv.maxpool_blocked(x, r * (k - 1) + 1)), (k, r)
    z = x.clone()
    z[0, 0, 4, 5, 3] = float("nan")
    y = mv.sppf_blocked(z, 5, 2)
    rows, cols = torch.nonzero(torch.isnan(y[0, 4, :, :, 3]), as_tuple=True)
    assert (rows.min(), rows.max(), cols.min(), cols.max()) == (0, 8, 1, 9)
