"""Pins the attention-contraction oracle (CPU only)."""
import itertools

import pytest
import torch

from oracle import bmm as ob
from oracle.numerics import bits_equal


def small_ints(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-3, 4, shape, generator=g).half()


def element(x, b, r, c, transpose, groups, origin):
    """Raw element of operand x at logical (b, r, c), indexed by hand."""
    if transpose:
        r, c = c, r
    if x.dim() == 3:
        return int(x[b, r + origin, c])
    if groups:
        ch = b * (x.shape[1] * 16 // groups) + r + origin
        return int(x[0, ch // 16, c, ch % 16])
    ch = r + origin
    return int(x[b, ch // 16, c, ch % 16])


def brute(a, b, batch, m, k, n, ta=False, tb=False, groups=0, ao=0, bo=0):
    out = torch.zeros(batch, m, n, dtype=torch.int64)
    for bt, i, j in itertools.product(range(batch), range(m), range(n)):
        out[bt, i, j] = sum(element(a, bt, i, kk, ta, groups if a.dim() == 4 else 0, ao) *
                            element(b, bt, kk, j, tb, groups if b.dim() == 4 else 0, bo) for kk in range(k))
    return out


@pytest.mark.parametrize("ta,tb", list(itertools.product((False, True), repeat=2)))
def test_rank3_exact_products(ta, tb):
    batch, m, k, n = 2, 5, 7, 3
    a = small_ints((batch, k, m) if ta else (batch, m, k), 1)
    b = small_ints((batch, n, k) if tb else (batch, k, n), 2)
    got = ob.layout_bmm(a, b, ta, tb)
    assert got.shape == (batch, m, n)
    assert torch.equal(got.long(), brute(a, b, batch, m, k, n, ta, tb))
    # a row range of the untransposed operand (origin applies before transposition)
    a2 = small_ints((batch, k + 3, m) if ta else (batch, m + 3, k), 3)
    got = ob.layout_bmm(a2, b, ta, tb, a_offset=2, a_channels=k if ta else m)
    assert torch.equal(got.long(), brute(a2, b, batch, m, k, n, ta, tb, ao=2))


def test_blocked_grouped_heads_and_packing():
    heads, key, dim, tokens = 2, 8, 16, 6
    x = small_ints((1, heads * (2 * key + dim) // 16, tokens, 16), 4)
    # q^T k per head: [tokens, key] x [key, tokens]
    got = ob.layout_bmm(x, x, True, False, False, heads, 0, key, key, key)
    assert torch.equal(got.long(), brute(x, x, heads, tokens, key, tokens, True, False, heads, 0, key))
    # v p^T per head with the blocked output [1, heads*dim/16, tokens, 16]
    p = small_ints((heads, tokens, tokens), 5)
    flat = brute(x, p, heads, dim, tokens, tokens, False, True, heads, 2 * key, 0)
    got = ob.layout_bmm(x, p, False, True, True, heads, 2 * key, dim)
    assert got.shape == (1, heads * dim // 16, tokens, 16)
    for bt, i, j in itertools.product(range(heads), range(dim), range(tokens)):
        r = bt * dim + i
        assert int(got[0, r // 16, j, r % 16]) == int(flat[bt, i, j])
    # heads whose channel count is not a multiple of 16 (only heads * m is)
    heads, key, dim, tokens = 8, 3, 6, 5
    x = small_ints((1, heads * (2 * key + dim) // 16, tokens, 16), 6)
    p = small_ints((heads, tokens, tokens), 7)
    flat = brute(x, p, heads, dim, tokens, tokens, False, True, heads, 2 * key, 0)
    got = ob.layout_bmm(x, p, False, True, True, heads, 2 * key, dim)
    for bt, i, j in itertools.product(range(heads), range(dim), range(tokens)):
        r = bt * dim + i
        assert int(got[0, r // 16, j, r % 16]) == int(flat[bt, i, j])


def test_blocked_ungrouped_batch_output():
    a = small_ints((2, 2, 5, 16), 8)   # 2 images, 32 channels, 5 tokens
    b = small_ints((2, 5, 3), 9)
    flat = brute(a, b, 2, 32, 5, 3)
    got = ob.layout_bmm(a, b, blocked_output=True)
    assert got.shape == (2, 2, 3, 16)
    for bt, i, j in itertools.product(range(2), range(32), range(3)):
        assert int(got[bt, i // 16, j, i % 16]) == int(flat[bt, i, j])


def test_sequential_order_and_fp32_accumulator():
    a = torch.tensor([[[4096., 1., 4096.]]]).half()
    b = torch.tensor([[[4096.], [1.], [-4096.]]]).half()
    # 2^24 + 1 rounds to 2^24 in fp32, so the sequential sum is 0 (exactly 1)
    assert ob.sequential_bmm(a, b).item() == 0.0
    a = torch.tensor([[[4096., 4096., 1.]]]).half()
    b = torch.tensor([[[4096.], [-4096.], [1.]]]).half()
    assert ob.sequential_bmm(a, b).item() == 1.0
    ones = torch.ones(1, 1, 4096).half()
    assert ob.sequential_bmm(ones, ones.transpose(1, 2)).item() == 4096.0
    # -0 products from a +0 start give +0
    z = ob.sequential_bmm(torch.tensor([[[-1.]]]).half(), torch.tensor([[[0.]]]).half())
    assert z.view(torch.int16).item() == 0


@pytest.mark.parametrize("shape", [(4, 400, 32, 400), (4, 64, 400, 400), (2, 17, 9, 23), (3, 5, 37, 1031),
                                   (1, 1, 1, 1)])
def test_random_within_reference_tolerance_of_torch(shape):
    batch, m, k, n = shape
    g = torch.Generator().manual_seed(2026)
    for transposed in (False, True):
        a = (torch.randn(batch, k, m, generator=g).transpose(1, 2) if transposed
             else torch.randn(batch, m, k, generator=g)).half()
        b = (torch.randn(batch, n, k, generator=g).transpose(1, 2) if transposed
             else torch.randn(batch, k, n, generator=g)).half()
        torch.testing.assert_close(ob.bmm(a, b), torch.bmm(a.float(), b.float()).half(), rtol=0.002, atol=0.002)


@pytest.mark.parametrize("heads,key,dim,tokens", [(4, 32, 64, 400), (4, 8, 16, 37), (2, 24, 48, 19),
                                                  (8, 3, 6, 19)])
def test_channel_select_matches_reference_construction(heads, key, dim, tokens):
    group = 2 * key + dim
    logical = torch.randn(heads, group, tokens, generator=torch.Generator().manual_seed(894)).half()
    source = logical.reshape(1, heads * group // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
    _, _, vr = logical.split((key, key, dim), 1)
    expect = vr.reshape(1, heads * dim // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
    assert bits_equal(ob.channel_select(source, heads, 2 * key, dim), expect)
    if heads * key % 16 == 0:
        qr = logical[:, :key]
        expect = qr.reshape(1, heads * key // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
        assert bits_equal(ob.channel_select(source, heads, 0, key), expect)
