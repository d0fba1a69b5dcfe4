"""GPU parity of the attention contractions (through the C ABI): layout_bmm /
bmm bit-equal to the sequential fp32 oracle (the reference's contract,
verify_bmm_layout.py:16-37), channel_select bit-exact."""
import itertools

import pytest
import torch

from oracle import bmm as ob
from oracle.numerics import bits_equal
from tests.helpers import gen

pytestmark = pytest.mark.gpu


def same_bits(got, expect):
    """Bit-equal, except that a NaN result only has to be a NaN (the payload a
    NaN operand leaves depends on the FMA unit's propagation rules)."""
    got, expect = got.cpu().contiguous(), expect.contiguous()
    assert got.shape == expect.shape and got.dtype == expect.dtype
    nan = expect.isnan()
    assert torch.equal(got.isnan(), nan)
    g, e = got.view(torch.int16), expect.view(torch.int16)
    return torch.equal(g[~nan], e[~nan])


@pytest.mark.parametrize("shape", [(4, 400, 32, 400), (4, 64, 400, 400), (2, 17, 9, 23), (3, 5, 37, 1031),
                                   (1, 1, 1, 1)])
def test_bmm_reference_shapes(gpu, shape):
    """verify_bmm_flow.py:15-25: plain and transposed-view operands."""
    from thintnpu_amd import capi
    batch, m, k, n = shape
    g = gen(2026)
    for transposed in (False, True):
        a = (torch.randn(batch, k, m, generator=g).transpose(1, 2) if transposed
             else torch.randn(batch, m, k, generator=g)).half()
        b = (torch.randn(batch, n, k, generator=g).transpose(1, 2) if transposed
             else torch.randn(batch, k, n, generator=g)).half()
        ad = a.contiguous().to(gpu) if not transposed else a.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
        bd = b.contiguous().to(gpu) if not transposed else b.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
        got = capi.bmm(ad, bd)
        assert got.shape == (batch, m, n) and got.stride(1) == (n + 15) // 16 * 16
        expect = ob.sequential_bmm(a, b)
        assert bits_equal(got, expect), (shape, transposed)
        torch.testing.assert_close(got.cpu(), torch.bmm(a.float(), b.float()).half(), rtol=0.002, atol=0.002)


@pytest.mark.parametrize("shape", [(2, 19, 33, 23), (1, 1, 600, 257), (3, 5, 37, 1031)])
@pytest.mark.parametrize("ta,tb", list(itertools.product((False, True), repeat=2)))
def test_bmm_strided_offset_views(gpu, shape, ta, tb):
    """verify_bmm_layout.py:42-57: operands are [.., 1:] views (odd storage
    offsets, non-unit row strides) in all four transpose combinations."""
    from thintnpu_amd import capi
    batch, m, k, n = shape
    g = gen(894)
    ac = torch.randn(batch, k, m + 1, generator=g).half() if ta else torch.randn(batch, m, k + 1, generator=g).half()
    bc = torch.randn(batch, n, k + 1, generator=g).half() if tb else torch.randn(batch, k, n + 1, generator=g).half()
    ad, bd = ac.to(gpu), bc.to(gpu)
    a = ad[:, :, 1:].transpose(1, 2) if ta else ad[:, :, 1:]
    b = bd[:, :, 1:].transpose(1, 2) if tb else bd[:, :, 1:]
    ar = ac[:, :, 1:].transpose(1, 2) if ta else ac[:, :, 1:]
    br = bc[:, :, 1:].transpose(1, 2) if tb else bc[:, :, 1:]
    assert bits_equal(capi.bmm(a, b), ob.sequential_bmm(ar, br))


@pytest.mark.parametrize("heads,key,dim,tokens", [(4, 32, 64, 400), (2, 16, 32, 160), (1, 16, 16, 1),
                                                  (3, 48, 80, 37)])
def test_layout_bmm_blocked_heads(gpu, heads, key, dim, tokens):
    """verify_bmm_layout.py:58-85: q^T k and v p^T over split blocked QKV, and
    the blocked output."""
    from thintnpu_amd import capi
    g = gen(894 + tokens)
    source = torch.randn(heads, (2 * key + dim) // 16, tokens, 16, generator=g).half()
    device = source.to(gpu)
    q, k, v = device.split((key // 16, key // 16, dim // 16), 1)
    qr, kr, vr = source.split((key // 16, key // 16, dim // 16), 1)
    got = capi.layout_bmm(q, k, True, False, False)
    assert bits_equal(got, ob.layout_bmm(qr, kr, True, False, False))
    probability = torch.randn(heads, tokens, tokens, generator=g).half()
    pd = probability.to(gpu)
    assert bits_equal(capi.layout_bmm(v, pd, False, True, False), ob.layout_bmm(vr, probability, False, True, False))
    got = capi.layout_bmm(v, pd, False, True, True)
    assert got.shape == (heads, dim // 16, tokens, 16)
    assert bits_equal(got, ob.layout_bmm(vr, probability, False, True, True))


@pytest.mark.parametrize("heads,key,dim,tokens", [(4, 32, 64, 400), (4, 8, 16, 37), (2, 24, 48, 19),
                                                  (8, 3, 6, 19)])
def test_layout_bmm_grouped_and_select(gpu, heads, key, dim, tokens):
    """verify_bmm_layout.py:86-106: head groups over one N=1 blocked QKV tensor,
    channel ranges per head, the grouped blocked output and channel_select."""
    from thintnpu_amd import capi
    group = 2 * key + dim
    logical = torch.randn(heads, group, tokens, generator=gen(heads * 100 + key)).half()
    source = logical.reshape(1, heads * group // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
    device = source.to(gpu)
    qr, kr, vr = logical.split((key, key, dim), 1)
    got = capi.layout_bmm(device, device, True, False, False, heads, 0, key, key, key)
    assert bits_equal(got, ob.sequential_bmm(qr.transpose(1, 2), kr))
    probability = torch.randn(heads, tokens, tokens, generator=gen(5)).half()
    pd = probability.to(gpu)
    expect = ob.sequential_bmm(vr, probability.transpose(1, 2))
    expect = expect.reshape(1, heads * dim // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
    got = capi.layout_bmm(device, pd, False, True, True, heads, 2 * key, dim)
    assert bits_equal(got, expect)
    expect = vr.reshape(1, heads * dim // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
    assert bits_equal(capi.channel_select(device, heads, 2 * key, dim), expect)


def test_summation_order_and_specials(gpu):
    from thintnpu_amd import capi
    # sequential fp32: 2^24 + 1 rounds back to 2^24, so the sum is 0 (exactly 1)
    a = torch.tensor([[[4096., 1., 4096.], [4096., 4096., 1.]]]).half()
    b = torch.tensor([[[4096., 4096.], [1., -4096.], [-4096., 1.]]]).half()
    got = capi.bmm(a.to(gpu), b.to(gpu)).cpu()
    assert bits_equal(got, ob.sequential_bmm(a, b))
    assert got[0, 0, 0].item() == 0.0 and got[0, 1, 1].item() == 1.0
    # fp32 accumulator over a long reduction (an fp16 one stalls at 2048)
    ones = torch.ones(2, 3, 4096).half()
    got = capi.bmm(ones.to(gpu), ones.transpose(1, 2).contiguous().to(gpu)).cpu()
    assert got.eq(4096).all()
    # infinities, NaNs, signed zeros, subnormals and overflow to inf
    vals = torch.tensor([0., -0., float("inf"), -float("inf"), float("nan"), 2 ** -24, -2 ** -24, 65504., -65504.,
                         1., -1., 0.5, 300.]).half()
    g = gen(3)
    a = vals[torch.randint(0, len(vals), (3, 21, 13), generator=g)]
    b = vals[torch.randint(0, len(vals), (3, 13, 70), generator=g)]
    assert same_bits(capi.bmm(a.to(gpu), b.to(gpu)), ob.sequential_bmm(a, b))
    # tiny products: subnormal fp16 results and -0 from negative underflow
    a = torch.full((1, 2, 3), 2 ** -12).half()
    b = torch.tensor([[[2 ** -8, -2 ** -14], [0., 0.], [2 ** -9, -2 ** -20]]]).half()
    got = capi.bmm(a.to(gpu), b.to(gpu))
    assert bits_equal(got, ob.sequential_bmm(a, b))
    assert got[0, 0, 0].item() == 1.5 * 2 ** -20 and got.cpu().view(torch.int16)[0, 0, 1].item() == -32768


@pytest.mark.parametrize("shape", [(1, 63, 17, 65), (1, 64, 31, 64), (5, 129, 33, 127), (300, 3, 5, 7),
                                   (1, 1000, 3, 1), (2, 16, 2048, 16)])
def test_bmm_tile_edges(gpu, shape):
    """Row / column counts around the 64-column tile, a batch of many small
    products, one column, and a reduction over many staging rounds."""
    from thintnpu_amd import capi
    batch, m, k, n = shape
    g = gen(sum(shape))
    a = torch.randn(batch, m, k, generator=g).half()
    b = torch.randn(batch, k, n, generator=g).half()
    assert bits_equal(capi.bmm(a.to(gpu), b.to(gpu)), ob.sequential_bmm(a, b))
    out = torch.full((batch, m, n + 3), 7.0, dtype=torch.float16, device=gpu)
    capi.bmm(a.to(gpu), b.to(gpu), out=out[:, :, 2:2 + n])
    assert bits_equal(out[:, :, 2:2 + n], ob.sequential_bmm(a, b))
    assert out[:, :, :2].cpu().eq(7).all() and out[:, :, 2 + n:].cpu().eq(7).all()


def test_blocked_ungrouped_batch(gpu):
    from thintnpu_amd import capi
    a = torch.randn(3, 2, 9, 16, generator=gen(9)).half()   # 3 images, 32 channels, 9 tokens
    b = torch.randn(3, 9, 40, generator=gen(10)).half()
    got = capi.layout_bmm(a.to(gpu), b.to(gpu), blocked_output=True)
    assert got.shape == (3, 2, 40, 16)
    assert bits_equal(got, ob.layout_bmm(a, b, blocked_output=True))
    # a channel range of a rank-4 operand read transposed (tokens x channels)
    got = capi.layout_bmm(a.to(gpu), a[:, :, :, :].to(gpu), True, False, False, 0, 5, 11, 3, 11)
    assert bits_equal(got, ob.layout_bmm(a, a, True, False, False, 0, 5, 11, 3, 11))


def test_channel_select_views(gpu):
    from thintnpu_amd import capi
    x = torch.randint(-32768, 32768, (1, 6, 23, 16), dtype=torch.int16, generator=gen(4)).view(torch.float16)
    for groups, begin, count in ((3, 0, 16), (3, 5, 16), (2, 7, 8), (6, 1, 8), (1, 0, 96), (4, 10, 4)):
        assert bits_equal(capi.channel_select(x.to(gpu), groups, begin, count),
                          ob.channel_select(x, groups, begin, count))
    # a token-strided view of a larger tensor
    big = torch.randint(-32768, 32768, (1, 6, 50, 16), dtype=torch.int16, generator=gen(5)).view(torch.float16)
    view = big.to(gpu)[:, :, 3::2]
    assert bits_equal(capi.channel_select(view, 2, 7, 8), ob.channel_select(big[:, :, 3::2], 2, 7, 8))


def test_bmm_errors(gpu):
    from thintnpu_amd import capi
    h = lambda *s: torch.zeros(s, dtype=torch.float16, device=gpu)
    cases = [
        (lambda: capi.bmm(h(2, 3, 4), h(2, 5, 6)), "do not match or are empty"),
        (lambda: capi.bmm(h(2, 3, 4), h(3, 4, 6)), "do not match or are empty"),
        (lambda: capi.bmm(h(2, 3, 4), h(2, 4, 0)), "do not match or are empty"),
        (lambda: capi.bmm(h(2, 0, 4), h(2, 4, 6)), "exceeds its group"),  # zero rows: the channel check first
        (lambda: capi.bmm(h(2, 3, 4).float(), h(2, 4, 6)), "FP16 rank-3 or channel-blocked"),
        (lambda: capi.bmm(h(3, 4), h(4, 6)), "FP16 rank-3 or channel-blocked"),
        (lambda: capi.layout_bmm(h(1, 2, 5, 16), h(1, 2, 5, 16), True, False, False, 3), "divisible channels"),
        (lambda: capi.layout_bmm(h(2, 2, 5, 16), h(2, 2, 5, 16), True, False, False, 2), "requires N=1"),
        (lambda: capi.layout_bmm(h(1, 2, 5, 16), h(1, 2, 5, 16), True, False, False, 2, 10, 8, 0, 8),
         "exceeds its group"),
        (lambda: capi.layout_bmm(h(1, 2, 5, 16), h(1, 2, 5, 16), True, False, False, 0, -1), "invalid channel grouping"),
        (lambda: capi.layout_bmm(h(2, 5, 3), h(2, 3, 4), blocked_output=True), "C0-aligned channels"),
        (lambda: capi.channel_select(h(2, 2, 5, 16), 2, 0, 8), "N=1 FP16 blocked"),
        (lambda: capi.channel_select(h(1, 2, 5, 16), 3, 0, 8), "valid equal groups"),
        (lambda: capi.channel_select(h(1, 2, 5, 16), 2, 10, 8), "valid equal groups"),
        (lambda: capi.channel_select(h(1, 2, 5, 16), 2, 0, 4), "C0-aligned total output"),
    ]
    for fn, text in cases:
        with pytest.raises(capi.ThinError, match=text):
            fn()
    with pytest.raises(capi.ThinError, match="out must be"):
        capi.bmm(h(2, 3, 4), h(2, 4, 6), out=h(2, 3, 5))


@pytest.mark.parametrize("key", [80, 128, 528])
def test_streamed_long_reductions(gpu, key):
    """q^T k with K = key channels: the streamed-column kernel's 64-step
    staging rounds (K > 64), several vector rounds, a partial last round, and
    (K = 528) two rounds of staged rows."""
    from thintnpu_amd import capi
    heads, tokens = 2, 70
    source = torch.randn(heads, 2 * key // 16, tokens, 16, generator=gen(key)).half()
    q, k = source.to(gpu).split((key // 16, key // 16), 1)
    qr, kr = source.split((key // 16, key // 16), 1)
    assert bits_equal(capi.layout_bmm(q, k, True, False, False), ob.layout_bmm(qr, kr, True, False, False))


@pytest.mark.parametrize("k", [21, 77])
def test_streamed_reduction_tail(gpu, k):
    """Columns contiguous along k at a 24-element stride with K % 8 != 0: the
    streamed kernel's whole vectors plus its scalar tail."""
    from thintnpu_amd import capi
    batch, m, n = 2, 9, 70
    pitch = (k + 7) // 8 * 8 + 8
    a = torch.randn(batch, m, k, generator=gen(k)).half()
    store = torch.randn(batch, n, pitch, generator=gen(k + 1)).half()
    b = store[:, :, :k].transpose(1, 2)          # [batch, k, n], column stride `pitch`
    bd = store.to(gpu)[:, :, :k].transpose(1, 2)
    assert bits_equal(capi.bmm(a.to(gpu), bd), ob.sequential_bmm(a, b))
