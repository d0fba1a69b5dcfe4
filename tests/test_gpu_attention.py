"""GPU parity of the fused blocked attention (thin_attention, through the C
ABI): bit-equal to the op chain it replaces, channel_select -> mul ->
layout_bmm -> softmax -> layout_bmm (whole_blocked.py:91-103), run op by op
through the same library; that chain is pinned against the oracle here too
(exact contractions, softmax within 1e-3 relative)."""
import pytest
import torch

from oracle import bmm as ob
from oracle import elementwise as ew
from oracle import reductions as rd
from oracle.numerics import assert_rel, bits_equal
from tests.helpers import gen, normal16

pytestmark = pytest.mark.gpu


def same_bits(got, expect):
    """Bit-equal, except that a NaN only has to be a NaN (its payload follows
    the arithmetic unit's propagation rules)."""
    got, expect = got.cpu().contiguous(), expect.cpu().contiguous()
    assert got.shape == expect.shape and got.dtype == expect.dtype
    nan = expect.isnan()
    assert torch.equal(got.isnan(), nan)
    g, e = got.view(torch.int16), expect.view(torch.int16)
    return torch.equal(g[~nan], e[~nan])


def qkv_tensor(heads, key, dim, tokens, seed, device, std=1.0):
    channels = heads * (2 * key + dim)
    return (normal16((1, channels // 16, tokens, 16), seed) * std).to(device)


def chain(capi, qkv, heads, key, dim, scale, prescale):
    """The unfused chain through the C ABI; returns (scores, probabilities,
    mixed values)."""
    if prescale:
        query = capi.binary_scalar(capi.MUL, capi.channel_select(qkv, heads, 0, key), scale)
        scores = capi.layout_bmm(query, qkv, True, False, False, heads, 0, key, key, key)
    else:
        scores = capi.layout_bmm(qkv, qkv, True, False, False, heads, 0, key, key, key)
        scores = capi.binary_scalar(capi.MUL, scores, scale)
    probability = capi.softmax(scores, 2)
    mixed = capi.layout_bmm(qkv, probability, False, True, True, heads, 2 * key, dim)
    return scores, probability, mixed


def fp16_scale(key):
    """key ** -0.5 as the reference's 0-d operand rule rounds it (to fp16)."""
    return float(torch.tensor(key ** -0.5, dtype=torch.float64).half())


@pytest.mark.parametrize("prescale", [True, False])
@pytest.mark.parametrize("heads,key,dim,tokens", [
    (4, 32, 64, 400),    # C2PSA of YOLO26 / YOLO11-s at 640x640 (one wave per row)
    (2, 32, 64, 400),    # YOLO11-n
    (8, 32, 64, 400),    # 3200 score rows: two rows per wave in the softmax
    (4, 32, 64, 256),    # 16 lanes per row
    (4, 16, 32, 408),    # tokens not a multiple of 16 (scores rows padded to 416)
    (2, 64, 128, 200),   # two channel groups per lane
    (3, 32, 48, 144),    # head_dim below a wave, odd head count
])
def test_attention_matches_chain(gpu, heads, key, dim, tokens, prescale):
    from thintnpu_amd import capi
    qkv = qkv_tensor(heads, key, dim, tokens, 7000 + heads * 31 + tokens, gpu)
    scale = fp16_scale(key)
    got = capi.attention(qkv, heads, key, dim, scale, prescale)
    _, _, expect = chain(capi, qkv, heads, key, dim, scale, prescale)
    torch.cuda.synchronize()
    assert got.shape == (1, heads * dim // 16, tokens, 16)
    assert same_bits(got, expect), (heads, key, dim, tokens, prescale)


@pytest.mark.parametrize("prescale", [True, False])
def test_attention_chain_against_oracle(gpu, prescale):
    """The chain the fused kernel is held to, step by step against the oracle
    on the device's own input to each step, at the C2PSA shape; the fused
    result against a float32 attention as a sanity bound."""
    from thintnpu_amd import capi
    heads, key, dim, tokens = 4, 32, 64, 400
    qkv = qkv_tensor(heads, key, dim, tokens, 4242, gpu)
    scale = fp16_scale(key)
    scores, probability, mixed = chain(capi, qkv, heads, key, dim, scale, prescale)
    torch.cuda.synchronize()
    q_cpu = qkv.cpu()
    if prescale:
        query = ew.binary_scalar_rounded(1, ob.channel_select(q_cpu, heads, 0, key), key ** -0.5)
        expect_scores = ob.layout_bmm(query, q_cpu, True, False, False, heads, 0, key, key, key)
    else:
        raw = ob.layout_bmm(q_cpu, q_cpu, True, False, False, heads, 0, key, key, key)
        expect_scores = ew.binary_scalar_rounded(1, raw, key ** -0.5)
    assert bits_equal(scores.cpu(), expect_scores)
    assert_rel(probability.cpu(), rd.softmax(scores.cpu(), -1), 1e-3)
    assert bits_equal(mixed.cpu(), ob.layout_bmm(q_cpu, probability.cpu(), False, True, True, heads, 2 * key, dim))
    fused = capi.attention(qkv, heads, key, dim, scale, prescale).cpu()
    # float32 attention over the same fp16 inputs
    x = q_cpu.float().permute(0, 1, 3, 2).reshape(heads, 2 * key + dim, tokens)
    q, k, v = x[:, :key], x[:, key:2 * key], x[:, 2 * key:]
    p = torch.softmax(torch.bmm(q.transpose(1, 2).contiguous(), k) * scale, -1)
    o = torch.bmm(v, p.transpose(1, 2).contiguous())                       # [heads, dim, tokens]
    o_blocked = o.reshape(1, heads * dim // 16, 16, tokens).permute(0, 1, 3, 2)
    torch.testing.assert_close(fused.float(), o_blocked, rtol=0.02, atol=0.01)


def test_attention_fp32_scale(gpu):
    """An unrounded scale (PyTorch CPU's fp32 rule for mul) gives the chain's
    bits as well."""
    from thintnpu_amd import capi
    heads, key, dim, tokens = 4, 32, 64, 400
    qkv = qkv_tensor(heads, key, dim, tokens, 77, gpu)
    for prescale in (True, False):
        got = capi.attention(qkv, heads, key, dim, key ** -0.5, prescale)
        _, _, expect = chain(capi, qkv, heads, key, dim, key ** -0.5, prescale)
        torch.cuda.synchronize()
        assert same_bits(got, expect), prescale


def test_attention_nonfinite(gpu):
    """NaN and infinity in q and k: rows whose scores hold a NaN or +inf turn
    all NaN in both forms, exactly where the chain's do; overflowing scores
    (large operands) too."""
    from thintnpu_amd import capi
    heads, key, dim, tokens = 4, 32, 64, 400
    qkv = qkv_tensor(heads, key, dim, tokens, 5150, "cpu")
    flat = qkv.permute(0, 1, 3, 2).reshape(-1, tokens)                     # [channels, tokens] view
    group = 2 * key + dim
    flat[0 * group + 3, 17] = float("nan")                                   # q of head 0, row 17
    flat[1 * group + key + 5, 230] = float("inf")                            # k of head 1, column 230
    flat[2 * group + 2 * key + 9, 301] = float("-inf")                       # v of head 2
    qkv = flat.reshape(1, -1, 16, tokens).permute(0, 1, 3, 2).contiguous()
    for std in (1.0, 40.0):
        x = (qkv.float() * std).half().to(gpu)
        for prescale in (True, False):
            got = capi.attention(x, heads, key, dim, fp16_scale(key), prescale)
            _, _, expect = chain(capi, x, heads, key, dim, fp16_scale(key), prescale)
            torch.cuda.synchronize()
            assert expect.isnan().any()
            assert same_bits(got, expect), (std, prescale)


def test_attention_strided_blocks(gpu):
    """qkv as a channel-block slice of a larger tensor (block stride beyond
    T * 16) and out written into a strided view."""
    from thintnpu_amd import capi
    heads, key, dim, tokens = 2, 32, 64, 400
    big = normal16((1, 20, tokens, 16), 919).to(gpu)
    qkv = big[:, 2:18]
    out_big = torch.full((1, 12, tokens, 16), 7.0, dtype=torch.float16, device=gpu)
    out = out_big[:, 1:9]
    capi.attention(qkv, heads, key, dim, fp16_scale(key), True, out=out)
    _, _, expect = chain(capi, qkv.contiguous(), heads, key, dim, fp16_scale(key), True)
    torch.cuda.synchronize()
    assert same_bits(out, expect)
    assert bool((out_big[:, :1] == 7).all()) and bool((out_big[:, 9:] == 7).all())


@pytest.mark.parametrize("heads,key,dim,tokens", [
    (4, 32, 64, 100),    # tokens not a multiple of 8
    (4, 32, 64, 128),    # short rows (eight lanes per row in the softmax)
    (4, 32, 64, 1600),   # v beyond the kernel's LDS
    (4, 24, 64, 400),    # key_dim outside 16/32/64
])
def test_attention_unsupported_shapes(gpu, heads, key, dim, tokens):
    """Shapes outside the fused kernel's range are refused with
    THIN_ERR_UNSUPPORTED before any launch."""
    from thintnpu_amd import capi
    channels = heads * (2 * key + dim)
    qkv = torch.zeros((1, (channels + 15) // 16, tokens, 16), dtype=torch.float16, device=gpu)
    with pytest.raises(capi.ThinError) as info:
        capi.attention(qkv, heads, key, dim, 0.25, True)
    assert info.value.status == 2


def test_attention_invalid_arguments(gpu):
    from thintnpu_amd import capi
    qkv = torch.zeros((1, 32, 400, 16), dtype=torch.float16, device=gpu)
    with pytest.raises(capi.ThinError) as info:
        capi.attention(qkv, 3, 32, 64, 0.25, True)       # 512 channels do not split into 3 heads
    assert info.value.status == 1
    with pytest.raises(capi.ThinError):
        capi.attention(qkv, 4, 32, 64, 0.25, True,
                       out=torch.empty((1, 16, 399, 16), dtype=torch.float16, device=gpu))
