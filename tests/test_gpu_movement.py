"""GPU parity of the data-movement entry points (through the C ABI): all
bit-exact against the CPU oracle, NaN payloads included."""
import pytest
import torch

from oracle import movement as mv
from oracle.numerics import bits_equal
from tests.helpers import gen, normal16, random_bits16, to_blocked

pytestmark = pytest.mark.gpu


def rand_dtype(shape, dtype, seed):
    g = gen(seed)
    if dtype == torch.float16:
        return torch.randint(-32768, 32768, shape, dtype=torch.int16, generator=g).view(torch.float16)
    return torch.randint(-2 ** 31, 2 ** 31 - 1, shape, dtype=torch.int32, generator=g).view(torch.float32)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_cat_reference_cases(gpu, dtype):
    """verify_cat.py:20-54 restated."""
    from thintnpu_amd import capi
    seed = 0
    for dim in range(4):
        for outer in (1, 3):
            shape = [outer, 3, 32, 32]
            parts = []
            for size in (1, 2, 5):
                cur = shape.copy()
                cur[dim] = size if dim != 3 else size * 32
                seed += 1
                parts.append(rand_dtype(tuple(cur), dtype, seed))
            got = capi.cat([p.to(gpu) for p in parts], dim).cpu()
            assert bits_equal(got, mv.cat(parts, dim)), (dim, outer)
    for length in (16, 8192, 16384, 16384 + 16, 131072 + 16):
        parts = [rand_dtype((3, length), dtype, 100 + i) for i in range(3)]
        assert bits_equal(capi.cat([p.to(gpu) for p in parts], 1).cpu(), mv.cat(parts, 1))
    for offset in (1, 16):
        src = rand_dtype((3 * 64 * 64 + offset,), dtype, 7)
        dev = src.to(gpu)
        cv, dv = src[offset:].view(3, 64, 64), dev[offset:].view(3, 64, 64)
        assert bits_equal(capi.cat([dv, dv], 1).cpu(), mv.cat([cv, cv], 1))
        assert bits_equal(capi.cat([dv.transpose(0, 2)] * 2, 1).cpu(), mv.cat([cv.transpose(0, 2)] * 2, 1))
    src = rand_dtype((3, 64, 32), dtype, 8)
    dev = src.to(gpu)
    assert bits_equal(capi.cat(list(dev.split(32, 1)), 1).cpu(), src)
    assert bits_equal(capi.cat([dev[:1].expand(3, -1, -1)] * 2, 1).cpu(), mv.cat([src[:1].expand(3, -1, -1)] * 2, 1))
    shaped_empty = torch.empty(3, 0, 32, dtype=dtype)
    assert bits_equal(capi.cat([shaped_empty.to(gpu), dev], 1).cpu(), src)
    assert bits_equal(capi.cat([dev], 1).cpu(), src)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_cat_plan_cases(gpu, dtype):
    """verify_cat_plan.py:15-52: 1..17 NC1HWC0 inputs, split -> cat round trips."""
    from thintnpu_amd import capi
    for count in (1, 2, 3, 4, 6, 8, 9, 17):
        for batch in (1, 3):
            for plane in (20, 80):
                parts = [rand_dtype((batch, 1 + i % 3, plane, plane, 16), dtype, 1000 + i) for i in range(count)]
                got = capi.cat([p.to(gpu) for p in parts], 1).cpu()
                assert bits_equal(got, mv.cat(parts, 1)), (count, batch, plane)
    for rows in (8, 81, 129):
        parts = [rand_dtype((1, rows, length), dtype, rows + length) for length in (6400, 1600, 400)]
        assert bits_equal(capi.cat([p.to(gpu) for p in parts], 2).cpu(), mv.cat(parts, 2))
    for batch in (1, 3):
        x = rand_dtype((batch, 12, 40, 40, 16), dtype, 5)
        xd = x.to(gpu)
        for sizes in ((3, 3, 6), (1, 2, 3, 6)):
            assert bits_equal(capi.cat(list(xd.split(sizes, 1)), 1).cpu(), x)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_strided_concat_cases(gpu, dtype):
    """verify_materialize.py:44-74 strided/broadcast/offset concat cases."""
    from thintnpu_amd import capi
    for rows in (1, 7, 127, 128, 129, 6400):
        for widths in ((2, 2, 12), (1, 7, 24), (3, 5, 8), (6, 10)):
            parts = [rand_dtype((rows, w), dtype, rows * 31 + w) for w in widths]
            assert bits_equal(capi.cat([p.to(gpu) for p in parts], 1).cpu(), mv.cat(parts, 1))
    for mode, tr in (("sliced", lambda t: t[::3]), ("broadcast", lambda t: t[:1].expand(273, -1)),
                     ("offset", lambda t: t[:, 1:])):
        widths = (2, 2, 12)
        src = [rand_dtype((273, w + (mode == "offset")), dtype, 77 + w) for w in widths]
        dev = [tr(s.to(gpu)) for s in src]
        assert bits_equal(capi.cat(dev, 1).cpu(), mv.cat([tr(s) for s in src], 1)), mode


def test_cat_c3_c2f(gpu):
    """C3: C2f concat of 2+n=4 chunks [N,64,80,80] in NC1HWC0 (two are the halves
    of one [N,128,80,80] tensor), N in {1,32}."""
    from thintnpu_amd import capi
    for n in (1, 32):
        parent = to_blocked(normal16((n, 128, 80, 80), 3))
        m1 = to_blocked(normal16((n, 64, 80, 80), 4))
        m2 = to_blocked(normal16((n, 64, 80, 80), 5))
        pd = parent.to(gpu)
        a, b = pd.chunk(2, 1)
        got = capi.cat([a, b, m1.to(gpu), m2.to(gpu)], 1).cpu()
        ca, cb = parent.chunk(2, 1)
        assert bits_equal(got, mv.cat([ca, cb, m1, m2], 1)), n


@pytest.mark.parametrize("n", [1, 32])
def test_upsample_and_fused_cat_c3(gpu, n):
    """C3: nearest 2x [N,256,40,40] -> [N,256,80,80], then cat with [N,128,80,80];
    the fused op must equal the two-step composition bit for bit."""
    from thintnpu_amd import capi
    x = to_blocked(normal16((n, 256, 40, 40), 6))
    o = to_blocked(normal16((n, 128, 80, 80), 7))
    xd, od = x.to(gpu), o.to(gpu)
    up = capi.upsample2x_nc1hwc0(xd)
    assert bits_equal(up.cpu(), mv.upsample2x_blocked(x))
    fused = capi.upsample_cat_nc1hwc0([xd, od], [True, False]).cpu()
    assert bits_equal(fused, mv.upsample_cat_blocked([x, o], [True, False]))
    fused2 = capi.upsample_cat_nc1hwc0([od, xd], [False, True]).cpu()
    assert bits_equal(fused2, mv.upsample_cat_blocked([o, x], [False, True]))


def test_upsample_blocked_bit_patterns(gpu):
    """verify_fast_flow_bits.py:16-22: random int16 patterns, identity of bits."""
    from thintnpu_amd import capi
    for c1, h, w in ((16, 20, 20), (32, 20, 20), (16, 40, 40), (8, 40, 40), (2, 13, 17)):
        for n in (1, 3):
            x = random_bits16((n, c1, h, w, 16), c1 * h + w + n)
            assert bits_equal(capi.upsample2x_nc1hwc0(x.to(gpu)).cpu(), mv.upsample2x_blocked(x))
    # narrowed channel view (any N/C1 strides)
    x = random_bits16((3, 8, 10, 12, 16), 99)
    v = x[:, 2:6]
    assert bits_equal(capi.upsample2x_nc1hwc0(x.to(gpu)[:, 2:6]).cpu(), mv.upsample2x_blocked(v))
    # a non-dense layout goes through the element map
    xt = random_bits16((2, 3, 6, 5, 16), 98)
    vt = xt.transpose(2, 3)
    assert bits_equal(capi.upsample2x_nc1hwc0(xt.to(gpu).transpose(2, 3)).cpu(), mv.upsample2x_blocked(vt))


def test_upsample_streaming_block_windows(gpu):
    """Streaming upsample launches (output >= 4 MB) run their blocks in XCD
    runs of 32 tiles per window of 256 blocks: grids of whole windows only
    and grids with a partial last window (whose blocks keep their order),
    alone and with a copied input beside the upsampled one."""
    from thintnpu_amd import capi
    for n, c1, h, w in ((3, 16, 40, 40), (1, 64, 28, 36), (5, 7, 33, 31), (2, 12, 51, 49)):
        x = random_bits16((n, c1, h, w, 16), n * c1 + h)
        o = random_bits16((n, 3, 2 * h, 2 * w, 16), w)
        assert n * c1 * 4 * h * w * 32 >= 4 << 20  # the streaming form
        xd, od = x.to(gpu), o.to(gpu)
        assert bits_equal(capi.upsample2x_nc1hwc0(xd).cpu(), mv.upsample2x_blocked(x)), (n, c1, h, w)
        fused = capi.upsample_cat_nc1hwc0([od, xd], [False, True]).cpu()
        assert bits_equal(fused, mv.upsample_cat_blocked([o, x], [False, True])), (n, c1, h, w)


@pytest.mark.parametrize("n", [1, 8])
def test_upsample_cat_many_inputs(gpu, n):
    """Three to six inputs (the general input-count form of the plane
    kernel), upsampled and copied ones interleaved, an input with no channel
    blocks among them and at the end; n=8 crosses the streaming size from
    four inputs on."""
    from thintnpu_amd import capi
    h, w = 20, 24
    specs = [(3, True), (2, False), (0, False), (4, True), (1, False), (0, True)]
    parts, flags = [], []
    for k, (c1, up) in enumerate(specs):
        hh, ww = (h, w) if up else (2 * h, 2 * w)
        parts.append(random_bits16((n, c1, hh, ww, 16), 500 + 10 * n + k))
        flags.append(up)
    for count in (3, 4, 6):
        ps, fs = parts[:count], flags[:count]
        got = capi.upsample_cat_nc1hwc0([p.to(gpu) for p in ps], fs).cpu()
        assert bits_equal(got, mv.upsample_cat_blocked(ps, fs)), (n, count)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_upsample_nchw(gpu, dtype):
    """verify_all.py:88-94 shapes, atol 0."""
    from thintnpu_amd import capi
    for shape in ((1, 2, 5, 7), (2, 3, 13, 11), (1, 64, 40, 40), (2, 4, 6, 8)):
        x = rand_dtype(shape, dtype, sum(shape))
        assert bits_equal(capi.upsample2x_nchw(x.to(gpu)).cpu(), mv.upsample2x_nchw(x)), shape
    x = rand_dtype((2, 14, 15, 17), dtype, 3)
    sec = x[:, 7:]
    assert bits_equal(capi.upsample2x_nchw(x.to(gpu)[:, 7:]).cpu(), mv.upsample2x_nchw(sec))
    # rows the 16-byte form cannot take: odd widths, stepped and transposed inputs
    x = rand_dtype((3, 8, 41, 37), dtype, 6)
    assert bits_equal(capi.upsample2x_nchw(x.to(gpu)).cpu(), mv.upsample2x_nchw(x)), "41x37"
    x = rand_dtype((2, 5, 9, 22), dtype, 4)
    assert bits_equal(capi.upsample2x_nchw(x.to(gpu)[..., ::2]).cpu(), mv.upsample2x_nchw(x[..., ::2])), "stepped"
    x = rand_dtype((2, 5, 11, 9), dtype, 5)
    got = capi.upsample2x_nchw(x.to(gpu).transpose(2, 3)).cpu()
    assert bits_equal(got, mv.upsample2x_nchw(x.transpose(2, 3))), "transposed"


def test_pack_unpack(gpu):
    """C1 repack [1,64,160,160] -> [1,4,160,160,16]; zero pad of a partial C0
    block (conv_flow.cpp:420); any N; odd planes; non-dense inputs."""
    from thintnpu_amd import capi
    for shape in ((1, 64, 160, 160), (2, 3, 16, 16), (3, 17, 13, 17), (32, 64, 20, 20), (1, 40, 7, 9)):
        x = random_bits16(shape, sum(shape))
        y = capi.pack_nc1hwc0(x.to(gpu))
        assert bits_equal(y.cpu(), mv.pack_blocked(x)), shape
        back = capi.unpack_nc1hwc0(y, shape[1]).cpu()
        assert bits_equal(back, x), shape
    x = random_bits16((2, 32, 12, 10), 4)
    xt = x.transpose(2, 3)
    assert bits_equal(capi.pack_nc1hwc0(x.to(gpu).transpose(2, 3)).cpu(), mv.pack_blocked(xt))
    # channels-last x (NHWC memory seen as NCHW), packed and unpacked back into one
    cl = random_bits16((3, 11, 7, 48), 9).permute(0, 3, 1, 2)
    yc = capi.pack_nc1hwc0(cl.to(gpu))
    assert bits_equal(yc.cpu(), mv.pack_blocked(cl)), "channels-last pack"
    out = torch.empty(3, 11, 7, 48, dtype=torch.float16, device=gpu).permute(0, 3, 1, 2)
    assert bits_equal(capi.unpack_nc1hwc0(yc, 48, out=out).cpu(), cl), "channels-last unpack"


def test_movement_errors(gpu):
    from thintnpu_amd import capi
    a = torch.zeros(2, 3, device=gpu, dtype=torch.float16)
    b = torch.zeros(2, 4, device=gpu, dtype=torch.float32)
    with pytest.raises(capi.ThinError, match="matching dtypes"):
        capi.cat([a, b], 1)
    with pytest.raises(capi.ThinError):
        capi.upsample_cat_nc1hwc0([torch.zeros(1, 1, 2, 2, 16, device=gpu, dtype=torch.float16)], [False],
                                  out=torch.zeros(1, 1, 4, 4, 16, device=gpu, dtype=torch.float16))


MAXPOOL_SHAPES = [(256, 20, 20, 5), (128, 40, 40, 5), (512, 20, 20, 5), (32, 13, 17, 3), (16, 7, 9, 7),
                  (48, 1, 31, 5)]


def pool_specials(x):
    """+0/-0 ties in both orders, infinities and NaNs written into x (fp16)."""
    x = x.clone()
    flat = x.view(-1)
    n = flat.numel()
    g = gen(77)
    for value, count in ((0.0, n // 20), (-0.0, n // 20), (float("inf"), 3), (float("-inf"), 5), (float("nan"), 4)):
        flat[torch.randint(0, n, (count,), generator=g)] = value
    return x


def check_pool(got, want, what):
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan), f"{what}: NaN mask"
    assert bits_equal(got[~nan], want[~nan]), f"{what}: bits"


@pytest.mark.parametrize("n", [1, 3])
def test_maxpool_nc1hwc0(gpu, n):
    """verify_flow_ops.py:55-67 shapes (SPPF k5 and odd windows), any N."""
    from thintnpu_amd import capi
    for c, h, w, k in MAXPOOL_SHAPES:
        x = to_blocked(normal16((n, c, h, w), c + h + k))
        check_pool(capi.maxpool_nc1hwc0(x.to(gpu), k).cpu(), mv.maxpool_blocked(x, k), f"{c}x{h}x{w} k{k}")
    x = pool_specials(to_blocked(normal16((n, 32, 9, 11), 5)))
    for k in (1, 3, 5, 7, 9, 11, 13, 15):
        check_pool(capi.maxpool_nc1hwc0(x.to(gpu), k).cpu(), mv.maxpool_blocked(x, k), f"specials k{k}")


def pool_specials_packed(x, zero, seed):
    """Infinities, NaNs of both signs, subnormals of both signs and zeros of
    one sign (`zero` = 0.0, -0.0 or None) written into x (fp16): tiles the
    packed IEEE-maximum path takes, since only a +0/-0 tie separates it from
    the first-maximum rule."""
    x = x.clone()
    bits = x.view(-1).view(torch.int16)
    n = bits.numel()
    g = gen(seed)
    at = lambda count: torch.randint(0, n, (count,), generator=g)  # noqa: E731
    sub = torch.randint(1, 0x400, (n // 50,), generator=g, dtype=torch.int32)
    sub = torch.where(torch.rand(n // 50, generator=g) < 0.5, sub, sub | 0x8000)
    bits[at(n // 50)] = (sub - ((sub >> 15) << 16)).to(torch.int16)  # subnormals, both signs
    for pattern, count in ((0x7C00, 3), (0xFC00 - 0x10000, 5), (0x7E00, 3), (0xFE01 - 0x10000, 3), (0x7C01, 2)):
        bits[at(count)] = pattern  # +inf, -inf, +qNaN, -NaN, +sNaN payload
    if zero is not None:
        x.view(-1)[at(n // 20)] = zero
    return x


@pytest.mark.parametrize("zero", [None, 0.0, -0.0])
def test_maxpool_packed_specials(gpu, zero):
    """fp16 NC1HWC0 tiles without a +0/-0 mix: NaN propagation, infinities,
    subnormals and single-signed zeros through the packed maximum."""
    from thintnpu_amd import capi
    x = pool_specials_packed(to_blocked(normal16((2, 64, 20, 20), 31)), zero, 41)
    for k in (1, 3, 5, 7, 15):
        check_pool(capi.maxpool_nc1hwc0(x.to(gpu), k).cpu(), mv.maxpool_blocked(x, k), f"packed zero={zero} k{k}")
    # subnormal-only windows: maxima between subnormals are kept exactly
    tiny = to_blocked(normal16((1, 32, 12, 12), 5)) * 1e-6
    tiny[tiny == 0] = 2.0 ** -24
    assert (tiny.abs() < 6.1e-5).all() and (tiny != 0).all()
    check_pool(capi.maxpool_nc1hwc0(tiny.to(gpu), 5).cpu(), mv.maxpool_blocked(tiny, 5), "subnormal planes")


def test_maxpool_mixed_blocks(gpu):
    """One plane holds +0/-0 ties (first-maximum selects) while the rest of the
    launch takes the packed path."""
    from thintnpu_amd import capi
    x = to_blocked(normal16((2, 64, 20, 20), 12))
    x[1, 2] = pool_specials(x[1, 2:3])[0]
    x[0, 1] = -x[0, 1].abs()
    x[0, 1, ::3, ::2] = -0.0
    x[0, 1, 1::4, 1::3] = 0.0
    for k in (3, 5, 9):
        check_pool(capi.maxpool_nc1hwc0(x.to(gpu), k).cpu(), mv.maxpool_blocked(x, k), f"mixed k{k}")


def test_maxpool_views(gpu):
    from thintnpu_amd import capi
    x = to_blocked(normal16((2, 64, 12, 10), 8))
    xd = x.to(gpu)
    got = capi.maxpool_nc1hwc0(xd[:, 1:3], 5).cpu()
    check_pool(got, mv.maxpool_blocked(x[:, 1:3].contiguous(), 5), "channel-block slice")
    parent = random_bits16((2, 6, 12, 10, 16), 9)
    pd = parent.to(gpu)
    capi.maxpool_nc1hwc0(xd[:, :2], 3, out=pd[:, 4:6])
    got = pd.cpu()
    check_pool(got[:, 4:6], mv.maxpool_blocked(x[:, :2].contiguous(), 3), "narrowed output")
    assert bits_equal(got[:, :4], parent[:, :4])


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_maxpool2d_nchw(gpu, dtype):
    """thin_backend.maxpool2d (backend.cpp:245-266) semantics, any odd k, any strides."""
    from thintnpu_amd import capi
    x = pool_specials(normal16((2, 5, 13, 17), 3)).to(dtype)
    for k in (1, 3, 5, 7, 15):
        check_pool(capi.maxpool2d_nchw(x.to(gpu), k).cpu(), mv.maxpool_nchw(x, k), f"nchw k{k}")
    t = x.transpose(2, 3)
    check_pool(capi.maxpool2d_nchw(x.to(gpu).transpose(2, 3), 5).cpu(), mv.maxpool_nchw(t.contiguous(), 5),
               "transposed")
    with pytest.raises(capi.ThinError, match="odd integer"):
        capi.maxpool2d_nchw(x.to(gpu), 4)


def test_fill(gpu):
    from thintnpu_amd import capi
    for dtype, value in ((torch.float16, 1.5), (torch.float32, -2.25), (torch.float64, 1e300), (torch.bfloat16, 3.0),
                         (torch.int64, 2 ** 60 + 1), (torch.int32, -7), (torch.int16, 300), (torch.uint8, 200),
                         (torch.bool, 1), (torch.float16, float("nan")), (torch.float32, float("-inf"))):
        t = torch.zeros((3, 37, 5), dtype=dtype, device=gpu)
        capi.fill(t, value)
        want = torch.full((3, 37, 5), value, dtype=dtype)
        assert torch.equal(t.cpu(), want) or (dtype.is_floating_point and torch.isnan(want).all() and
                                              torch.isnan(t.cpu()).all()), (dtype, value)
        parent = torch.zeros((3, 37, 9), dtype=dtype, device=gpu)
        capi.fill(parent[:, ::2, 1:6], value)
        ref = torch.zeros((3, 37, 9), dtype=dtype)
        ref[:, ::2, 1:6] = want[:, :19]
        got = parent.cpu()
        assert torch.equal(torch.isnan(got.float()), torch.isnan(ref.float())) if dtype.is_floating_point else True
        assert torch.equal(got.nan_to_num(), ref.nan_to_num()) if dtype.is_floating_point else torch.equal(got, ref)


@pytest.mark.parametrize("c,h,w,k", [(16, 3, 300, 5), (16, 5, 130, 15), (32, 9, 64, 15), (16, 33, 7, 3)])
def test_maxpool_wide_rows(gpu, c, h, w, k):
    """Rows too wide for the LDS band (register form) and tall narrow planes."""
    from thintnpu_amd import capi
    x = pool_specials(to_blocked(normal16((2, c, h, w), w + k)))
    check_pool(capi.maxpool_nc1hwc0(x.to(gpu), k).cpu(), mv.maxpool_blocked(x, k), f"{c}x{h}x{w} k{k}")
    y = pool_specials(normal16((1, 3, h, w * 5), k))
    check_pool(capi.maxpool2d_nchw(y.to(gpu), k).cpu(), mv.maxpool_nchw(y, k), f"nchw {h}x{w * 5} k{k}")


@pytest.mark.parametrize("k", [3, 5])
def test_maxpool_band_and_register_forms(gpu, k):
    """Planes too large for the whole-plane kernel: bands of rows staged in
    LDS (a 72x72 NC1HWC0 plane, through both the packed maximum and the
    first-maximum selects), and the register window for rows too wide for a
    band of 2R + 1 rows (520 pixels NC1HWC0, 8200 NCHW)."""
    from thintnpu_amd import capi
    band = to_blocked(normal16((2, 32, 72, 72), 70 + k))
    for what, x in (("band, +0/-0 ties", pool_specials(band)), ("band, packed", pool_specials_packed(band, 0.0, 90 + k))):
        check_pool(capi.maxpool_nc1hwc0(x.to(gpu), k).cpu(), mv.maxpool_blocked(x, k), f"{what} k{k}")
    x = pool_specials(to_blocked(normal16((1, 16, 8, 520), 60 + k)))
    check_pool(capi.maxpool_nc1hwc0(x.to(gpu), k).cpu(), mv.maxpool_blocked(x, k), f"register 8x520 k{k}")
    y = pool_specials(normal16((1, 2, 5, 8200), 50 + k))
    check_pool(capi.maxpool2d_nchw(y.to(gpu), k).cpu(), mv.maxpool_nchw(y, k), f"nchw register 5x8200 k{k}")


def test_cat_beyond_4gib(gpu):
    """A cat whose output passes 4 GiB (the second input lands 2 GiB in): the
    row and column offsets are 64-bit.  Small integers make torch.cat on the
    device an exact reference at this size."""
    from thintnpu_amd import capi
    half = (1 << 30) + 64
    a = (torch.arange(half, device=gpu, dtype=torch.int32) % 2039).to(torch.float16).view(1, half)
    b = (torch.arange(half, device=gpu, dtype=torch.int32) % 1021).to(torch.float16).view(1, half)
    assert torch.equal(capi.cat([a, b], 1), torch.cat([a, b], 1))
    del a, b
    torch.cuda.empty_cache()


SPPF_SHAPES = [(256, 20, 20, 5, 3), (32, 13, 17, 3, 2), (16, 7, 9, 7, 1), (32, 9, 11, 1, 3), (16, 5, 6, 15, 4)]


@pytest.mark.parametrize("n", [1, 2])
def test_sppf_chain(gpu, n):
    """thin_sppf_nc1hwc0 = cat([x, p(x), p(p(x)), ...], 1): bit-exact against
    chained oracle pools (+0/-0 ties through the first-maximum path, special
    values through the packed path)."""
    from thintnpu_amd import capi
    for c, h, w, k, r in SPPF_SHAPES:
        x = to_blocked(normal16((n, c, h, w), c + h + k))
        check_pool(capi.sppf_nc1hwc0(x.to(gpu), k, r).cpu(), mv.sppf_blocked(x, k, r), f"{c}x{h}x{w} k{k} r{r}")
    x = pool_specials(to_blocked(normal16((n, 32, 9, 11), 6)))
    for k in (3, 5, 7):
        check_pool(capi.sppf_nc1hwc0(x.to(gpu), k, 3).cpu(), mv.sppf_blocked(x, k, 3), f"specials k{k}")
    for zero in (None, 0.0, -0.0):
        x = pool_specials_packed(to_blocked(normal16((n, 64, 20, 20), 32)), zero, 43)
        check_pool(capi.sppf_nc1hwc0(x.to(gpu), 5, 3).cpu(), mv.sppf_blocked(x, 5, 3), f"packed zero={zero}")


def test_pool_twenty_square_planes(gpu):
    """The compile-time 20x20 form (k5, at least 256 planes: SPPF at a
    640-pixel input): zero maxima with +0/-0 ties in both orders redone by
    first-maximum selects inside packed-maximum planes, NaN and infinities,
    for the single pool and the SPPF chain."""
    from thintnpu_amd import capi
    x = to_blocked(normal16((16, 256, 20, 20), 74))
    for n, c1 in ((0, 1), (3, 7), (15, 15)):
        plane = -x[n, c1].abs()
        plane[::3, ::2] = -0.0
        plane[1::4, 1::3] = 0.0
        x[n, c1] = plane
    x[5, 9] = pool_specials(x[5, 9:10])[0]
    check_pool(capi.maxpool_nc1hwc0(x.to(gpu), 5).cpu(), mv.maxpool_blocked(x, 5), "20x20 maxpool k5")
    check_pool(capi.sppf_nc1hwc0(x.to(gpu), 5, 3).cpu(), mv.sppf_blocked(x, 5, 3), "20x20 sppf k5 x3")


@pytest.mark.parametrize("n", [15, 16])
def test_pool_block_forms(gpu, n):
    """Under 256 (n, c1) planes a block pools one C0 half of a plane (n=15: 240
    planes); from 256 on it pools all 16 lanes (n=16): both forms bit-exact,
    with special values and +0/-0 ties, for the single pool and the SPPF chain."""
    from thintnpu_amd import capi
    x = pool_specials(to_blocked(normal16((n, 256, 7, 9), 71)))
    check_pool(capi.maxpool_nc1hwc0(x.to(gpu), 5).cpu(), mv.maxpool_blocked(x, 5), f"n={n} maxpool k5")
    check_pool(capi.sppf_nc1hwc0(x.to(gpu), 5, 3).cpu(), mv.sppf_blocked(x, 5, 3), f"n={n} sppf k5 x3")
    for zero in (0.0, -0.0):
        x = pool_specials_packed(to_blocked(normal16((n, 256, 6, 5), 72)), zero, 44)
        check_pool(capi.sppf_nc1hwc0(x.to(gpu), 3, 2).cpu(), mv.sppf_blocked(x, 3, 2), f"n={n} packed zero={zero}")


def test_sppf_large_planes_and_views(gpu):
    """A 40x40 plane (118 KB of LDS per block), a 64x64 plane (beyond one
    block's LDS: copy plus chained pools), a channel-block slice as x, and an
    output that is a slice of a larger tensor."""
    from thintnpu_amd import capi
    for c, h, w in ((32, 40, 40), (16, 64, 64)):
        x = pool_specials(to_blocked(normal16((2, c, h, w), h)))
        check_pool(capi.sppf_nc1hwc0(x.to(gpu), 5, 3).cpu(), mv.sppf_blocked(x, 5, 3), f"{c}x{h}x{w}")
    x = to_blocked(normal16((2, 64, 12, 10), 9))
    xd = x.to(gpu)
    check_pool(capi.sppf_nc1hwc0(xd[:, 1:3], 5, 3).cpu(), mv.sppf_blocked(x[:, 1:3].contiguous(), 5, 3), "x slice")
    parent = random_bits16((2, 12, 12, 10, 16), 10)
    pd = parent.to(gpu)
    capi.sppf_nc1hwc0(xd[:, :2], 3, 2, out=pd[:, 5:11])
    got = pd.cpu()
    check_pool(got[:, 5:11], mv.sppf_blocked(x[:, :2].contiguous(), 3, 2), "out slice")
    assert bits_equal(got[:, :5], parent[:, :5]) and bits_equal(got[:, 11:], parent[:, 11:])
    with pytest.raises(capi.ThinError, match="repeats"):
        capi.sppf_nc1hwc0(xd[:, :2], 5, 0, out=torch.empty((2, 2, 12, 10, 16), dtype=torch.float16, device=gpu))
    with pytest.raises(capi.ThinError, match="out must be"):
        capi.sppf_nc1hwc0(xd[:, :2], 5, 3, out=torch.empty((2, 6, 12, 10, 16), dtype=torch.float16, device=gpu))
