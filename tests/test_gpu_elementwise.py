"""GPU parity of the elementwise entry points (through the C ABI) against the
CPU oracle.  Bars: add/sub/mul/div bit-exact (correctly rounded), sigmoid /
SiLU / fused chains <= 2 fp16 ulp; fp32 tensors within 1e-5 relative."""
import math

import pytest
import torch

from oracle import elementwise as ew
from oracle.numerics import assert_ulp, assert_fused_cancel, bits_equal, ulp16_spacing, ulp_report
from tests.helpers import normal16, random_bits16, specials16, to_blocked, gen

pytestmark = pytest.mark.gpu

SHAPES = [(1,), (3,), (7,), (100,), (2047,), (2048,), (2049,), (16385,), (65537,), (0,), (), (3, 5, 7)]


def run_binary(capi, op, a, b, dev, alpha=1.0):
    return capi.binary(op, a.to(dev), b.to(dev), alpha).cpu()


def check(actual, expected, max_ulp, what):
    if expected.dtype == torch.float16:
        return assert_ulp(actual, expected, max_ulp, what)
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=1e-6, equal_nan=True, msg=what)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_binary_shapes(gpu, dtype):
    from thintnpu_amd import capi
    g = gen(42)
    for shape in SHAPES:
        a = (torch.rand(shape, generator=g) * 2 - 1).to(dtype)
        b = (torch.rand(shape, generator=g) + 0.5).to(dtype)
        for op in (0, 1, 2, 3):
            check(run_binary(capi, op, a, b, gpu), ew.binary(op, a, b), 0, f"op{op} {shape}")
    a = torch.rand(2, 5, 7, generator=g).to(dtype)
    b = (torch.rand(2, 5, 7, generator=g) + 0.5).to(dtype)
    for op in (0, 1, 2, 3):
        got = capi.binary(op, a.to(gpu).transpose(0, 2), b.to(gpu).transpose(0, 2)).cpu()
        check(got, ew.binary(op, a.transpose(0, 2), b.transpose(0, 2)), 0, f"transposed op{op}")
    for op in (0, 3):
        for alpha in (2.0, 0.3):
            check(run_binary(capi, op, a, b, gpu, alpha), ew.binary(op, a, b, alpha), 0, f"alpha {alpha}")


def test_binary_all_encodings_bit_exact(gpu):
    from thintnpu_amd import capi
    a = torch.cat([random_bits16((1 << 20,), 1), specials16().repeat_interleave(16)])
    b = torch.cat([random_bits16((1 << 20,), 2), specials16().repeat(16)])
    for op in (0, 1, 2, 3):
        assert_ulp(run_binary(capi, op, a, b, gpu), ew.binary(op, a, b), 0, f"op{op} encodings")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_strided_broadcast_cases(gpu, dtype):
    """The case list of the reference's strided-binary test (verify_strided_binary.py:24-33)."""
    from thintnpu_amd import capi
    g = gen(71)
    for width in (16, 48, 2048, 2064, 8400):
        data = torch.randn(4, width * 2 + 16, generator=g).to(dtype)
        full = torch.randn(4, width, generator=g).to(dtype)
        scalar = torch.tensor(2, dtype=dtype)
        dd, fd, sd = data.to(gpu), full.to(gpu), scalar.to(gpu)
        cases = [
            ("interleaved-left", lambda d, f, s: (d[:, 1:1 + 2 * width:2], f)),
            ("interleaved-right", lambda d, f, s: (f, d[:, :2 * width:2])),
            ("unaligned", lambda d, f, s: (d[:, 1:1 + width], f)),
            ("row-broadcast", lambda d, f, s: (f, f[:1])),
            ("column-broadcast", lambda d, f, s: (f, f[:, :1])),
            ("scalar", lambda d, f, s: (f, s)),
            ("both-expanded", lambda d, f, s: (f[:1], f[:, :1])),
            ("rank-four", lambda d, f, s: (f.view(2, 2, 1, width), d[:, :2 * width:2].view(2, 2, 1, width))),
        ]
        for label, make in cases:
            xc, yc = make(data, full, scalar)
            xg, yg = make(dd, fd, sd)
            for op in (0, 1, 2, 3):
                for alpha in ((1.0, 0.3) if op in (0, 3) else (1.0,)):
                    got = capi.binary(op, xg, yg, alpha).cpu()
                    check(got, ew.binary(op, xc, yc, alpha), 0, f"{label} w{width} op{op} a{alpha}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_narrowed_blocked_views(gpu, dtype):
    """Channel-lane slices of 5-D NC1HWC0 tensors (verify_narrow_binary.py:24-69)."""
    from thintnpu_amd import capi
    g = gen(2931)
    for h, w in ((80, 80), (44, 76), (20, 20), (1, 16), (1, 2064)):
        full = torch.randn(1, 3, h, w, 16, generator=g).to(dtype)
        grid = torch.randn(h, w, 2, generator=g).to(dtype)
        anchors = torch.randn(1, 3, 1, 1, 2, generator=g).to(dtype)
        contiguous = torch.randn(1, 3, h, w, 2, generator=g).to(dtype)
        scalar = torch.tensor(2, dtype=dtype)
        cpu = dict(full=full, grid=grid, anchors=anchors, contiguous=contiguous, scalar=scalar)
        dev = {k: v.to(gpu) for k, v in cpu.items()}
        cases = {
            "slice-scalar": lambda t: (t["full"][..., :2], t["scalar"]),
            "offset-slice-scalar": lambda t: (t["full"][..., 2:4], t["scalar"]),
            "grid": lambda t: (t["contiguous"], t["grid"]),
            "anchors": lambda t: (t["contiguous"], t["anchors"]),
            "narrow-both": lambda t: (t["full"][..., :2], t["full"][..., 2:4]),
            "narrow-swapped": lambda t: (t["scalar"], t["full"][..., 2:4]),
            "narrow-broadcast": lambda t: (t["full"][:, :1, ..., :2], t["full"][..., :1]),
            "lanes-four": lambda t: (t["full"][..., 1:5], t["scalar"]),
            "lanes-eight": lambda t: (t["full"][..., 1:9], t["scalar"]),
        }
        for label, make in cases.items():
            xc, yc = make(cpu)
            xg, yg = make(dev)
            for op in (0, 1, 2, 3):
                got = capi.binary(op, xg, yg).cpu()
                check(got, ew.binary(op, xc, yc), 0, f"{label} {h}x{w} op{op}")



@pytest.mark.parametrize("n,c1,h,w", [(2, 8, 20, 20), (1, 16, 40, 40), (3, 4, 7, 9), (2, 130, 2, 2), (1, 1, 1, 1)])
def test_channel_broadcast_blocked(gpu, n, c1, h, w):
    """aten add / sub / mul / div of an NC1HWC0 fp16 tensor and a per-channel
    [1,C1,1,1,16] operand (ops.cpp:464-497), full and C2f-narrowed
    (x[:, C1/2:]) views, both operand orders and alpha: the flat per-channel
    kernel (C1 <= 128) and the generic map path beyond it give the oracle's
    bits, specials included."""
    from thintnpu_amd import capi
    g = gen(4000 + n * 131 + c1)
    x = torch.randn(n, c1, h, w, 16, generator=g).half()
    flat = x.view(-1)
    sp = specials16()
    flat[: min(flat.numel(), sp.numel())] = sp[: flat.numel()]
    s = (torch.randn(1, c1, 1, 1, 16, generator=g) * 2).half()
    s.view(-1)[:3] = torch.tensor([0.0, float("inf"), float("nan")]).half()
    xd, sd = x.to(gpu), s.to(gpu)
    views = [("full", lambda t: t)]
    if c1 > 1:
        views.append(("narrowed", lambda t: t[:, c1 // 2:]))
    for label, view in views:
        xc, sc_, xg, sg = view(x), view(s), view(xd), view(sd)
        for op in (0, 1, 2, 3):
            for alpha in ((1.0, 0.3) if op in (0, 1) else (1.0,)):
                got = capi.binary(op, xg, sg, alpha).cpu()
                check(got, ew.binary(op, xc, sc_.expand_as(xc), alpha), 0, f"{label} x op s op{op} a{alpha}")
                got = capi.binary(op, sg, xg, alpha).cpu()
                check(got, ew.binary(op, sc_.expand_as(xc), xc, alpha), 0, f"{label} s op x op{op} a{alpha}")

def test_scalar_operands(gpu):
    from thintnpu_amd import capi
    x = torch.cat([random_bits16((100_000,), 5), specials16()])
    xg = x.to(gpu)
    for sc in (0.17677669529663687, 0.5, 3.0, -7.25):
        for op in (0, 1, 2, 3):
            for first in ((False, True) if op in (0, 3) else (False,)):
                got = capi.binary_scalar(op, xg, sc, first).cpu()
                assert_ulp(got, ew.binary_scalar(op, x, sc, first), 0, f"scalar {sc} op{op} first{first}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_unary(gpu, dtype):
    from thintnpu_amd import capi
    for shape in ((1,), (5000,), (65537,), (0,), (), (2, 7, 5, 7)):
        n = math.prod(shape)
        x = torch.linspace(-8, 8, max(1, n))[:n].reshape(shape).to(dtype)
        for op, ref in ((capi.SIGMOID, ew.sigmoid), (capi.SILU, ew.silu)):
            check(capi.unary(op, x.to(gpu)).cpu(), ref(x), 2, f"unary{op} {shape}")
    if dtype == torch.float16:
        x = torch.cat([random_bits16((1 << 20,), 9), specials16()])
        for op, ref in ((capi.SIGMOID, ew.sigmoid), (capi.SILU, ew.silu)):
            rep = assert_ulp(capi.unary(op, x.to(gpu)).cpu(), ref(x), 2, f"unary{op} encodings")
            assert rep["exact"] > 0.99 * rep["finite"]


def test_unary_in_place_on_strided_parent(gpu):
    """silu_ on a channel split of a parent tensor (verify_ops.py:105-115)."""
    from thintnpu_amd import capi
    a = normal16((2, 7, 5, 7), 10)
    x = a.to(gpu)
    part = torch.split(x, [3, 4], 1)[1]
    capi.unary(capi.SILU, part, out=part)
    ref = a.clone()
    torch.split(ref, [3, 4], 1)[1].copy_(ew.silu(torch.split(a, [3, 4], 1)[1]))
    assert_ulp(x.cpu(), ref, 2, "silu_ in place")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_row_views(gpu, dtype):
    """Operands that coalesce to rows of contiguous vectors with their own row
    strides (narrowed NC1HWC0 halves, column slices, a row broadcast), in
    place and into dense outputs: unary, binary and copy against the oracle."""
    from thintnpu_amd import capi
    g = gen(4242)
    parent = torch.randn(3, 8, 7, 9, 16, generator=g).to(dtype)
    other = torch.randn(3, 8, 7, 9, 16, generator=g).to(dtype)
    pd, od = parent.to(gpu), other.to(gpu)
    halves = [(lambda t: t[:, 4:]), (lambda t: t[:, :4]), (lambda t: t[:, 2:6])]
    for k, view in enumerate(halves):
        xc, xg = view(parent), view(pd)
        for op, ref in ((capi.SIGMOID, ew.sigmoid), (capi.SILU, ew.silu)):
            check(capi.unary(op, xg).cpu(), ref(xc), 2, f"unary{op} view{k}")
        for op in (0, 1, 2, 3):
            check(capi.binary(op, xg, view(od)).cpu(), ew.binary(op, xc, view(other)), 0, f"binary{op} view{k}")
            check(capi.binary(op, xg, od[:, :4]).cpu(), ew.binary(op, xc, other[:, :4]), 0, f"binary{op} mixed{k}")
        dense = torch.empty(xg.shape, dtype=dtype, device=gpu)
        capi.copy(xg, dense)
        assert torch.equal(dense.cpu().view(torch.uint8), xc.contiguous().view(torch.uint8)), f"copy view{k}"
    # in place on a narrowed half: the rest of the parent stays as it was
    work = pd.clone()
    capi.unary(capi.SILU, work[:, 4:], out=work[:, 4:])
    expect = parent.clone()
    expect[:, 4:] = ew.silu(parent[:, 4:])
    check(work.cpu(), expect, 2, "silu_ in place on a half")
    # column slices of a matrix and a broadcast row
    mat = torch.randn(40, 272, generator=g).to(dtype)
    row = torch.randn(1, 128, generator=g).to(dtype)
    md, rd = mat.to(gpu), row.to(gpu)
    for op in (0, 1, 2, 3):
        check(capi.binary(op, md[:, 8:136], rd).cpu(), ew.binary(op, mat[:, 8:136], row), 0, f"binary{op} row")
        check(capi.binary(op, rd, md[:, 136:264]).cpu(), ew.binary(op, row, mat[:, 136:264]), 0, f"binary{op} row first")


# C1's recorded bar: how many elements (of 1.6 M at N=1, 52 M at N=32) may pass
# only through the cancellation arm, and how many fp16 ulps apart.  Measured:
# none at either batch; every element is within 2 ulp (N=32: 52,427,659 of
# 52,428,800 exact), so the arm is kept for other inputs only.
C1_CANCEL_ONLY = {1: (0, 0), 32: (0, 0)}


@pytest.mark.parametrize("n", [1, 32])
def test_silu_add_c1(gpu, n):
    """C1: z = y + SiLU(x) on NC1HWC0 [n,4,160,160,16] from NCHW N(0,1), seed 1."""
    from thintnpu_amd import capi
    x = to_blocked(normal16((n, 64, 160, 160), 1))
    y = to_blocked(normal16((n, 64, 160, 160), 101))
    got = capi.silu_add(x.to(gpu), y.to(gpu)).cpu()
    # <= 2 fp16 ulp, or <= 4 fp32 ulp of |silu(x)| where y + silu(x) cancels
    rep = assert_fused_cancel(got, ew.silu_add(x, y), ew.silu(x.float()), 2, 4, f"silu_add n={n}")
    assert rep["exact"] > 0.999 * rep["finite"]
    # the side report: distance to the op-by-op half chain (y + silu(x), two roundings)
    unfused = ulp_report(got, ew.silu_add_unfused(x, y))
    print(f"silu_add n={n}: {rep['finite']} finite, {rep['exact']} exact, max {rep['max_ulp']} ulp; "
          f"{rep['cancel_only']} pass only through the cancellation arm (max {rep['cancel_max_ulp']} ulp); "
          f"against the half chain: max {unfused['max_ulp']} ulp, {unfused['exact']} exact")
    assert rep["cancel_only"] <= C1_CANCEL_ONLY[n][0] and rep["cancel_max_ulp"] <= C1_CANCEL_ONLY[n][1]


def test_silu_add_all_encodings(gpu):
    """y + SiLU(x) for every fp16 encoding of x against each special y (signed
    zeros, infinities, NaN, extremes, subnormals) and a random y: the fp16
    SiLU's argument split, Newton quotient and special-operand fix-up (x <=
    -88.7 where exp(-x) overflows, x = -inf -> NaN, x = +inf -> +inf) within
    the fused bound, NaNs and infinities where the oracle has them."""
    from thintnpu_amd import capi
    x_all = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(torch.float16)
    ys = list(specials16()) + [random_bits16((65536,), 21)]
    x = x_all.repeat(len(ys))
    y = torch.cat([yv.expand(65536) if yv.dim() == 0 else yv for yv in ys]).contiguous()
    got = capi.silu_add(x.to(gpu), y.to(gpu)).cpu()
    rep = assert_fused_cancel(got, ew.silu_add(x, y), ew.silu(x.float()), 2, 4, "silu_add encodings")
    assert rep["exact"] > 0.999 * rep["finite"]


C2_SHAPES = [(128, 80, 80), (256, 40, 40), (512, 20, 20)]


def report_fp32_chain(got, x, s, b, what):
    """The side report against the single-rounding fp32 chain SiLU(x*s + b):
    the half chain's two intermediate roundings (x*s and the add, each at most
    half an fp16 ulp, passed through SiLU's slope <= 1.1) plus the output
    roundings bound the distance, which is large in fp16 ulps only where
    x*s + b cancels."""
    r = ew.affine_silu_fp32(x, s, b)
    rep = ulp_report(got, r)
    xs = x.double() * s.double()
    t = xs + b.double()
    bound = 1.1 * 0.5 * (ulp16_spacing(xs) + ulp16_spacing(t)) + 3 * ulp16_spacing(r)
    d = (got.double() - r.double()).abs()
    ratio = float((d / bound).max())
    print(f"{what} against the fp32 chain: {rep['exact']} of {rep['finite']} exact, max {rep['max_ulp']} ulp, "
          f"max abs {float(d.max()):.3g}, {ratio:.2f} of the rounding bound")
    assert ratio <= 1.0, f"{what}: {ratio} of the rounding bound"


def c2_inputs(n, c, h, w, seed=2):
    x = to_blocked(normal16((n, c, h, w), seed))
    g = gen(seed + 1000)
    s = (torch.rand((1, c, 1, 1), generator=g) + 0.5).half()
    b = (torch.randn((1, c, 1, 1), generator=g) * 0.1).half()
    return x, to_blocked(s), to_blocked(b)


@pytest.mark.parametrize("n", [1, 32])
@pytest.mark.parametrize("chw", C2_SHAPES)
def test_affine_silu_c2(gpu, n, chw):
    """C2: y = SiLU(x*s + b), per-channel [1,C,1,1] broadcast in NC1HWC0, plus the
    C2f half-split narrowed view x[:, C/2:] (blocked dim-1 offset C/32)."""
    from thintnpu_amd import capi
    c, h, w = chw
    x, s, b = c2_inputs(n, c, h, w)
    xg, sg, bg = x.to(gpu), s.to(gpu), b.to(gpu)
    got = capi.affine_silu(xg, sg, bg).cpu()
    assert_ulp(got, ew.affine_silu(x, s, b), 2, f"affine_silu {n} {chw}")
    report_fp32_chain(got, x, s, b, f"affine_silu n={n} {chw}")
    c1 = c // 16
    xn, sn, bn = x[:, c1 // 2:], s[:, c1 // 2:], b[:, c1 // 2:]
    got = capi.affine_silu(xg[:, c1 // 2:], sg[:, c1 // 2:], bg[:, c1 // 2:]).cpu()
    assert_ulp(got, ew.affine_silu(xn, sn, bn), 2, f"affine_silu narrowed {n} {chw}")


@pytest.mark.parametrize("case", ["per_image_scale", "channel_stride", "wide_c1", "tiny_planes",
                                  "narrowed_out", "strided_scale", "n1_offset", "mid_size_tail"])
def test_affine_silu_layouts(gpu, case):
    """Every NC1HWC0 layout the fused kernel accepts, flat-span and per-plane
    forms alike, against the op-by-op fp16 chain; outputs written through a
    view leave the rest of their parent untouched."""
    from thintnpu_amd import capi
    n, c, h, w = {"per_image_scale": (3, 64, 5, 7), "channel_stride": (2, 128, 6, 10),
                  "wide_c1": (2, 4096, 2, 3), "tiny_planes": (5, 16, 1, 1), "narrowed_out": (4, 96, 9, 11),
                  "strided_scale": (2, 64, 8, 8), "n1_offset": (1, 256, 20, 20),
                  # 209,824 vectors (3.4 MB): two vectors per thread with cached loads,
                  # a partial last block
                  "mid_size_tail": (2, 128, 79, 83)}[case]
    x, s, b = c2_inputs(n, c, h, w, seed=len(case))
    if case == "per_image_scale":
        s = (torch.rand((n, c // 16, 1, 1, 16), generator=gen(5)) + 0.5).half()
        b = (torch.randn((n, c // 16, 1, 1, 16), generator=gen(6)) * 0.1).half()
    xv = lambda t: t  # noqa: E731
    sv = lambda t: t  # noqa: E731
    if case == "channel_stride":
        xv = sv = lambda t: t[:, ::2]  # noqa: E731
    if case == "strided_scale":
        s2 = (torch.rand((1, c // 8, 1, 1, 16), generator=gen(7)) + 0.5).half()
        b2 = (torch.randn((1, c // 8, 1, 1, 16), generator=gen(8)) * 0.1).half()
        s, b = s2, b2
        sv = lambda t: t[:, ::2]  # noqa: E731
    if case == "n1_offset":
        xv = sv = lambda t: t[:, 3:11]  # noqa: E731
    xg, sg, bg = xv(x.to(gpu)), sv(s.to(gpu)), sv(b.to(gpu))
    ref = ew.affine_silu(xv(x), sv(s), sv(b).expand_as(sv(s)))
    if case == "narrowed_out":
        fill = random_bits16((n, c // 16 + 2, h, w, 16), 11)
        parent = fill.to(gpu)
        capi.affine_silu(xg, sg, bg, out=parent[:, 2:])
        got = parent.cpu()
        assert_ulp(got[:, 2:], ref, 2, case)
        assert bits_equal(got[:, :2], fill[:, :2])
        return
    got = capi.affine_silu(xg, sg, bg).cpu()
    assert_ulp(got, ref, 2, case)


def test_copy_bit_exact(gpu):
    from thintnpu_amd import capi
    raw = random_bits16((3, 32, 48), 913)
    for view in (lambda t: t.transpose(1, 2), lambda t: t[..., 2:4], lambda t: t[:, ::2, ::2],
                 lambda t: t[:, :1].expand(-1, 31, -1), lambda t: t):
        src = view(raw.to(gpu))
        dst = torch.empty(src.shape, dtype=src.dtype, device=gpu)
        capi.copy(src, dst)
        assert bits_equal(dst.cpu(), view(raw).contiguous())
    for dtype in (torch.float32, torch.int64, torch.uint8):
        t = torch.arange(3 * 5 * 7).reshape(3, 5, 7).to(dtype)
        src = t.to(gpu).permute(2, 0, 1)
        dst = torch.empty(src.shape, dtype=dtype, device=gpu)
        capi.copy(src, dst)
        assert torch.equal(dst.cpu(), t.permute(2, 0, 1).contiguous())


def test_errors_are_reported(gpu):
    from thintnpu_amd import capi
    a = torch.ones(4, device=gpu, dtype=torch.float16)
    b = torch.ones(4, device=gpu, dtype=torch.float32)
    with pytest.raises(capi.ThinError, match="matching dtypes"):
        capi.binary(capi.ADD, a, b)
    with pytest.raises(capi.ThinError, match="float32/float16"):
        capi.unary(capi.SILU, torch.ones(4, device=gpu, dtype=torch.int64))


@pytest.mark.parametrize("dtype,shape", [(torch.float16, (4, 64, 48, 48)), (torch.float32, (2, 64, 48, 48))])
def test_transposed_operand_first(gpu, dtype, shape):
    """An operand that is a batched 2-D transpose of a dense output of 1 MB or
    more goes through the tiled transpose into the output first.  The results
    equal, bit for bit, the same op on a contiguous copy of that operand: as
    either operand of every binary op (alpha 1 and 0.5), with a scalar, through
    the unary ops and silu_add; and against the oracle.  An output that shares
    bytes with an operand (x += y^T) keeps the direct path."""
    from thintnpu_amd import capi
    n, c, h, w = shape
    bits = torch.int16 if dtype == torch.float16 else torch.int32
    same = lambda a, b: torch.equal(a.cpu().view(bits), b.cpu().view(bits))  # noqa: E731
    xt = torch.randn(n, h, w, c, generator=gen(7)).to(dtype).to(gpu).permute(0, 3, 1, 2)
    xc = xt.contiguous()
    y = (torch.randn(shape, generator=gen(8)).abs() + 0.5).to(dtype).to(gpu)
    for op in range(4):
        for alpha in ((1.0, 0.5) if op < 2 else (1.0,)):
            got = capi.binary(op, xt, y, alpha)
            assert same(got, capi.binary(op, xc, y, alpha)), f"op{op} a{alpha} x^T"
            assert same(capi.binary(op, y, xt, alpha), capi.binary(op, y, xc, alpha)), f"op{op} a{alpha} y^T"
            if dtype == torch.float16:
                assert_ulp(got.cpu(), ew.binary(op, xt.cpu(), y.cpu(), alpha), 0, f"oracle op{op} a{alpha}")
    for op in (capi.SIGMOID, capi.SILU):
        assert same(capi.unary(op, xt), capi.unary(op, xc)), f"unary {op}"
    assert same(capi.binary_scalar(2, xt, 0.3), capi.binary_scalar(2, xc, 0.3)), "scalar"
    assert same(capi.silu_add(xt, y), capi.silu_add(xc, y)), "silu_add"
    acc = y.clone()
    capi.binary(0, acc, xt, 1.0, out=acc)
    assert same(acc, capi.binary(0, y, xc, 1.0)), "in place"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.int32, torch.bfloat16])
def test_transpose_copy(gpu, dtype):
    """Batched 2-D transposes take the tiled path: full and partial tiles,
    several tile rows and batches, aligned and misaligned rows, NCHW <-> NHWC
    permutes; bit-exact."""
    from thintnpu_amd import capi
    g = gen(5)
    raw = torch.randint(-2 ** 31, 2 ** 31 - 1, (3, 130, 1040), generator=g, dtype=torch.int64).to(torch.int32)
    base = raw.view(dtype) if dtype.itemsize == 4 else raw.view(torch.int16).view(dtype)[..., :1040]
    for shape in ((2, 64, 6400), (3, 128, 1024), (1, 130, 257), (3, 17, 1000), (1, 64, 64), (2, 100, 16)):
        b, m, n = shape
        x = base[:b, :m, :n]
        for offset in (0, 1):
            src = x[..., offset:]
            got = torch.empty(src.transpose(1, 2).shape, dtype=dtype, device=gpu)
            capi.copy(src.to(gpu).transpose(1, 2) if offset == 0 else x.to(gpu)[..., offset:].transpose(1, 2), got)
            assert torch.equal(got.cpu().view(torch.uint8), src.transpose(1, 2).contiguous().view(torch.uint8))
    x = torch.randn(2, 64, 20, 20, generator=g).to(dtype) if dtype.is_floating_point else \
        torch.randint(-1000, 1000, (2, 64, 20, 20), generator=g).to(dtype)
    for perm in ((0, 2, 3, 1), (0, 3, 1, 2)):
        src = x.permute(*perm)
        got = torch.empty(src.shape, dtype=dtype, device=gpu)
        capi.copy(x.to(gpu).permute(*perm), got)
        assert torch.equal(got.cpu().view(torch.uint8), src.contiguous().view(torch.uint8))


def test_beyond_32bit_extents(gpu):
    """Operands past 2^31 elements (4 GiB of fp16) run as several launches over
    slabs whose offsets fit 32 bits: a contiguous 1-D add across the slab
    boundaries, and a column slice of a [33000, 65536] tensor whose span passes
    2^31.  Small integers keep every result exact, so torch's own device ops are
    an exact reference at this size."""
    from thintnpu_amd import capi
    n = (1 << 31) + 4096 + 8
    x = (torch.arange(n, device=gpu, dtype=torch.int32) % 2039).to(torch.float16)
    y = torch.full((1,), 3.0, dtype=torch.float16, device=gpu)
    got = capi.binary(capi.ADD, x, y, alpha=2.0)
    assert torch.equal(got, x + 6)
    del got, x
    torch.cuda.empty_cache()
    rows, cols = 33000, 65536
    base = (torch.arange(rows * cols, device=gpu, dtype=torch.int32) % 1021).to(torch.float16).view(rows, cols)
    view = base[:, 16:]
    assert torch.equal(capi.binary_scalar(capi.MUL, view, 2.0), view * 2)
    del base, view
    torch.cuda.empty_cache()
