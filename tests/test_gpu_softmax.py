"""GPU parity of softmax / DFL (through the C ABI).

Bars: fp16 outputs <= 1e-3 relative (floor 2^-14) against the single-rounded
fp32 softmax and <= 1e-3 absolute against PyTorch CPU's fp16 op (the reference
test's tolerance); fp32 outputs <= 1e-5 absolute; NaN / +inf / -inf masks equal
to CPU exactly."""
import pytest
import torch

from oracle import elementwise as ew
from oracle import reductions as rd
from oracle.numerics import assert_rel, assert_ulp
from tests.helpers import gen, normal16

pytestmark = pytest.mark.gpu


def check_softmax(got, x, dim, half_to_float=False, what=""):
    cpu = rd.softmax(x, dim, half_to_float)
    assert got.dtype == cpu.dtype and got.shape == cpu.shape, what
    assert torch.equal(torch.isnan(got), torch.isnan(cpu)), f"{what}: NaN mask"
    assert torch.equal(torch.isposinf(got), torch.isposinf(cpu)), f"{what}: +inf mask"
    assert torch.equal(torch.isneginf(got), torch.isneginf(cpu)), f"{what}: -inf mask"
    fin = torch.isfinite(cpu)
    if not bool(fin.any()):
        return
    if got.dtype == torch.float16:
        assert_rel(got, rd.softmax_rounded(x, dim), 1e-3, what)
        err = (got.float()[fin] - cpu.float()[fin]).abs().max().item()
        assert err <= 1e-3, f"{what}: abs {err}"
    else:
        err = (got[fin] - cpu[fin]).abs().max().item()
        assert err <= 1e-5, f"{what}: abs {err}"


def run(capi, xd, dim, half_to_float=False):
    return capi.softmax(xd, dim, half_to_float).cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_softmax_reference_cases(gpu, dtype):
    """verify_softmax.py:74-136 restated."""
    from thintnpu_amd import capi
    g = gen(2718)
    for shape, dims in (
        ((), (0, -1)), ((0,), (0,)), ((2, 0, 3), (0, 1, 2)),
        ((1,), (0,)), ((3,), (0,)), ((7,), (-1,)), ((100,), (0,)),
        ((3, 16), (-1, 0)), ((5, 1000), (1,)),
        ((2, 2049), (1,)), ((2, 4097), (-1,)), ((2, 65537), (-1,)),
        ((2, 3, 7), (0, 1, 2, -2)), ((2, 16, 17), (1,)),
        ((2, 1000, 17), (1,)), ((3, 7, 1), (1,)),
        ((1, 4, 16, 8400), (1, 2)), ((1, 16, 4, 8400), (1,)),
        ((2, 4, 16, 2100), (2,)),
        # every lanes-per-row bucket of the row kernel (fp16 / fp32 16-byte chunks)
        ((9, 24), (1,)), ((3, 64), (1,)), ((5, 200), (1,)), ((3, 4000), (1,)), ((2, 2000), (1,)),
        ((7, 512), (1,)), ((3, 1024), (1,)),
    ):
        x = (torch.randn(shape, generator=g) * 3).to(dtype)
        xd = x.to(gpu)
        for dim in dims:
            d = dim % max(1, x.dim())
            check_softmax(run(capi, xd, d), x, d, what=f"random {shape} {dim}")
    for shape, dim in (((3, 1000), 1), ((2, 16, 37), 1), ((2, 1000, 17), 1)):
        for shift in (-10000, 10000):
            x = (torch.randn(shape, generator=g) * 10 + shift).to(dtype)
            check_softmax(run(capi, x.to(gpu), dim), x, dim, what=f"shift {shift}")
        x = torch.zeros(shape, dtype=dtype)
        check_softmax(run(capi, x.to(gpu), dim), x, dim, what="uniform")
    x = torch.randn(2, 3, 7, generator=g).to(dtype)
    xd = x.to(gpu)
    for dim in (0, 1, 2):
        check_softmax(run(capi, xd.transpose(0, 2), dim), x.transpose(0, 2), dim, what="transpose")
    check_softmax(run(capi, xd.as_strided((2, 3, 5), (21, 7, 1), 1), 2), x[:, :, 1:6], 2, what="offset")
    check_softmax(run(capi, xd.as_strided((2, 3, 5), (21, 7, 1), 1), 1), x[:, :, 1:6], 1, what="offset inner")
    check_softmax(run(capi, xd.unsqueeze(0).expand(4, -1, -1, -1), 0), x.unsqueeze(0).expand(4, -1, -1, -1), 0,
                  what="expanded")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_softmax_nonfinite(gpu, dtype):
    from thintnpu_amd import capi
    for values in ([float("-inf"), 0, 1], [float("-inf")] * 3, [0, float("inf"), 1], [0, float("nan"), 1]):
        a = torch.tensor(values, dtype=dtype)
        for shape, dim in (((1, 3), 1), ((3, 1), 0), ((3, 17), 0)):
            x = a.reshape((1, 3) if dim else (3, 1)).expand(shape).contiguous()
            check_softmax(run(capi, x.to(gpu), dim), x, dim, what=f"nonfinite {values} {shape}")
    x = torch.tensor([[0, 0, float("-inf"), 0, 0],
                      [1, float("nan"), float("-inf"), float("inf"), float("-inf")],
                      [2, 2, float("-inf"), 1, 3]], dtype=dtype)
    check_softmax(run(capi, x.to(gpu), 0), x, 0, what="mixed inner")
    xt = x.t().contiguous()
    check_softmax(run(capi, xt.to(gpu), 1), xt, 1, what="mixed last")


def test_softmax_half_to_float(gpu):
    from thintnpu_amd import capi
    for shape, dim in (((3, 1000), 1), ((2, 16, 17), 1), ((2, 400), 1)):
        x = normal16(shape, 5)
        check_softmax(run(capi, x.to(gpu), dim, True), x, dim, True, what=f"half_to_float {shape}")


@pytest.mark.parametrize("n", [1, 32])
def test_attention_softmax_c5(gpu, n):
    """C5: row softmax over fp16 scores [N,4,400,400] ~ N(0,2)."""
    from thintnpu_amd import capi
    x = normal16((n, 4, 400, 400), 5, std=2.0)
    check_softmax(run(capi, x.to(gpu), 3), x, 3, what=f"attention n={n}")


def dfl_views():
    return {
        "transpose": lambda t: t.transpose(1, 2),
        "contiguous": None,
    }


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_dfl_softmax_views(gpu, dtype):
    """verify_dfl_softmax.py:54-92: softmax over the 16 bins of [B,16,4,A] views."""
    from thintnpu_amd import capi
    g = gen(1928)

    def check(label, base, view, half_to_float=False):
        got = capi.softmax(view(base.to(gpu)), 1, half_to_float).cpu()
        check_softmax(got, view(base), 1, half_to_float, what=label)

    for width in (16, 80, 1040, 8400):
        cpu = (torch.randn(2, 4, 16, width, generator=g) * 3).to(dtype)
        check(f"{width}-transpose", cpu, lambda x: x.transpose(1, 2))
        check(f"{width}-contiguous", cpu, lambda x, w=width: x.reshape(2, 16, 4, w))
        if dtype == torch.float16:
            check(f"{width}-h2f", cpu, lambda x: x.transpose(1, 2), True)
    cpu = torch.randn(2, 4, 16, 1120, generator=g).to(dtype)
    check("offset", cpu, lambda x: x[:, :, :, 16:1056].transpose(1, 2))
    cpu = torch.randn(1, 4, 16, 80, generator=g).to(dtype)
    check("broadcast", cpu, lambda x: x.expand(2, -1, -1, -1).transpose(1, 2))
    cpu = torch.randn(1, 4, 16, 17, generator=g).to(dtype)
    check("unaligned", cpu, lambda x: x.transpose(1, 2))
    cpu = torch.randn(1, 4, 16, 80, generator=g).to(dtype)
    for mode in ("nan", "positive-inf", "negative-inf", "zeros", "large-shift"):
        special = cpu.clone()
        if mode == "nan":
            special[:, :, 5, 3] = float("nan")
        elif mode == "positive-inf":
            special[:, :, 5, 3] = float("inf")
        elif mode == "negative-inf":
            special[:, :, :, 3] = -float("inf")
        elif mode == "zeros":
            special.zero_()
            special[:, :, 4, :] = -0.0
        else:
            special.add_(10000)
        check(mode, special, lambda x: x.transpose(1, 2))


@pytest.mark.parametrize("n", [1, 32])
def test_dfl_expect_c4(gpu, n):
    """C4: fp16 logits [N,64,8400] ~ N(0,3) -> expectation [N,4,8400]."""
    from thintnpu_amd import capi
    x = normal16((n, 64, 8400), 4, std=3.0)
    xd = x.to(gpu)
    got = capi.dfl_expect(xd).cpu()
    ref = rd.dfl_expect(x, torch.float32)
    assert_rel(got, ref, 1e-3, f"dfl n={n}")
    got32 = capi.dfl_expect(xd, torch.float32).cpu()
    assert (got32 - ref).abs().max().item() <= 1e-5
    assert float(got32.min()) >= 0 and float(got32.max()) <= 15


def test_dfl_expect_views_and_specials(gpu):
    from thintnpu_amd import capi
    x = normal16((2, 8400, 64), 6, std=3.0)
    v = x.transpose(1, 2)  # [2,64,8400] with anchor stride 64
    got = capi.dfl_expect(x.to(gpu).transpose(1, 2)).cpu()
    assert_rel(got, rd.dfl_expect(v, torch.float32), 1e-3, "dfl transposed")
    for width in (17, 18, 20, 24, 64):  # one-, two-, four- and eight-anchor thread forms
        y = normal16((2, 64, width), 7 + width, std=3.0)
        y[0, 3, 2] = float("nan")
        y[0, 20, 5] = float("inf")
        y[0, 20, 4] = float("inf")
        y[0, 32:48, 7] = float("-inf")
        y[0, 48:64, 9] = 0
        y[1, 0:16, 10] = y[1, 0:16, 10] + 10000      # large shift
        y[1, 16:32, 11] = y[1, 16:32, 11] - 10000
        y[1, 32, 12], y[1, 47, 12] = 65504.0, -65504.0  # fp16 extremes in one side
        y[1, 48:64, 13] = float("-inf")
        y[1, 50, 13] = 1.0                            # one finite bin: expectation 2
        # the same values anchor-major (each anchor's 64 bins contiguous)
        ya = y.transpose(1, 2).contiguous().transpose(1, 2)
        for out_dtype in (torch.float16, torch.float32):
            got = capi.dfl_expect(y.to(gpu), out_dtype).cpu()
            assert_rel(got, rd.dfl_expect(y, out_dtype), 1e-3, f"dfl specials {width} {out_dtype}")
            got = capi.dfl_expect(ya.to(gpu).transpose(1, 2).contiguous().transpose(1, 2), out_dtype).cpu()
            assert_rel(got, rd.dfl_expect(ya, out_dtype), 1e-3, f"dfl anchor-major specials {width} {out_dtype}")
        assert float(capi.dfl_expect(y.to(gpu)).cpu()[1, 3, 13]) == 2.0
        assert float(capi.dfl_expect(y.to(gpu).transpose(1, 2).contiguous().transpose(1, 2)).cpu()[1, 3, 13]) == 2.0


@pytest.mark.parametrize("n", [1, 32])
def test_class_sigmoid_c4(gpu, n):
    """C4: sigmoid of class logits [N,80,8400] ~ N(-4,2), <= 2 ulp."""
    from thintnpu_amd import capi
    x = normal16((n, 80, 8400), 14, mean=-4.0, std=2.0)
    assert_ulp(capi.unary(capi.SIGMOID, x.to(gpu)).cpu(), ew.sigmoid(x), 2, f"sigmoid n={n}")


def test_softmax_row_widths(gpu):
    """fp16 rows whose 16-byte chunk count is not a power of two (idle lanes
    in the last chunk round), row counts that leave a partial last block, and
    rows with NaN, +inf, all -inf, -inf mixed in and large shifts."""
    from thintnpu_amd import capi
    for rows, width in ((100, 400), (7, 120), (33, 2040), (41, 136)):
        x = normal16((rows, width), rows + width, std=3.0)
        x[0, 5] = float("nan")
        x[1, 7] = float("inf")
        x[2] = float("-inf")
        x[3, ::3] = float("-inf")
        x[4] += 10000
        x[5] -= 10000
        check_softmax(run(capi, x.to(gpu), 1), x, 1, what=f"tiles {rows}x{width}")


@pytest.mark.parametrize("half_to_float", [False, True])
def test_softmax_long_columns(gpu, half_to_float):
    """Reductions of more than 16 (vector units) or 32 (single columns) rows
    over a non-innermost dim: few units, whose rows split over the slices of
    a block (16-byte units, and unaligned single columns with a partial last
    block of units), and enough units for one thread per unit; NaN, +inf, an
    all -inf column and a large shift among them; long rows of both kinds."""
    from thintnpu_amd import capi
    for shape in ((8, 400, 400), (3, 100, 37), (2, 33, 24), (1, 24, 524288)):
        x = normal16(shape, sum(shape) + half_to_float, std=3.0)
        x[0, 3, 5] = float("nan")
        x[0, 7, 6] = float("inf")
        x[-1, :, 1] = float("-inf")
        x[-1, 2, 2] += 10000
        check_softmax(run(capi, x.to(gpu), 1, half_to_float), x, 1, half_to_float, what=f"long columns {shape}")
    for width in (8400, 8401):
        x = normal16((5, width), width, std=3.0)
        x[1, 77] = float("nan")
        x[2] = float("-inf")
        check_softmax(run(capi, x.to(gpu), 1, half_to_float), x, 1, half_to_float, what=f"long rows {width}")


def test_softmax_short_columns(gpu):
    """Reductions of <= 16 rows whose columns run contiguous in the innermost
    dim (the DFL bin softmax layout), staged through LDS tiles: reductions
    shorter than 16, a partial last tile of innermost columns (136 = 128 + 8),
    outer column counts that leave a partial group, NaN / +inf / all -inf
    columns, and the transposed DFL view itself."""
    from thintnpu_amd import capi
    for shape in ((3, 5, 3, 136), (2, 16, 4, 64), (1, 1, 2, 8), (2, 9, 1, 256)):
        x = normal16(shape, sum(shape), std=3.0)
        x[0, 0, 0, 3] = float("nan")
        x[0, :, 0, 5] = float("-inf")
        x[-1, -1, -1, 7] = float("inf")
        x[0, 0, -1, 1] += 10000
        check_softmax(run(capi, x.to(gpu), 1), x, 1, what=f"short columns {shape}")
    a = 8400
    logits = normal16((2, 64, a), 3, std=3.0)
    logits[0, 17, 9] = float("nan")
    logits[1, 32:48, 100] = float("-inf")
    view = logits.view(2, 4, 16, a).transpose(1, 2)
    got = capi.softmax(logits.to(gpu).view(2, 4, 16, a).transpose(1, 2), 1).cpu()
    check_softmax(got, view, 1, what="DFL bin view")


@pytest.mark.parametrize("half_to_float", [False, True])
def test_dfl_softmax_eight_and_two_column_forms_agree(gpu, half_to_float):
    """The DFL bin view runs eight columns per thread when every row is
    16-byte aligned and two when only 4-byte aligned; both evaluate the same
    expressions in the same order, so their outputs are bit-identical."""
    from oracle.numerics import bits_equal
    from thintnpu_amd import capi
    a = 8400
    logits = normal16((2, 64, a + 2), 19, std=3.0)
    logits[0, 17, 9] = float("nan")
    logits[1, 32:48, 100] = float("-inf")
    logits[1, 5, 200] = float("inf")
    d = logits.to(gpu)
    two = capi.softmax(d[..., 2:].view(2, 4, 16, a).transpose(1, 2), 1, half_to_float).cpu()  # 4-byte aligned rows
    eight = capi.softmax(d[..., 2:].contiguous().view(2, 4, 16, a).transpose(1, 2), 1, half_to_float).cpu()
    nan = torch.isnan(two)
    assert torch.equal(torch.isnan(eight), nan)  # NaN payloads may differ between the forms
    assert bits_equal(eight[~nan], two[~nan])
    check_softmax(eight, logits[..., 2:].reshape(2, 4, 16, a).transpose(1, 2), 1, half_to_float, what="eight-column")
