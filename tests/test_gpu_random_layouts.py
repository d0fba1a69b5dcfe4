"""Seeded random layouts through the C ABI: permuted, sliced, stepped and
broadcast views of fp16 / fp32 tensors, non-contiguous outputs, and the
binary and unary ops, strided copy, concatenation and softmax on them, each
against the oracle.
The fixed shapes of the other tests pin the paths the model takes; these
exercise the dimension coalescing and kernel selection on layouts that no
fixed case names."""
import random

import pytest
import torch

from oracle import elementwise as ew
from oracle import movement as mv
from oracle.numerics import assert_ulp
from tests.helpers import gen

pytestmark = pytest.mark.gpu

SIZES = [1, 2, 3, 5, 7, 8, 9, 16, 17, 33]
BITS = {torch.float16: torch.int16, torch.float32: torch.int32}


def random_view(rng, shape, dtype, dev, seed, positive=False):
    """A view of `shape` over a larger buffer: a stepped, offset slice per
    dim, with the dims permuted in memory -- so element order in memory is
    unrelated to the logical order.  Returns the same view on the host and
    on `dev`."""
    rank = len(shape)
    perm = list(range(rank))
    rng.shuffle(perm)
    steps = [rng.choice((1, 1, 2)) for _ in range(rank)]
    offs = [rng.choice((0, 0, 1)) for _ in range(rank)]
    buf_shape = [shape[p] * steps[p] + offs[p] for p in perm]
    buf = torch.randn(buf_shape, generator=gen(seed))
    if positive:
        buf = buf.abs() + 0.5
    buf = buf.to(dtype)
    index = tuple(slice(offs[p], offs[p] + shape[p] * steps[p], steps[p]) for p in perm)
    inv = [perm.index(d) for d in range(rank)]
    host = buf[index].permute(inv)
    device = buf.to(dev)[index].permute(inv)
    assert tuple(host.shape) == tuple(shape)
    return host, device


def broadcastable(rng, shape):
    """shape with some dims set to 1, or a suffix of it (broadcast operands)."""
    s = [1 if rng.random() < 0.3 else d for d in shape]
    if len(s) > 1 and rng.random() < 0.25:
        s = s[rng.randrange(1, len(s)):]
    return s


def check(got, expect, what):
    if expect.dtype == torch.float16:
        assert_ulp(got, expect, 0, what)
    else:  # fp32 add/sub with alpha: one fma on the GPU, mul then add in the oracle
        torch.testing.assert_close(got, expect, rtol=1e-5, atol=1e-6, equal_nan=True, msg=what)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_binary_random_views(gpu, dtype):
    from thintnpu_amd import capi
    rng = random.Random(20261202 + (dtype == torch.float32))
    for case in range(60):
        shape = [rng.choice(SIZES) for _ in range(rng.randint(1, 5))]
        xs, ys = shape, broadcastable(rng, shape)
        if rng.random() < 0.5:
            xs, ys = ys, xs
        xc, xg = random_view(rng, xs, dtype, gpu, 3 * case + 1)
        yc, yg = random_view(rng, ys, dtype, gpu, 3 * case + 2, positive=True)  # away from 0 for div
        full = list(torch.broadcast_shapes(xc.shape, yc.shape))
        out_view = rng.random() < 0.5
        for op in (0, 1, 2, 3):
            alpha = rng.choice((1.0, 1.0, 0.3, 2.0)) if op in (0, 1) else 1.0
            what = (f"case {case} op{op} a{alpha} x{list(xc.shape)}/{list(xc.stride())} "
                    f"y{list(yc.shape)}/{list(yc.stride())} out_view={out_view}")
            if out_view:
                _, outg = random_view(rng, full, dtype, gpu, 3 * case + 3)
                capi.binary(op, xg, yg, alpha, out=outg)
                got = outg.cpu()
            else:
                got = capi.binary(op, xg, yg, alpha).cpu()
            check(got, ew.binary(op, xc, yc, alpha), what)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_copy_random_views(gpu, dtype):
    """thin_copy between two random views of one shape moves the bits."""
    from thintnpu_amd import capi
    rng = random.Random(77 + (dtype == torch.float32))
    for case in range(60):
        shape = [rng.choice(SIZES) for _ in range(rng.randint(1, 5))]
        src_c, src_g = random_view(rng, shape, dtype, gpu, 2 * case + 100)
        _, dst_g = random_view(rng, shape, dtype, gpu, 2 * case + 101)
        capi.copy(src_g, dst_g)
        got = dst_g.cpu().contiguous().view(BITS[dtype])
        assert torch.equal(got, src_c.contiguous().view(BITS[dtype])), f"case {case} {shape}"


def test_cat_random_views(gpu):
    """thin_cat of 1-6 random views (empty ones among them) along a random dim."""
    from thintnpu_amd import capi
    rng = random.Random(555)
    for case in range(50):
        rank = rng.randint(1, 5)
        shape = [rng.choice(SIZES) for _ in range(rank)]
        dim = rng.randrange(rank)
        host, devs = [], []
        for k in range(rng.randint(1, 6)):
            s = list(shape)
            s[dim] = rng.choice([0, 1, 2, 3, 5, 16, 17]) if k else s[dim]
            if s[dim] == 0:
                c, g = torch.empty(s, dtype=torch.float16), torch.empty(s, dtype=torch.float16, device=gpu)
            else:
                c, g = random_view(rng, s, torch.float16, gpu, 10 * case + k)
            host.append(c)
            devs.append(g)
        got = capi.cat(devs, dim).cpu()
        expect = mv.cat(host, dim)
        what = f"case {case} dim {dim} {[list(t.shape) for t in host]}"
        assert got.shape == expect.shape, what
        assert torch.equal(got.view(torch.int16), expect.view(torch.int16)), what


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_unary_random_views(gpu, dtype):
    """sigmoid and SiLU of random views, into fresh and into random-view outputs."""
    from thintnpu_amd import capi
    rng = random.Random(909 + (dtype == torch.float32))
    for case in range(40):
        shape = [rng.choice(SIZES) for _ in range(rng.randint(1, 5))]
        xc, xg = random_view(rng, shape, dtype, gpu, 4 * case + 7)
        for op, ref in ((capi.SIGMOID, ew.sigmoid), (capi.SILU, ew.silu)):
            what = f"case {case} op{op} {shape}/{list(xc.stride())}"
            if rng.random() < 0.5:
                _, outg = random_view(rng, shape, dtype, gpu, 4 * case + 8)
                capi.unary(op, xg, out=outg)
                got = outg.cpu()
            else:
                got = capi.unary(op, xg).cpu()
            if dtype == torch.float16:
                assert_ulp(got, ref(xc), 2, what)
            else:
                torch.testing.assert_close(got, ref(xc), rtol=1e-5, atol=1e-6, msg=what)


@pytest.mark.parametrize("half_to_float", [False, True])
def test_softmax_random_views(gpu, half_to_float):
    """fp16 softmax over a random dim of a random view (row, column, short
    column and stream forms alike), to the bars of the softmax tests."""
    from tests.test_gpu_softmax import check_softmax
    from thintnpu_amd import capi
    rng = random.Random(31337 + half_to_float)
    sizes = SIZES + [64, 400, 2048]
    for case in range(40):
        rank = rng.randint(1, 4)
        shape = [rng.choice(sizes if rng.random() < 0.3 else SIZES) for _ in range(rank)]
        while torch.Size(shape).numel() > (1 << 20):
            shape[rng.randrange(rank)] = rng.choice(SIZES)
        dim = rng.randrange(rank)
        xc, xg = random_view(rng, shape, torch.float16, gpu, 5 * case + 11)
        got = capi.softmax(xg, dim, half_to_float).cpu()
        check_softmax(got, xc, dim, half_to_float, f"case {case} dim {dim} {shape}/{list(xc.stride())}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_channels_last_views(gpu, dtype):
    """Operands and outputs that are NCHW views of NHWC memory (the dims go
    in the output's stride order before coalescing), with a per-channel
    operand and a contiguous operand among them, against the oracle."""
    from thintnpu_amd import capi
    n, c, h, w = 2, 48, 9, 13
    cl = lambda seed: torch.randn(n, h, w, c, generator=gen(seed)).to(dtype)  # noqa: E731
    xh, yh = cl(1).permute(0, 3, 1, 2), (cl(2).abs() + 0.5).permute(0, 3, 1, 2)
    bias = torch.randn(1, c, 1, 1, generator=gen(3)).to(dtype)
    dense = torch.randn(n, c, h, w, generator=gen(4)).to(dtype)
    xg, yg, bg, dg = (t.to(gpu) for t in (xh, yh, bias, dense))
    for op in range(4):
        for (a, b), (ag, bg2) in (((xh, yh), (xg, yg)), ((xh, bias), (xg, bg)), ((dense, xh), (dg, xg))):
            out = torch.empty(n, h, w, c, dtype=dtype, device=gpu).permute(0, 3, 1, 2)
            capi.binary(op, ag, bg2, 1.0, out=out)
            check(out.cpu(), ew.binary(op, a, b, 1.0), f"op{op} {list(a.stride())} {list(b.stride())}")
    for op, ref in ((capi.SIGMOID, ew.sigmoid), (capi.SILU, ew.silu)):
        out = torch.empty(n, h, w, c, dtype=dtype, device=gpu).permute(0, 3, 1, 2)
        capi.unary(op, xg, out=out)
        if dtype == torch.float16:
            assert_ulp(out.cpu(), ref(xh), 2, f"unary {op}")
        else:
            torch.testing.assert_close(out.cpu(), ref(xh), rtol=1e-5, atol=1e-6)
