"""Detect-head decode (whole_blocked.py:118-146) on the GPU.

The fused kernel must equal, bit for bit, the composition of entries pinned
elsewhere: thin_dfl_expect (fp16 distances) -> the oracle's fp16 box steps ->
and thin_unary SIGMOID for the scores.  Against the full CPU oracle the boxes
differ only through the DFL expectation's 1e-3 relative bar, carried through
the box steps with one fp16 rounding per step (box_bound)."""
import pytest
import torch

from oracle import detect as dt
from oracle import elementwise as ew
from oracle import reductions as rd
from oracle.numerics import assert_ulp, bits_equal, ulp16_spacing
from tests.helpers import normal16

pytestmark = pytest.mark.gpu

YOLO = ([(80, 80), (40, 40), (20, 20)], [8.0, 16.0, 32.0])
ODD = ([(3, 5), (2, 3)], [8.0, 16.0])


def inputs(b, nc, shapes, seed):
    a = sum(h * w for h, w in shapes)
    return normal16((b, 64, a), seed, std=3.0), normal16((b, nc, a), seed + 1, mean=-4.0, std=2.0)


def composed(capi, gpu, boxes, scores, shapes, strides, xywh):
    distance = capi.dfl_expect(boxes.to(gpu)).cpu()
    return torch.cat((dt.box_decode(distance, shapes, strides, xywh),
                      capi.unary(capi.SIGMOID, scores.to(gpu)).cpu()), 1)


@pytest.mark.parametrize("xywh", [False, True])
@pytest.mark.parametrize("case", ["yolo", "odd"])
def test_decode_equals_composition(gpu, xywh, case):
    from thintnpu_amd import capi
    shapes, strides = YOLO if case == "yolo" else ODD
    boxes, scores = inputs(2, 80 if case == "yolo" else 3, shapes, 7)
    got = capi.detect_decode(boxes.to(gpu), scores.to(gpu), shapes, strides, xywh).cpu()
    want = composed(capi, gpu, boxes, scores, shapes, strides, xywh)
    assert bits_equal(got, want)
    ref = dt.detect_decode(boxes, scores, shapes, strides, xywh)
    assert_ulp(got[:, 4:], ref[:, 4:], 2, "scores")
    distance = capi.dfl_expect(boxes.to(gpu)).cpu()
    bound = box_bound(distance, rd.dfl_expect(boxes, torch.float16), shapes, strides, xywh)
    assert ((got[:, :4].double() - ref[:, :4].double()).abs() <= bound * (1 + 1e-9)).all()


def box_bound(d_dev, d_ref, shapes, strides, xywh):
    """Largest |device box - oracle box| the contracts allow.  The two
    distances differ by at most the DFL bar (1e-3 of |d|, floored at 2^-14);
    each fp16 box step of either path adds at most half an ulp of its
    result; the stride multiply is exact (a power of two).  In units of the
    output (pixels)."""
    anchors, scale = dt.grid(shapes, strides)
    a, st = anchors.double().unsqueeze(0), scale.double().unsqueeze(0)
    e = 1e-3 * d_ref.double().abs().clamp_min(2.0 ** -14)
    h = lambda t: 0.5 * ulp16_spacing(t)  # noqa: E731  (half an ulp at |t|)
    lo = [a - d[:, :2].double() for d in (d_dev, d_ref)]
    up = [a + d[:, 2:].double() for d in (d_dev, d_ref)]
    r_lo = h(lo[0]) + h(lo[1])       # the rounding of each path's lower and upper
    r_up = h(up[0]) + h(up[1])
    if not xywh:
        return torch.cat((e[:, :2] + r_lo, e[:, 2:] + r_up), 1) * st
    c = [(l_ + u_) / 2 for l_, u_ in zip(lo, up)]
    w = [u_ - l_ for l_, u_ in zip(lo, up)]
    bc = (e[:, :2] + e[:, 2:]) / 2 + (r_lo + r_up) / 2 + h(c[0]) + h(c[1])
    bw = e[:, :2] + e[:, 2:] + r_lo + r_up + h(w[0]) + h(w[1])
    return torch.cat((bc, bw), 1) * st


def test_decode_views_and_specials(gpu):
    from thintnpu_amd import capi
    shapes, strides = YOLO
    a = 8400
    head = torch.cat(inputs(2, 80, shapes, 11), 1)        # [2, 144, A]: boxes then scores
    head[0, 5, 17] = float("nan")
    head[1, 20, 33] = float("inf")
    head[1, 40:56, 100] = float("-inf")
    head[0, 64 + 3, 9] = float("nan")
    head[1, 64 + 7, 10] = float("-inf")
    hd = head.to(gpu)
    parent = torch.zeros((2, 84, a + 8), dtype=torch.float16, device=gpu)
    capi.detect_decode(hd[:, :64], hd[:, 64:], shapes, strides, False, out=parent[..., :a])
    got = parent.cpu()
    want = composed(capi, gpu, head[:, :64].contiguous(), head[:, 64:].contiguous(), shapes, strides, False)
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got[..., :a]), nan)
    assert bits_equal(got[..., :a][~nan], want[~nan])
    assert not got[..., a:].any()


def test_decode_npu_to_selection(gpu):
    """thin_fused.detect_decode -> thin_native_flow.detection_select on the
    production transposed view, eager == captured replay, bit-exact vs oracle."""
    import thin_backend
    from thin_backend.graph import CapturedForward
    from oracle import selection as sel
    thin_backend.load_flow_libraries()
    npu = torch.device("npu:0")
    shapes, strides = YOLO
    boxes, scores = inputs(1, 80, shapes, 21)
    with torch.inference_mode():
        b, s = boxes.to(npu), scores.to(npu)

        def forward(_=None):
            decoded = torch.ops.thin_fused.detect_decode(b, s, [v for hw in shapes for v in hw], strides, False)
            return torch.ops.thin_native_flow.detection_select(decoded.transpose(1, 2), 300, False)
        eager = forward().cpu()
        decoded = torch.ops.thin_fused.detect_decode(b, s, [v for hw in shapes for v in hw], strides, False).cpu()
        assert bits_equal(eager, sel.select(decoded.transpose(1, 2), 300, False)["output"])
        graph = CapturedForward(forward, b)
        for _ in range(3):
            assert bits_equal(graph.replay().cpu(), eager)
        graph.close()


def test_offsets_beyond_4gib(gpu):
    """Logits whose byte offsets pass 4 GiB take the 64-bit pointer loads; they
    give the same bits as the 32-bit buffer-resource loads on a compact copy
    (DFL and decode)."""
    from thintnpu_amd import capi
    a = 8400
    shapes, strides = [(80, 80), (40, 40), (20, 20)], [8.0, 16.0, 32.0]
    batch_stride = (1 << 31) + 64 * a  # elements: image 1 starts 4 GiB + 1 MB past image 0
    storage = torch.empty(batch_stride + 64 * a, dtype=torch.float16, device=gpu)
    far = storage.as_strided((2, 64, a), (batch_stride, a, 1))
    near = (normal16((2, 64, a), 61) * 3).to(gpu)
    far.copy_(near)
    scores = normal16((2, 80, a), 62).to(gpu)
    try:
        for out_dtype in (torch.float16, torch.float32):
            assert bits_equal(capi.dfl_expect(far, out_dtype).cpu(), capi.dfl_expect(near, out_dtype).cpu())
        assert bits_equal(capi.detect_decode(far, scores, shapes, strides).cpu(),
                          capi.detect_decode(near, scores, shapes, strides).cpu())
    finally:
        del far, storage
        torch.cuda.empty_cache()


@pytest.mark.parametrize("xywh", [False, True])
def test_decode_direct_distances(gpu, xywh):
    """reg_max = 1 heads (YOLO26, whose module.dfl is the identity:
    whole_blocked.py:135; YOLO26.md:30-38): boxes [B,4,A] are the distances.
    Boxes bit-exact against the oracle's fp16 steps, scores within 2 ulp; the
    two-anchor and the single-anchor (unaligned view) forms."""
    from thintnpu_amd import capi
    from tests.helpers import gen
    shapes, strides = YOLO
    a = 8400
    dist = (torch.rand(2, 4, a, generator=gen(31)) * 20).half()
    dist[0, 1, 5] = float("nan")
    dist[1, 2, 9] = float("inf")
    scores = normal16((2, 80, a), 32, mean=-4.0, std=2.0)
    got = capi.detect_decode(dist.to(gpu), scores.to(gpu), shapes, strides, xywh).cpu()
    ref = dt.detect_decode(dist, scores, shapes, strides, xywh)
    nan = torch.isnan(ref[:, :4])
    assert torch.equal(torch.isnan(got[:, :4]), nan)
    assert bits_equal(got[:, :4][~nan], ref[:, :4][~nan])
    assert_ulp(got[:, 4:], ref[:, 4:], 2, "scores")
    # distances read through an unaligned strided view (single-anchor path)
    parent = torch.zeros((2, 6, a + 1), dtype=torch.float16)
    parent[:, 1:5, 1:] = dist
    view = parent.to(gpu)[:, 1:5, 1:]
    got = capi.detect_decode(view, scores.to(gpu), shapes, strides, xywh).cpu()
    assert torch.equal(torch.isnan(got[:, :4]), nan)
    assert bits_equal(got[:, :4][~nan], ref[:, :4][~nan])
    # the dispatcher op takes the same [B,4,A] boxes
    import thin_backend
    thin_backend.load_flow_libraries()
    with torch.inference_mode():
        flat = [v for hw in shapes for v in hw]
        npu = torch.ops.thin_fused.detect_decode(dist.to("npu"), scores.to("npu"), flat, strides, xywh).cpu()
    assert bits_equal(npu, capi.detect_decode(dist.to(gpu), scores.to(gpu), shapes, strides, xywh).cpu())
