"""GPU parity of detection selection (through the C ABI): output and all seven
trace stages bit-exact against the stable CPU oracle on the reference's
fixture list (verify_selection_flow.py:160-213) and the C5 input."""
import pytest
import torch

from oracle import selection as sel
from oracle.numerics import bits_equal
from tests.selection_fixtures import backing_and_view, c5_selection_input, fixtures

pytestmark = pytest.mark.gpu

STAGES = {"class_max": "class_max", "stage1": "stage1_indices", "gathered": "gathered_scores",
          "top_values": "top_values", "stage2": "stage2_indices", "anchors": "anchor_indices",
          "labels": "labels"}


def run_case(gpu, x, max_det, agnostic, layout, name):
    from thintnpu_amd import capi
    base, view = backing_and_view(x, layout)
    v = view(base)
    ref = sel.select(v, max_det, agnostic)
    dv = view(base.to(gpu))
    out, tr = capi.detection_select(dv, max_det, agnostic, trace=True)
    assert bits_equal(out.cpu(), ref["output"]), f"{name}: output"
    for mine, theirs in STAGES.items():
        got = tr[mine].cpu()
        exp = ref[theirs]
        assert got.shape == exp.shape, (name, mine, got.shape, exp.shape)
        assert bits_equal(got, exp.to(got.dtype)), f"{name}: {mine}"
    plain = capi.detection_select(dv, max_det, agnostic)
    assert bits_equal(plain.cpu(), ref["output"]), f"{name}: production != trace"
    # every stage but the gathered scores (whose trace takes the full gather)
    partial = [n for n in STAGES if n != "gathered"]
    out2, tr2 = capi.detection_select(dv, max_det, agnostic, trace=partial)
    assert bits_equal(out2.cpu(), ref["output"]), f"{name}: output (partial trace)"
    for mine in partial:
        assert bits_equal(tr2[mine].cpu(), ref[STAGES[mine]].to(tr2[mine].dtype)), f"{name}: {mine} (partial trace)"
    return ref, v


@pytest.mark.parametrize("case", list(fixtures(full=True)), ids=lambda c: c[0])
def test_selection_fixtures(gpu, case):
    name, x, max_det, agnostic, layout, unique = case
    ref, v = run_case(gpu, x, max_det, agnostic, layout, name)
    if unique and ref["stage1_indices"].numel():
        scores = v[..., 4:].float()
        top = scores.max(-1).values.topk(ref["stage1_indices"].shape[1], dim=1).indices
        assert torch.equal(ref["stage1_indices"], top)


@pytest.mark.parametrize("layout", ["contiguous", "transposed"])
@pytest.mark.parametrize("agnostic", [False, True])
def test_selection_c5(gpu, layout, agnostic):
    """C5: top-300 of [1,8400,80] with ties and NaNs, in the contiguous
    [1,8400,84] layout and the production transposed view of [1,84,8400]."""
    x = c5_selection_input()
    run_case(gpu, x, 300, agnostic, layout, f"c5-{layout}-{agnostic}")


def test_selection_batched_and_workspace_errors(gpu):
    from thintnpu_amd import capi
    from tests.selection_fixtures import predictions
    x = predictions(4, 3360, 80, seed=77)
    run_case(gpu, x, 300, False, "transposed", "batched")
    d = x.to(gpu)
    out = torch.empty((4, 300, 6), dtype=torch.float32, device=gpu)
    ws = torch.empty(16, dtype=torch.uint8, device=gpu)
    st = capi.lib().thin_detection_select(capi.ctypes.byref(capi.desc(d)), 300, 0, out.data_ptr(),
                                          ws.data_ptr(), 16, None, torch.cuda.current_stream().cuda_stream)
    assert st == 4 and b"workspace" in capi.lib().thin_last_error()


def _pair_case(kind, seed):
    """Inputs that steer stage 2 through each of its forms: every stage-1
    anchor with a second class at its best score (more second pairs than one
    wave merges), a few anchors with four classes at the top (their rows
    prefetched, few extras), forty such anchors (many extras), and NaN and
    signed-zero second scores (bits the key does not fix)."""
    g = torch.Generator().manual_seed(seed)
    if kind == "second-pairs":
        a, nc = 2000, 10
        s = torch.rand(1, a, nc, generator=g) * 0.1
        v = 0.5 + 0.5 * torch.rand(1, a, generator=g)
        c = torch.stack([torch.randperm(nc, generator=g)[:2] for _ in range(a)])
        s[0, torch.arange(a)[:, None], c] = v[0][:, None]
    elif kind in ("row-extras", "many-row-extras"):
        a, nc = 3000, 20
        s = torch.rand(1, a, nc, generator=g) * 0.9
        n = 10 if kind == "row-extras" else 40
        rows = torch.randperm(a, generator=g)[:n]
        for r in rows.tolist():
            s[0, r, torch.randperm(nc, generator=g)[:4]] = 0.995
    else:  # "ambiguous-seconds"
        a, nc = 64, 6
        s = -torch.rand(1, a, nc, generator=g)
        for r in range(0, a, 4):
            s[0, r, 1] = float("nan")
            s[0, r, 4] = float("nan")
        for r in range(1, a, 4):
            s[0, r, 0] = -0.0
            s[0, r, 3] = 0.0
        for r in range(2, a, 4):
            s[0, r, 2] = 0.0
            s[0, r, 5] = -0.0
    sh = s.half()
    if kind == "ambiguous-seconds":  # NaN payloads differ
        bits = sh.view(torch.int16)
        bits[0, 0::4, 1] = 0x7E01
        bits[0, 0::4, 4] = -0x0200  # 0xFE00
    boxes = torch.randn(1, a, 4, generator=g).half()
    return torch.cat((boxes, sh), -1)


@pytest.mark.parametrize("layout", ["transposed", "contiguous"])
@pytest.mark.parametrize("kind,max_det", [("second-pairs", 300), ("row-extras", 300), ("many-row-extras", 300),
                                          ("ambiguous-seconds", 64)])
def test_selection_pair_paths(gpu, kind, max_det, layout):
    x = _pair_case(kind, 31)
    run_case(gpu, x, max_det, False, layout, f"{kind}-{layout}")


@pytest.mark.parametrize("layout", ["transposed", "contiguous", "strided"])
@pytest.mark.parametrize("agnostic,max_det", [(False, 300), (True, 300), (False, 1024)])
def test_selection_every_encoding_two_launch(gpu, layout, agnostic, max_det):
    """Every fp16 encoding once, as the scores of 16384 anchors x 4 classes
    (shuffled), through the two-launch selection's class keys in its three
    load forms: 16-byte octets of anchors (transposed), 8-byte chunks of a
    contiguous row, and one score a lane (strided)."""
    g = torch.Generator().manual_seed(65536)
    bits = torch.randperm(65536, generator=g).to(torch.int32).to(torch.int16)
    scores = bits.view(torch.float16).reshape(1, 16384, 4)
    boxes = torch.randn(1, 16384, 4, generator=g).half()
    x = torch.cat((boxes, scores), -1)
    run_case(gpu, x, max_det, agnostic, layout, f"every-encoding-{layout}-{agnostic}-{max_det}")


@pytest.mark.parametrize("batch,anchors,nc,max_det", [(2, 129, 4, 100), (2, 257, 12, 300), (3, 1000, 100, 300),
                                                      (1, 3360, 256, 300), (2, 8400, 80, 300), (1, 1, 4, 300),
                                                      (3, 7, 8, 5), (1, 500, 1024, 32)])
@pytest.mark.parametrize("agnostic", [False, True])
def test_selection_row_form(gpu, batch, anchors, nc, max_det, agnostic):
    """Contiguous rows read as 8-byte class chunks (nc a multiple of 4): a
    partial last run of anchors, chunk counts not a multiple of the four
    lanes of an anchor, classes over two or more load passes (up to the
    1024-class maximum), single- and few-anchor images, and batches."""
    from tests.selection_fixtures import predictions
    x = predictions(batch, anchors, nc, seed=anchors + nc)
    run_case(gpu, x, max_det, agnostic, "contiguous", f"row-{batch}x{anchors}x{nc}-{agnostic}")


@pytest.mark.parametrize("noalloc", [False, True])
def test_selection_graph_replays(gpu, noalloc):
    """Selections captured into a HIP graph: every replay, with eager
    selections on the same device between replays, gives the eager result
    bit for bit, on the C5 image (transposed view) and a 4-image batch, with
    a workspace and on the static scratch."""
    from thintnpu_amd import capi
    from tests.selection_fixtures import predictions
    cases = []
    for x, layout, k in ((c5_selection_input(), "transposed", 300), (predictions(4, 3360, 80, seed=78), "contiguous", 300)):
        base, view = backing_and_view(x, layout)
        dv = view(base.to(gpu))
        ref = sel.select(view(base), k, False)["output"]
        eager = capi.detection_select(dv, k, noalloc=noalloc)
        assert bits_equal(eager.cpu(), ref)
        cases.append((dv, k, eager))
    outs = [torch.full_like(e, float("nan")) for _, _, e in cases]
    wss = [None if noalloc else torch.empty(capi.detection_select_workspace(dv.shape[0], dv.shape[1], dv.shape[2] - 4,
                                                                            k, False), dtype=torch.uint8, device=gpu)
           for dv, k, _ in cases]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for (dv, k, _), o, ws in zip(cases, outs, wss):
            capi.detection_select(dv, k, out=o, workspace=ws, noalloc=noalloc)
    for replay in range(4):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for (dv, k, eager), o in zip(cases, outs):
            assert bits_equal(o.cpu(), eager.cpu()), f"replay {replay}"
        # eager calls between replays
        for dv, k, eager in cases:
            assert bits_equal(capi.detection_select(dv, k, noalloc=noalloc).cpu(), eager.cpu())
