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
