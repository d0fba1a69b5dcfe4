"""thin_detection_select_noalloc (the allocation-free selection entry point)
against thin_detection_select with a workspace, through the C ABI: output rows
and every trace stage bit-equal, on two calls in a row (the second with a
smaller input, so stale scratch contents from the first would show), plus the
size-limit rejection."""
import ctypes

import pytest
import torch

from oracle import selection as sel
from oracle.numerics import bits_equal
from tests.selection_fixtures import backing_and_view, c5_selection_input, predictions

pytestmark = pytest.mark.gpu


def both_entries(gpu, x, max_det, agnostic, layout, name):
    from thintnpu_amd import capi
    base, view = backing_and_view(x, layout)
    dv = view(base.to(gpu))
    print(f"noalloc case {name}: shape={tuple(dv.shape)} K={max_det} agnostic={agnostic} layout={layout}",
          flush=True)
    ref_out, ref_tr = capi.detection_select(dv, max_det, agnostic, trace=True)
    out, tr = capi.detection_select(dv, max_det, agnostic, trace=True, noalloc=True)
    plain = capi.detection_select(dv, max_det, agnostic, noalloc=True)
    torch.cuda.synchronize()
    assert bits_equal(out.cpu(), ref_out.cpu()), f"{name}: output"
    assert bits_equal(plain.cpu(), ref_out.cpu()), f"{name}: output without trace"
    for stage, t in ref_tr.items():
        assert bits_equal(tr[stage].cpu(), t.cpu()), f"{name}: {stage}"
    expect = sel.select(view(base), max_det, agnostic)["output"]
    assert bits_equal(out.cpu(), expect), f"{name}: oracle"


@pytest.mark.parametrize("agnostic", [False, True])
def test_noalloc_matches_workspace_entry(gpu, agnostic):
    both_entries(gpu, c5_selection_input(), 300, agnostic, "transposed", "c5")
    small = predictions(1, 700, 20, seed=31)
    both_entries(gpu, small, 50, agnostic, "contiguous", "small")


def test_noalloc_batched_then_single(gpu):
    both_entries(gpu, predictions(4, 3360, 80, seed=77), 300, False, "transposed", "batched")
    both_entries(gpu, predictions(1, 1000, 80, seed=78), 100, False, "transposed", "single")


def test_noalloc_rejects_sizes_beyond_the_scratch(gpu):
    from thintnpu_amd import capi
    lib = capi.lib()
    b, a, nc, k = 100, 8400, 80, 300
    need = capi.detection_select_workspace(b, a, nc, k, False)
    assert need > capi.SELECT_SCRATCH_BYTES
    x = torch.zeros((b, a, nc + 4), dtype=torch.float16, device=gpu)
    out = torch.zeros((b, k, 6), dtype=torch.float32, device=gpu)
    st = lib.thin_detection_select_noalloc(ctypes.byref(capi.desc(x)), k, 0, out.data_ptr(), None,
                                           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st == 4 and b"scratch" in lib.thin_last_error()
    assert not out.any().item()  # nothing was launched
