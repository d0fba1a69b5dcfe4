"""Pins the selection oracle (CPU only)."""
import itertools

import numpy as np
import pytest
import torch

from oracle import selection as sel
from tests.selection_fixtures import backing_and_view, c5_selection_input, fixtures, predictions

ALL = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)


def test_score_key_order_equals_stable_descending_argsort():
    keys = sel.score_key(np.arange(65536))
    mine = np.lexsort((np.arange(65536), keys))
    ref = torch.argsort(ALL, descending=True, stable=True).numpy()
    assert np.array_equal(mine, ref)


def test_float_bits_equals_torch_half_to_float():
    mine = sel.float_bits(np.arange(65536))
    ref = ALL.float().view(torch.int32).numpy().astype(np.int64) & 0xFFFFFFFF
    assert np.array_equal(mine.astype(np.int64), ref)


def torch_stable_reference(x, max_det, agnostic):
    """Independent restatement with torch ops on halves: stable descending
    argsort, int16 gathers (keeps sNaN payloads)."""
    b, anchors, ch = x.shape
    nc, k = ch - 4, min(max_det, anchors)
    scores = x[..., 4:]
    keyed = torch.from_numpy(sel.score_key(scores.contiguous().view(torch.int16).numpy().astype(np.int64) & 0xFFFF))
    labels = keyed.argmin(-1) if anchors else torch.zeros(b, 0, dtype=torch.long)
    ib = lambda t: t.contiguous().view(torch.int16)
    maximum = ib(scores).gather(2, labels[..., None]).squeeze(-1).view(torch.float16)
    first = torch.argsort(maximum, dim=1, descending=True, stable=True)[:, :k]
    if agnostic:
        top = ib(maximum).gather(1, first).view(torch.float16)
        label, anchor = labels.gather(1, first), first
    else:
        gathered = ib(scores).gather(1, first[..., None].expand(-1, -1, nc)).view(torch.float16)
        flat = gathered.reshape(b, k * nc)
        second = torch.argsort(flat, dim=1, descending=True, stable=True)[:, :k]
        top = ib(flat).gather(1, second).view(torch.float16)
        label, anchor = second % nc, first.gather(1, second // nc)
    boxes = ib(x[..., :4]).gather(1, anchor[..., None].expand(-1, -1, 4))
    # half -> float through the KAT-pinned float_bits: torch's own conversion of
    # a NaN differs between its vectorized and scalar loops (0x7fc00000 vs
    # 0x7fffffff for 0x7e00)
    fb = lambda h: torch.from_numpy(sel.float_bits(h.numpy().astype(np.int64) & 0xFFFF).view(np.float32))
    return torch.cat((fb(boxes), fb(ib(top))[..., None], label[..., None].float()), -1)


def bits_eq(a, b):
    return a.shape == b.shape and torch.equal(a.contiguous().view(torch.int32), b.contiguous().view(torch.int32))


def test_brute_force_tiny():
    g = torch.Generator().manual_seed(3)
    for trial in range(40):
        b, a, nc = 1, int(torch.randint(1, 9, (1,), generator=g)), int(torch.randint(1, 5, (1,), generator=g))
        vals = torch.tensor([0.5, 0.25, 0.5, -0.0, 0.0, float("nan"), 1.0, float("inf")], dtype=torch.float16)
        idx = torch.randint(0, len(vals), (b, a, nc), generator=g)
        x = torch.cat((torch.randn(b, a, 4, generator=g).half(), vals[idx]), -1)
        k = int(torch.randint(0, a + 2, (1,), generator=g))
        r = sel.select(x, k, False)
        keys = sel.score_key(x[0, :, 4:].contiguous().view(torch.int16).numpy().astype(np.int64) & 0xFFFF)
        best = [min(range(nc), key=lambda c: (keys[i, c], c)) for i in range(a)]
        order = sorted(range(a), key=lambda i: (keys[i, best[i]], i))[:min(k, a)]
        assert r["stage1_indices"][0].tolist() == order
        pairs = sorted(((keys[order[r_], c], r_ * nc + c) for r_, c in itertools.product(range(len(order)), range(nc))))
        assert r["stage2_indices"][0].tolist() == [p[1] for p in pairs[:min(k, a)]]


@pytest.mark.parametrize("case", list(fixtures(full=False)), ids=lambda c: c[0])
def test_fixture_against_torch_restatement(case):
    name, x, max_det, agnostic, layout, unique = case
    base, view = backing_and_view(x, layout)
    v = view(base)
    r = sel.select(v, max_det, agnostic)
    assert bits_eq(r["output"], torch_stable_reference(v, max_det, agnostic)), name
    if unique and min(max_det, v.shape[1]) > 0:
        # tie-free scores: exact torch.topk parity (verify_selection_flow.py:267-268)
        scores = v[..., 4:].float()
        if agnostic:
            top = scores.max(-1).values.topk(min(max_det, v.shape[1]), dim=1)
            assert torch.equal(r["stage1_indices"], top.indices)
        else:
            m = scores.max(-1).values.topk(min(max_det, v.shape[1]), dim=1).indices
            assert torch.equal(r["stage1_indices"], m)


def test_c5_input_and_reference():
    x = c5_selection_input()
    r = sel.select(x, 300, False)
    assert r["output"].shape == (1, 300, 6)
    assert bits_eq(r["output"], torch_stable_reference(x, 300, False))
    assert torch.isnan(r["top_values"][0, :5].float()).all()  # NaNs rank first
