"""Pins the detect-decode oracle (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import detect as dt
from oracle.numerics import bits_equal

SHAPES = [(4, 6), (2, 3), (1, 2)]
STRIDES = [8.0, 16.0, 32.0]


def test_grid_brute_force():
    anchors, scale = dt.grid(SHAPES, STRIDES)
    i = 0
    for (h, w), s in zip(SHAPES, STRIDES):
        for y in range(h):
            for x in range(w):
                assert anchors[0, i].item() == x + 0.5 and anchors[1, i].item() == y + 0.5
                assert scale[0, i].item() == s
                i += 1
    assert i == anchors.shape[1]


@pytest.mark.parametrize("xywh", [False, True])
def test_box_steps_are_correctly_rounded(xywh):
    g = torch.Generator().manual_seed(3)
    a = sum(h * w for h, w in SHAPES)
    d = (torch.rand(2, 4, a, generator=g) * 15).half()
    got = dt.box_decode(d, SHAPES, STRIDES, xywh).numpy().astype(np.float64)
    anchors, scale = dt.grid(SHAPES, STRIDES)
    c, s = anchors.numpy().astype(np.float64), scale.numpy().astype(np.float64)
    r = lambda v: v.astype(np.float16).astype(np.float64)  # noqa: E731  one rounding
    dd = d.numpy().astype(np.float64)
    lower, upper = r(c[None] - dd[:, :2]), r(c[None] + dd[:, 2:])
    if xywh:
        want = np.concatenate((r(r(r(lower + upper) / 2) * s), r(r(upper - lower) * s)), 1)
    else:
        want = np.concatenate((r(lower * s), r(upper * s)), 1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("xywh", [False, True])
def test_closed_forms(xywh):
    a = sum(h * w for h, w in SHAPES)
    anchors, scale = dt.grid(SHAPES, STRIDES)
    zero = dt.box_decode(torch.zeros(1, 4, a, dtype=torch.float16), SHAPES, STRIDES, xywh)
    centre = (anchors * scale)[None]
    if xywh:
        assert bits_equal(zero[:, :2], centre) and not zero[:, 2:].any()
    else:
        assert bits_equal(zero[:, :2], centre) and bits_equal(zero[:, 2:], centre)
    # one-hot DFL logits: the expectation is the hot bin exactly
    hot = torch.tensor([3, 0, 15, 7])
    logits = torch.full((1, 64, a), -30.0, dtype=torch.float16)
    for side, k in enumerate(hot):
        logits[0, side * 16 + k] = 30.0
    out = dt.detect_decode(logits, torch.zeros(1, 5, a, dtype=torch.float16), SHAPES, STRIDES, xywh)
    d = hot.view(1, 4, 1).half().expand(1, 4, a)
    assert bits_equal(out[:, :4], dt.box_decode(d, SHAPES, STRIDES, xywh))
    assert (out[:, 4:] == 0.5).all()


def test_direct_distances_closed_form():
    """[B,4,A] boxes (reg_max = 1) are the distances: with small integer
    distances every fp16 step is exact, so xyxy equals float64 arithmetic."""
    a = sum(h * w for h, w in SHAPES)
    anchors, scale = dt.grid(SHAPES, STRIDES)
    d = torch.tensor([1.0, 2.0, 3.0, 4.0]).view(1, 4, 1).expand(1, 4, a).half()
    out = dt.detect_decode(d, torch.zeros(1, 2, a, dtype=torch.float16), SHAPES, STRIDES)
    cx, cy, s = anchors[0].double(), anchors[1].double(), scale[0].double()
    want = torch.stack(((cx - 1) * s, (cy - 2) * s, (cx + 3) * s, (cy + 4) * s))[None]
    assert torch.equal(out[:, :4].double(), want)
    assert (out[:, 4:] == 0.5).all()
