"""YOLO26 selection oracle (numpy on fp16 bit patterns; test infrastructure only).

  score_key(bits)   -- selection_flow.cpp:30-35: 0 for NaN, 0x7fff for +-0, raw
                       bits for negatives, ~(bits ^ 0x8000) & 0xffff for
                       positives; ascending key = NaN first, then descending value.
  float_bits(bits)  -- selection_flow.cpp:37-51: exact half -> float bits, NaNs
                       quieted with sign and payload kept.
  select(x, max_det, agnostic) -- the stable two-stage contract of
                       SELECTION_FLOW.md:8-16 and the stable reference of
                       verify_selection_flow.py:27-47: first best class per
                       anchor, top-K anchors by (key, index), gathered [K, nc]
                       scores, top-K pairs by (key, rank*nc + c), boxes of the
                       mapped anchors; returns the eight trace stages.

Pinning (tests/test_oracle_selection.py): score_key order over all 65,536
encodings equals torch's stable descending argsort; float_bits equals torch's
half -> float bits for all 65,536; select equals brute-force sorted() on tiny
inputs, an independent torch argsort restatement on the reference's fixture
list, and torch.topk on tie-free inputs.
"""
from __future__ import annotations

import numpy as np
import torch

TRACE_NAMES = ("output", "class_max", "stage1_indices", "gathered_scores", "top_values",
               "stage2_indices", "anchor_indices", "labels")


def score_key(bits: np.ndarray) -> np.ndarray:
    b = np.asarray(bits, dtype=np.int64) & 0xFFFF
    mag = b & 0x7FFF
    key = np.where(b & 0x8000, b, (~(b ^ 0x8000)) & 0xFFFF)
    key = np.where(mag == 0, 0x7FFF, key)
    return np.where(mag > 0x7C00, 0, key)


def float_bits(bits: np.ndarray) -> np.ndarray:
    h = np.asarray(bits, dtype=np.int64) & 0xFFFF
    sign = (h & 0x8000) << 16
    exp = (h >> 10) & 31
    man = h & 1023
    out = np.zeros_like(h)
    # inf / NaN
    special = exp == 31
    out = np.where(special, sign | 0x7F800000 | (man << 13) | np.where(man != 0, 0x00400000, 0), out)
    normal = (exp > 0) & (exp < 31)
    out = np.where(normal, sign | ((exp + 112) << 23) | (man << 13), out)
    sub = (exp == 0) & (man != 0)
    if sub.any():
        m = man[sub].copy()
        e = np.full_like(m, 113)
        for _ in range(11):
            shift = (m & 1024) == 0
            m = np.where(shift, m << 1, m)
            e = np.where(shift, e - 1, e)
        out[sub] = sign[sub] | (e << 23) | ((m & 1023) << 13)
    zero = (exp == 0) & (man == 0)
    out = np.where(zero, sign, out)
    return out.astype(np.uint32)


def _stable_topk(keys: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k smallest (key, index) pairs, in that order."""
    order = np.lexsort((np.arange(keys.shape[-1]), keys))
    return order[:k]


def select(x: torch.Tensor, max_det: int, agnostic: bool = False) -> dict:
    x = x.detach().cpu()
    bsz, anchors, ch = x.shape
    nc = ch - 4
    k = min(max_det, anchors)
    bits = x.contiguous().view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    out = np.zeros((bsz, k, 6), dtype=np.uint32)
    class_max = np.zeros((bsz, anchors), dtype=np.int64)
    stage1 = np.zeros((bsz, k), dtype=np.int64)
    gathered = np.zeros((bsz, 0 if agnostic else k, nc), dtype=np.int64)
    top = np.zeros((bsz, k), dtype=np.int64)
    stage2 = np.zeros((bsz, 0 if agnostic else k), dtype=np.int64)
    anchor_idx = np.zeros((bsz, k), dtype=np.int64)
    labels = np.zeros((bsz, k), dtype=np.int64)
    for b in range(bsz):
        sc = bits[b, :, 4:]
        keys = score_key(sc)
        cls = np.argmin(keys, axis=1) if anchors else np.zeros(0, dtype=np.int64)  # first best class
        mbits = sc[np.arange(anchors), cls] if anchors else np.zeros(0, dtype=np.int64)
        class_max[b] = mbits
        first = _stable_topk(score_key(mbits), k)
        stage1[b] = first
        if agnostic:
            top[b], labels[b], anchor_idx[b] = mbits[first], cls[first], first
        else:
            g = sc[first]                      # [k, nc]
            gathered[b] = g
            flat = g.reshape(-1)
            second = _stable_topk(score_key(flat), k)
            stage2[b] = second
            top[b] = flat[second]
            labels[b] = second % nc
            anchor_idx[b] = first[second // nc]
        boxes = bits[b, anchor_idx[b], :4]
        out[b, :, :4] = float_bits(boxes)
        out[b, :, 4] = float_bits(top[b])
        out[b, :, 5] = labels[b].astype(np.float32).view(np.uint32)

    def half(a):
        return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.float16)

    return dict(zip(TRACE_NAMES, (
        torch.from_numpy(out.view(np.float32)), half(class_max), torch.from_numpy(stage1),
        half(gathered), half(top), torch.from_numpy(stage2), torch.from_numpy(anchor_idx),
        torch.from_numpy(labels))))
