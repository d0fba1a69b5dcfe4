"""Detect-head decode oracle (PyTorch CPU; test infrastructure only).

Restates anchorfree_predictions (whole_blocked.py:118-146; YOLO26.md:30-38):

  grid(shapes, strides)  -- per-level cell centres (x + 0.5, y + 0.5) and
                            strides in fp16, anchors in level order, row-major
                            within a level (whole_blocked.py:126-134)
  box_decode(d, ...)     -- lower = anchor - d[:, :2], upper = anchor + d[:, 2:];
                            xyxy cat(lower, upper) * stride, or xywh
                            cat((lower+upper)/2, upper-lower) * stride, every
                            step an fp16 tensor op (whole_blocked.py:136-143)
  detect_decode(...)     -- cat(box_decode(dfl_expect(boxes)), sigmoid(scores))
                            with the fused DFL expectation (fp16 output) of
                            oracle.reductions (whole_blocked.py:135,144); for
                            [B,4,A] boxes (reg_max = 1, e.g. YOLO26, whose
                            module.dfl is the identity) the boxes are the
                            distances (YOLO26.md:30-38)

Pinning (tests/test_oracle_detect.py): the grid against a brute-force loop;
each fp16 box step against float64 arithmetic rounded once (fp16 tensor ops
are correctly rounded); closed forms for zero distances and one-hot DFL logits
(distance = the hot bin exactly).
"""
from __future__ import annotations

import torch

from oracle import elementwise as ew
from oracle import reductions as rd


def grid(shapes, strides):
    points, scales = [], []
    for (h, w), s in zip(shapes, strides):
        y, x = torch.meshgrid(torch.arange(h, dtype=torch.float16) + 0.5,
                              torch.arange(w, dtype=torch.float16) + 0.5, indexing="ij")
        points.append(torch.stack((x, y), 0).reshape(2, -1))
        scales.append(torch.full((1, h * w), s, dtype=torch.float16))
    return torch.cat(points, -1), torch.cat(scales, -1)


def box_decode(distance: torch.Tensor, shapes, strides, xywh: bool = False) -> torch.Tensor:
    anchors, scale = grid(shapes, strides)
    left_top, right_bottom = distance.split((2, 2), dim=1)
    lower, upper = anchors.unsqueeze(0) - left_top, anchors.unsqueeze(0) + right_bottom
    if xywh:
        return torch.cat(((lower + upper) / 2, upper - lower), 1) * scale
    return torch.cat((lower, upper), 1) * scale


def detect_decode(boxes: torch.Tensor, scores: torch.Tensor, shapes, strides, xywh: bool = False) -> torch.Tensor:
    distance = boxes if boxes.shape[1] == 4 else rd.dfl_expect(boxes, torch.float16)
    return torch.cat((box_decode(distance, shapes, strides, xywh), ew.sigmoid(scores)), 1)
