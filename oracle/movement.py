"""Data-movement oracle (numpy on raw bit patterns; test infrastructure only).

Every function moves bits only, so parity is bit-exact (NaN payloads included).

  cat(tensors, dim)          -- PyTorch cat semantics incl. skipping legacy 1-D
                                empty inputs (ops.cpp:419-462)
  upsample2x_blocked(x)      -- y[n,c1,2h+i,2w+j,:] = x[n,c1,h,w,:]
                                (flow_ops.cpp:129-164; verify_fast_flow_bits.py:21)
  upsample2x_nchw(x)         -- nearest 2x of NCHW (upsample.cpp:5-124)
  upsample_cat_blocked(...)  -- cat over C1 of (optionally upsampled) inputs
  pack_blocked(x)            -- NCHW -> NC1HWC0, channels >= C zero
                                (conv_flow.cpp:406-443; layout_blocked.h:2-55)
  unpack_blocked(y, c)       -- inverse, first c channels (layout_blocked.h:57-69)
  maxpool_nchw(x, k)         -- stride-1 k x k max pool, padding k//2, via PyTorch CPU on
                                fp32 (verify_flow_ops.py:31-33; backend.cpp:245-266)
  maxpool_blocked(x, k)      -- the same pool on NC1HWC0 (flow_ops.cpp:82-127,208-231)

Pinning (tests/test_oracle_movement.py): cat against torch.cat; the upsamples
against torch's F.interpolate(mode="nearest") and brute-force loops; pack and
unpack against brute-force index loops and the pack -> unpack round trip; the
max pools against a brute-force window loop (first maximum in row-major order,
NaN if the window holds one) with +0/-0 ties, infinities and NaNs.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

_INT = {1: np.uint8, 2: np.int16, 4: np.int32, 8: np.int64}
_TINT = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    return t.contiguous().view(_TINT[t.element_size()]).numpy()


def _from_bits(a: np.ndarray, like: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).view(like.dtype)


def cat(tensors, dim: int) -> torch.Tensor:
    live = [t for t in tensors if not (t.dim() == 1 and t.numel() == 0)]
    ref = live[0] if live else tensors[0]
    if not live:
        return ref.new_empty((0,))
    dim = dim % ref.dim()
    out = np.concatenate([_bits(t) for t in live], axis=dim)
    return _from_bits(out, ref)


def upsample2x_blocked(x: torch.Tensor) -> torch.Tensor:
    b = _bits(x)
    return _from_bits(b.repeat(2, axis=2).repeat(2, axis=3), x)


def upsample2x_nchw(x: torch.Tensor) -> torch.Tensor:
    b = _bits(x)
    return _from_bits(b.repeat(2, axis=2).repeat(2, axis=3), x)


def upsample_cat_blocked(tensors, upsample) -> torch.Tensor:
    parts = [upsample2x_blocked(t) if u else t for t, u in zip(tensors, upsample)]
    return cat(parts, 1)


def pack_blocked(x: torch.Tensor) -> torch.Tensor:
    b = _bits(x)
    n, c, h, w = b.shape
    c1 = (c + 15) // 16
    padded = np.zeros((n, c1 * 16, h, w), dtype=b.dtype)
    padded[:, :c] = b
    return _from_bits(padded.reshape(n, c1, 16, h, w).transpose(0, 1, 3, 4, 2), x)


def unpack_blocked(y: torch.Tensor, channels: int | None = None) -> torch.Tensor:
    b = _bits(y)
    n, c1, h, w, c0 = b.shape
    c = c1 * c0 if channels is None else channels
    return _from_bits(b.transpose(0, 1, 4, 2, 3).reshape(n, c1 * c0, h, w)[:, :c], y)


def maxpool_nchw(x: torch.Tensor, kernel: int) -> torch.Tensor:
    """F.max_pool2d on fp32, stride 1, padding kernel // 2, cast back: max only
    selects existing values, so the fp32 detour is exact (verify_flow_ops.py:31-33)."""
    return F.max_pool2d(x.float(), kernel, stride=1, padding=kernel // 2).to(x.dtype)


def maxpool_blocked(x: torch.Tensor, kernel: int) -> torch.Tensor:
    """maxpool_nchw on the NCHW view of an NC1HWC0 tensor, repacked."""
    n, c1, h, w, c0 = x.shape
    nchw = x.permute(0, 1, 4, 2, 3).reshape(n, c1 * c0, h, w)
    y = maxpool_nchw(nchw, kernel)
    return y.reshape(n, c1, c0, h, w).permute(0, 1, 3, 4, 2).contiguous()


def sppf_blocked(x: torch.Tensor, kernel: int = 5, repeats: int = 3) -> torch.Tensor:
    """The SPPF block's pooling and concat (Ultralytics SPPF.forward, whose
    pools the reference runs through maxpool_forward, whole_blocked.py:63-64,
    and whose cat is thin_ops::cat, ops.cpp:419-462): each pool takes the
    previous one's output, cat over C1."""
    ys = [x]
    for _ in range(repeats):
        ys.append(maxpool_blocked(ys[-1], kernel))
    return torch.cat(ys, 1)
