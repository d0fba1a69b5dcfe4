"""Attention-contraction oracle (numpy / torch on the CPU; test infrastructure
only).

  logical(x, transpose, groups, origin, channels)
                      -- the logical [batch, rows, cols] matrix an operand
                         denotes (bmm_flow.cpp:193-215,279-300): a blocked
                         [N, C1, T, 16] operand has channels as rows and tokens
                         as columns (verify_bmm_layout.py:59-60); groups split
                         the channels of an N=1 operand into heads; origin /
                         channels select a row range per head
  sequential_bmm(a, b) -- fp32 products summed in reduction order from zero,
                         one cast to fp16 (verify_bmm_layout.py:16-20;
                         bmm_flow.cpp:140-167)
  layout_bmm(...)      -- layout_bmm's result, incl. the NC1HWC0 packing of a
                         blocked output (bmm_flow.cpp:276-340,172-191)
  bmm(a, b)            -- rank-3 bmm (bmm_flow.cpp:342-345)
  channel_select(x, groups, begin, count)
                       -- channels [begin, begin+count) of each of `groups`
                         equal channel groups, packed (bmm_flow.cpp:217-266)

Pinning (tests/test_oracle_bmm.py): with small-integer operands every product
and partial sum is exact, so the result must equal an integer matrix product
formed by brute-force loops over the raw tensor elements -- this fixes the
index mapping of transposes, blocked rows, head groups, channel ranges and the
blocked output packing; known answers fix the summation order
([4096, 1, 4096] . [4096, 1, -4096] is 0 in sequential fp32, 1 exactly) and
the fp32 accumulator (4096 ones sum to 4096, an fp16 accumulator stalls at
2048); random operands stay within the reference's 0.002 tolerance of
torch.bmm in fp32 (verify_bmm_flow.py:20-25); channel_select matches the
reference test's own construction (verify_bmm_layout.py:89-104).
"""
from __future__ import annotations

import numpy as np
import torch


def logical(x: torch.Tensor, transpose: bool = False, groups: int = 0, origin: int = 0,
            channels: int = -1) -> torch.Tensor:
    """fp32 [batch, rows, cols] of operand x as layout_bmm reads it."""
    x = x.detach().cpu().float()
    if x.dim() == 4:
        batch, c1, tokens, c0 = x.shape
        m = x.permute(0, 1, 3, 2).reshape(batch, c1 * c0, tokens)
        if groups:
            m = m.reshape(groups, c1 * c0 // groups, tokens)
    else:
        m = x
    rows = m.shape[1]
    if channels < 0:
        channels = rows - origin
    m = m[:, origin:origin + channels]
    return m.transpose(1, 2) if transpose else m


def sequential_bmm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """fp16 of the fp32 sum over k = 0..K-1 of a[:, :, k] * b[:, k, :]."""
    a32 = np.ascontiguousarray(a.detach().cpu().float().numpy(), dtype=np.float32)
    b32 = np.ascontiguousarray(b.detach().cpu().float().numpy(), dtype=np.float32)
    acc = np.zeros((a32.shape[0], a32.shape[1], b32.shape[2]), dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):  # inf / NaN operands are part of the contract
        for k in range(a32.shape[2]):
            acc += a32[:, :, k, None] * b32[:, None, k, :]
        return torch.from_numpy(acc.astype(np.float16))


def layout_bmm(a: torch.Tensor, b: torch.Tensor, transpose_a: bool = False, transpose_b: bool = False,
               blocked_output: bool = False, groups: int = 0, a_offset: int = 0, a_channels: int = -1,
               b_offset: int = 0, b_channels: int = -1) -> torch.Tensor:
    la = logical(a, transpose_a, groups if a.dim() == 4 else 0, a_offset, a_channels)
    lb = logical(b, transpose_b, groups if b.dim() == 4 else 0, b_offset, b_channels)
    y = sequential_bmm(la, lb)
    if not blocked_output:
        return y
    batch, m, n = y.shape
    if groups:
        return y.reshape(1, batch * m // 16, 16, n).permute(0, 1, 3, 2).contiguous()
    return y.reshape(batch, m // 16, 16, n).permute(0, 1, 3, 2).contiguous()


def bmm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return layout_bmm(a, b)


def channel_select(x: torch.Tensor, groups: int, begin: int, count: int) -> torch.Tensor:
    """Bit copy: out channel c = x channel (c // count) * (C // groups) + begin + c % count."""
    bits = x.detach().cpu().contiguous().view(torch.int16).numpy()
    _, c1, tokens, c0 = bits.shape
    chans = bits.transpose(0, 1, 3, 2).reshape(c1 * c0, tokens)
    c = np.arange(groups * count)
    src = (c // count) * (c1 * c0 // groups) + begin + c % count
    sel = chans[src].reshape(1, groups * count // 16, 16, tokens).transpose(0, 1, 3, 2)
    return torch.from_numpy(np.ascontiguousarray(sel)).view(torch.float16)
