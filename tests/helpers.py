"""Shared input generators for the parity tests (CPU, seeded)."""
import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def normal16(shape, seed, mean=0.0, std=1.0):
    """fp32 N(mean, std) draws from a seeded CPU generator, cast to fp16."""
    return (torch.randn(shape, generator=gen(seed)) * std + mean).to(torch.float16)


def uniform16(shape, seed, lo=0.0, hi=1.0):
    return (torch.rand(shape, generator=gen(seed)) * (hi - lo) + lo).to(torch.float16)


def random_bits16(shape, seed):
    """Every fp16 encoding equally likely (NaN payloads, infinities, subnormals)."""
    return torch.randint(-32768, 32768, shape, dtype=torch.int16, generator=gen(seed)).view(torch.float16)


SPECIALS = [0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1.0, -1.0, 2.0,
            65504.0, -65504.0, 2.0 ** -24, -(2.0 ** -24), 2.0 ** -14, 0.5, -0.5, 11.0]


def specials16(n=None):
    t = torch.tensor(SPECIALS, dtype=torch.float16)
    if n is not None:
        t = t.repeat((n + t.numel() - 1) // t.numel())[:n]
    return t


def to_blocked(x):
    """NCHW -> NC1HWC0 (C0=16, zero padded) on CPU by reshape/permute."""
    n, c, h, w = x.shape
    c1 = (c + 15) // 16
    if c1 * 16 != c:
        x = torch.cat([x, x.new_zeros(n, c1 * 16 - c, h, w)], 1)
    return x.reshape(n, c1, 16, h, w).permute(0, 1, 3, 4, 2).contiguous()
