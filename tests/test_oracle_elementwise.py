"""Pins the elementwise oracle to what the mathematics fixes (CPU only)."""
import numpy as np
import torch

from oracle import elementwise as ew
from oracle.numerics import ulp_report, bits16
from tests.helpers import random_bits16, specials16, normal16


def exact_round16(values64: np.ndarray) -> torch.Tensor:
    # numpy float64 -> float16 cast rounds to nearest even once.
    return torch.from_numpy(values64.astype(np.float16))


def operands(n=200_000):
    a = random_bits16((n,), 1)
    b = random_bits16((n,), 2)
    s = specials16()
    a = torch.cat([a, s.repeat_interleave(len(s))])
    b = torch.cat([b, s.repeat(len(s))])
    return a, b


def test_binary_oracle_is_correctly_rounded():
    a, b = operands()
    a64, b64 = a.double().numpy(), b.double().numpy()
    with np.errstate(all="ignore"):
        exact = {0: a64 - b64, 1: a64 * b64, 2: a64 / b64, 3: a64 + b64}
    for op, ref64 in exact.items():
        got = ew.binary(op, a, b)
        rep = ulp_report(got, exact_round16(ref64))
        assert rep["nan_match"] and rep["inf_match"] and rep["max_ulp"] == 0, (op, rep)


def test_binary_alpha_follows_cpu_vector_rule():
    # One parallel chunk (< 32768 elements); CPU's scalar tail covers the last
    # few elements and evaluates alpha differently, so compare the vector part.
    a, b = random_bits16((20_000,), 11), random_bits16((20_000,), 12)
    for op in (0, 3):
        for alpha in (0.3, -2.0, 0.5, 1 / 3):
            cpu = (torch.add if op == 3 else torch.sub)(a, b, alpha=alpha)
            mine = ew.binary(op, a, b, alpha)
            rep = ulp_report(mine[:-64], cpu[:-64])
            assert rep["nan_match"] and rep["max_ulp"] == 0, (op, alpha, rep)
            # closed form: alpha rounded to fp16, fp32 evaluation, one cast
            al = np.float64(np.float16(alpha)) * (1 if op == 3 else -1)
            with np.errstate(all="ignore"):
                ref = torch.from_numpy(np.float32(a.double().numpy() + al * b.double().numpy())
                                       .astype(np.float16))
            assert ulp_report(mine, ref)["max_ulp"] == 0


def test_scalar_rules():
    x = random_bits16((8_000,), 13)
    x64 = x.double().numpy()
    for sc in (0.17677669529663687, 0.3, 3.0):
        s16, s32 = np.float64(np.float16(sc)), np.float64(np.float32(sc))
        with np.errstate(all="ignore"):
            models = {(3, False): x64 + s16, (0, False): x64 - s16, (0, True): s16 - x64,
                      (1, False): x64 * s32, (2, False): x64 / s32}
        for (op, first), ex in models.items():
            ref = torch.from_numpy(np.float32(ex).astype(np.float16))
            rep = ulp_report(ew.binary_scalar(op, x, sc, first), ref)
            assert rep["nan_match"] and rep["max_ulp"] == 0, (op, first, sc, rep)


def test_scalar_rounded_rule():
    """The reference's rule: the scalar is rounded to fp16 for every op, then
    each op is one correctly rounded fp16 operation on fp16 values.  1/sqrt(32)
    is not an fp16 value, so this rule and PyTorch CPU's fp32 rule for mul
    must disagree on some inputs (the check would pass either way otherwise)."""
    x = random_bits16((8_000,), 14)
    x64 = x.double().numpy()
    for sc in (0.17677669529663687, 0.3, 3.0):
        s16 = np.float64(np.float16(sc))
        with np.errstate(all="ignore"):
            models = {(3, False): x64 + s16, (0, False): x64 - s16, (0, True): s16 - x64, (3, True): s16 + x64,
                      (1, False): x64 * s16, (1, True): s16 * x64, (2, False): x64 / s16, (2, True): s16 / x64}
        for (op, first), ex in models.items():
            ref = torch.from_numpy(np.float32(ex).astype(np.float16))
            rep = ulp_report(ew.binary_scalar_rounded(op, x, sc, first), ref)
            assert rep["nan_match"] and rep["max_ulp"] == 0, (op, first, sc, rep)
    q = ew.binary_scalar_rounded(1, x, 32 ** -0.5)
    cpu = ew.binary_scalar(1, x, 32 ** -0.5)
    finite = torch.isfinite(q.float()) & torch.isfinite(cpu.float())
    assert (q[finite] != cpu[finite]).any()


def test_unary_oracles_within_one_ulp_of_float64():
    x = torch.cat([random_bits16((100_000,), 3), specials16()])
    x64 = x.double().numpy()
    with np.errstate(all="ignore"):
        sig = 1.0 / (1.0 + np.exp(-x64))
        silu = x64 / (1.0 + np.exp(-x64))
    for got, ref in ((ew.sigmoid(x), sig), (ew.silu(x), silu)):
        rep = ulp_report(got, exact_round16(ref))
        assert rep["nan_match"] and rep["inf_match"] and rep["max_ulp"] <= 1, rep


def test_silu_add_single_rounding():
    x, y = normal16((100_000,), 4), normal16((100_000,), 5)
    x64, y64 = x.double().numpy(), y.double().numpy()
    ref = exact_round16(y64 + x64 / (1.0 + np.exp(-x64)))
    rep = ulp_report(ew.silu_add(x, y), ref)
    assert rep["max_ulp"] <= 1, rep
    # the unfused chain rounds twice (far away only where y ~ -silu(x) cancels)
    unfused = ulp_report(ew.silu_add_unfused(x, y), ref)
    assert unfused["exact"] > 0.5 * unfused["count"]


def test_affine_silu_keeps_fp16_intermediates():
    x = normal16((4, 8, 5, 5, 16), 6)
    s = (torch.rand((1, 8, 1, 1, 16), generator=torch.Generator().manual_seed(7)) + 0.5).half()
    b = normal16((1, 8, 1, 1, 16), 8, std=0.1)
    t1 = exact_round16((x.double() * s.double()).numpy())
    t2 = exact_round16((t1.double() + b.double()).numpy())
    t264 = t2.double().numpy()
    ref = exact_round16(t264 / (1.0 + np.exp(-t264)))
    assert ulp_report(ew.affine_silu(x, s, b), ref)["max_ulp"] <= 1
    # a dropped bias or a swapped operand moves far away
    wrong = ew.affine_silu(x, s, torch.zeros_like(b))
    assert ulp_report(wrong, ref)["max_ulp"] > 2


def test_ulp_metric_encodings():
    r = torch.tensor([1.0, -0.0, 0.0, 65504.0], dtype=torch.float16)
    a = torch.tensor([1.0009765625, 0.0, -(2.0 ** -24), float("inf")], dtype=torch.float16)
    rep = ulp_report(a[:3], r[:3])
    assert rep["max_ulp"] == 1 and rep["exact"] == 1
    assert not ulp_report(a, r)["inf_match"]
    assert bits16(torch.tensor([-0.0], dtype=torch.float16))[0] == 0x8000
