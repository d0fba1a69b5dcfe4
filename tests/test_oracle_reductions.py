"""Pins the softmax / DFL oracle (CPU only)."""
import numpy as np
import torch

from oracle import reductions as rd
from oracle.numerics import rel_error, FP16_MIN_NORMAL


def np_softmax(x: np.ndarray, axis: int) -> np.ndarray:
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def test_softmax_against_float64():
    g = torch.Generator().manual_seed(2718)
    for shape, dim in (((5, 1000), 1), ((2, 16, 37), 1), ((1, 4, 16, 8400), 2), ((3, 400), -1)):
        x = torch.randn(shape, generator=g) * 3
        ref = np_softmax(x.double().numpy(), dim)
        got32 = rd.softmax(x, dim).double().numpy()
        assert np.max(np.abs(got32 - ref) / np.maximum(np.abs(ref), 1e-30)) < 1e-5
        ref16 = torch.from_numpy(np_softmax(x.half().double().numpy(), dim))
        rel, _ = rel_error(rd.softmax_rounded(x.half(), dim), ref16)
        assert rel <= 2.0 ** -11 * 1.01          # one rounding of a ~exact fp32 value
        _, ab = rel_error(rd.softmax(x.half(), dim), ref16)
        assert ab <= 1e-3                         # CPU fp16 op, reference test's atol
        np.testing.assert_allclose(got32.sum(axis=dim), 1.0, rtol=1e-5)


def test_softmax_nonfinite_rules():
    # [.., NaN, ..] -> all NaN; all -inf -> all NaN; +inf -> all NaN; -inf alone -> 0
    x = torch.tensor([[0.0, float("nan"), 1.0], [float("-inf")] * 3, [0.0, float("inf"), 1.0],
                      [float("-inf"), 0.0, 0.0]], dtype=torch.float16)
    y = rd.softmax(x, 1)
    assert torch.isnan(y[0]).all() and torch.isnan(y[1]).all() and torch.isnan(y[2]).all()
    assert y[3, 0] == 0 and abs(float(y[3, 1]) - 0.5) < 1e-3


def test_softmax_half_to_float():
    x = torch.randn(3, 100).half()
    y = rd.softmax(x, 1, True)
    assert y.dtype == torch.float32
    ref = np_softmax(x.double().numpy(), 1)
    assert np.max(np.abs(y.double().numpy() - ref)) < 1e-6


def test_dfl_expect_closed_form_and_invariants():
    g = torch.Generator().manual_seed(1928)
    x = (torch.randn(2, 64, 8400, generator=g) * 3).half()
    got = rd.dfl_expect(x, torch.float32).double()
    xn = x.double().numpy().reshape(2, 4, 16, 8400)
    ref = (np_softmax(xn, 2) * np.arange(16).reshape(1, 1, 16, 1)).sum(2)
    assert np.max(np.abs(got.numpy() - ref)) < 1e-5
    assert float(got.min()) >= 0 and float(got.max()) <= 15
    rel, _ = rel_error(rd.dfl_expect(x), torch.from_numpy(ref))
    assert rel <= 2.0 ** -11
    # one-hot: bin k dominant -> expectation ~ k (a swapped bin order would fail)
    hot = torch.full((1, 64, 4), -20.0)
    for s, k in enumerate((0, 5, 11, 15)):
        hot[0, 16 * s + k, :] = 20.0
    e = rd.dfl_expect(hot.half(), torch.float32)[0, :, 0]
    assert torch.allclose(e, torch.tensor([0.0, 5.0, 11.0, 15.0]), atol=1e-3)
    # the unfused chain stays within the fp16 rounding of its probabilities
    rel_u, _ = rel_error(rd.dfl_expect_unfused(x), torch.from_numpy(ref))
    assert rel_u < 4e-3
