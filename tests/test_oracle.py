"""Pins the numpy oracle (oracle/converse_oracle.py) with checks that do not restate its formulas:
library routines (torch F.pad / F.interpolate / F.layer_norm / F.conv2d / F.gelu), closed forms
derived from the reference's definitions (identities I1-I8), brute-force normal equations on tiny
planes, and planted mistakes in copies of the oracle that the same checks must reject."""
import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import converse_oracle as O
from tests.conftest import seeded as _rng
from tests.conftest import softmax_psf


# -------------------------------------------------------------------------------- a2 padding
@pytest.mark.parametrize("mode", ["circular", "reflect", "replicate", "constant"])
@pytest.mark.parametrize("p", [1, 2, 3])
def test_pad_matches_torch(mode, p):
    x = _rng(mode, p).standard_normal((2, 3, 7, 9))
    ref = F.pad(torch.from_numpy(x), [p] * 4, mode=mode, value=0).numpy()
    np.testing.assert_array_equal(O.pad_nchw(x, p, mode), ref)


def test_pad_index_closed_forms():
    # circular: (i - p) mod n; reflect: mirror without repeating the edge; replicate: clamp
    assert [O.pad_index(i, 5, 2, "circular") for i in range(9)] == [3, 4, 0, 1, 2, 3, 4, 0, 1]
    assert [O.pad_index(i, 5, 2, "reflect") for i in range(9)] == [2, 1, 0, 1, 2, 3, 4, 3, 2]
    assert [O.pad_index(i, 5, 2, "replicate") for i in range(9)] == [0, 0, 0, 1, 2, 3, 4, 4, 4]
    assert [O.pad_index(i, 5, 2, "constant") for i in range(9)] == [-1, -1, 0, 1, 2, 3, 4, -1, -1]


# -------------------------------------------------------------------------------- a5/a6 (I1, I2)
@pytest.mark.parametrize("s", [1, 2, 3, 4])
def test_nearest_matches_torch(s):
    x = _rng("n", s).standard_normal((1, 2, 5, 6))
    ref = F.interpolate(torch.from_numpy(x), scale_factor=s, mode="nearest").numpy()
    np.testing.assert_array_equal(O.nearest(x, s), ref)


@pytest.mark.parametrize("s", [2, 3])
def test_I1_zero_insert_tiles_spectrum(s):
    x = _rng("I1", s).standard_normal((1, 1, 6, 7))
    lhs = np.fft.fft2(O.upsample_zero(x, s))
    rhs = np.tile(np.fft.fft2(x), (1, 1, s, s))
    np.testing.assert_allclose(lhs, rhs, atol=1e-12)


@pytest.mark.parametrize("s", [2, 3])
def test_I2_nearest_hold_spectrum(s):
    x = _rng("I2", s).standard_normal((1, 1, 6, 7))
    h, w = x.shape[-2:]
    Hs, Ws = h * s, w * s
    hold = lambda N: np.exp(-2j * np.pi * np.outer(np.arange(N), np.arange(s)) / N).sum(1)
    rhs = np.tile(np.fft.fft2(x), (1, 1, s, s)) * hold(Hs)[:, None] * hold(Ws)[None, :]
    np.testing.assert_allclose(np.fft.fft2(O.nearest(x, s)), rhs, atol=1e-10)


# -------------------------------------------------------------------------------- a7 (I3)
@pytest.mark.parametrize("k,shape", [(3, (8, 9)), (4, (10, 12)), (5, (13, 11)), (2, (6, 6)), (7, (14, 15))])
def test_I3_p2o_direct_dft(k, shape):
    psf = _rng("I3", k).random((2, 1, k, k))
    np.testing.assert_allclose(O.p2o(psf, shape), O.otf_direct(psf, shape), atol=1e-12)


# -------------------------------------------------------------------------------- a8-a11
@pytest.mark.parametrize("k", [3, 5])
def test_I4_s1_closed_form(k):
    rng = _rng("I4", k)
    x = rng.standard_normal((1, 2, 10, 11))
    psf = softmax_psf(rng, 2, k).astype(np.float64)
    b = 0.3 * rng.standard_normal((1, 2, 1, 1))
    lmb = 1 / (1 + np.exp(-(b - 9))) + 1e-5
    K = O.otf_direct(psf, (10, 11))
    X = (np.conj(K) + lmb) * np.fft.fft2(x) / (np.abs(K) ** 2 + lmb)
    np.testing.assert_allclose(O.converse2d_op(x, x, psf, b, 1, 1e-5), np.fft.ifft2(X).real, atol=1e-9)


@pytest.mark.parametrize("s,k", itertools.product([1, 2, 3], [2, 3, 5]))
def test_I5_stable_form_equals_reference_order(s, k):
    rng = _rng("I5", s, k)
    x = rng.standard_normal((2, 2, 7, 9))
    x0 = rng.standard_normal((2, 2, 7 * s, 9 * s))
    psf = softmax_psf(rng, 2, k)
    b = 0.5 * rng.standard_normal((1, 2, 1, 1))
    np.testing.assert_allclose(O.converse2d_op(x, x0, psf, b, s, 1e-5),
                               O.converse2d_op_stable(x, x0, psf, b, s, 1e-5), atol=1e-9)


@pytest.mark.parametrize("s,k", itertools.product([1, 2, 3], [2, 3, 5]))
def test_I6_normal_equations(s, k):
    rng = _rng("I6", s, k)
    h, w = 5, 6
    y = rng.standard_normal((h, w))
    x0 = rng.standard_normal((h * s, w * s))
    psf = softmax_psf(rng, 1, k)[0, 0].astype(np.float64)
    b = np.array([[[[0.7]]]])
    lmb = O.lam(b, 1e-5).item()
    brute = O.normal_equation_solve(y, x0, psf, lmb, s)
    got = O.converse2d_op(y[None, None], x0[None, None], psf[None, None], b, s, 1e-5)[0, 0]
    # the reference order divides by lambda ~ 1e-4: compare at fp64 rounding x 1/lambda
    np.testing.assert_allclose(got, brute, atol=1e-7)


@pytest.mark.parametrize("s", [1, 2, 3])
def test_I7_delta_psf(s):
    rng = _rng("I7", s)
    x = rng.standard_normal((1, 2, 9, 8))
    psf = np.zeros((1, 2, 5, 5))
    psf[..., 2, 2] = 1.0
    out = O.converse2d_module(x, psf, np.zeros((1, 2, 1, 1)), s, 2, "circular", 1e-5)
    np.testing.assert_allclose(out, O.nearest(x, s), atol=1e-8)


def test_I8_linearity_and_dc():
    rng = _rng("I8")
    x1, x2 = rng.standard_normal((2, 1, 2, 9, 10))
    psf = softmax_psf(rng, 2, 5).astype(np.float64)
    b = np.zeros((1, 2, 1, 1))
    f = lambda x: O.converse2d_module(x, psf, b, 2, 2, "reflect", 1e-5)
    np.testing.assert_allclose(f(2 * x1 - 3 * x2), 2 * f(x1) - 3 * f(x2), atol=1e-8)
    y = O.pad_nchw(x1, 2, "circular")
    full = O.converse2d_op(y, y, psf, b, 1, 1e-5)
    np.testing.assert_allclose(full.mean(axis=(-2, -1)), y.mean(axis=(-2, -1)), atol=1e-10)


# -------------------------------------------------------------------------------- planted mistakes
def _wrong_roll_op(x, x0, psf, bias, s, eps):
    """Oracle copy with the psf rolled the wrong way (+k/2 instead of -k/2)."""
    orig = O.p2o

    def bad_p2o(p, shape):
        kh, kw = p.shape[-2:]
        otf = np.zeros(p.shape[:-2] + tuple(shape))
        otf[..., :kh, :kw] = p
        return np.fft.fft2(np.roll(otf, (kh // 2, kw // 2), axis=(-2, -1)))
    O.p2o = bad_p2o
    try:
        return O.converse2d_op(x, x0, psf, bias, s, eps)
    finally:
        O.p2o = orig


def _transposed_splits_op(x, x0, psf, bias, s, eps):
    """Oracle copy whose alias-group mean uses the wrong block permutation."""
    orig = O.splits_mean

    def bad(a, s_):
        *lead, W, H = a.shape
        b = a.reshape(*lead, W // s_, s_, H // s_, s_)  # interleaved instead of blocked
        return b.mean(axis=(-3, -1))
    O.splits_mean = bad
    try:
        return O.converse2d_op(x, x0, psf, bias, s, eps)
    finally:
        O.splits_mean = orig


@pytest.mark.parametrize("mutant,s", [(_wrong_roll_op, 1), (_transposed_splits_op, 2)])
def test_planted_mistakes_fail_normal_equations(mutant, s):
    rng = _rng("mut", s)
    y = rng.standard_normal((4, 5))
    x0 = rng.standard_normal((4 * s, 5 * s))
    psf = rng.random((4, 4))  # asymmetric, even-sized: both mistakes are visible
    b = np.array([[[[0.7]]]])
    brute = O.normal_equation_solve(y, x0, psf, O.lam(b, 1e-5).item(), s)
    bad = mutant(y[None, None], x0[None, None], psf[None, None], b, s, 1e-5)[0, 0]
    assert np.abs(bad - brute).max() > 1e-3


# -------------------------------------------------------------------------------- a13/a14
def test_layernorm_cf():
    rng = _rng("ln")
    x = rng.standard_normal((2, 8, 5, 6))
    w, b = rng.standard_normal(8), rng.standard_normal(8)
    ref = F.layer_norm(torch.from_numpy(x).permute(0, 2, 3, 1), (8,), torch.from_numpy(w), torch.from_numpy(b),
                       1e-6).permute(0, 3, 1, 2).numpy()
    np.testing.assert_allclose(O.layernorm_cf(x, w, b, 1e-6), ref, atol=1e-12)
    y = O.layernorm_cf(x, np.ones(8), np.zeros(8), 0.0)
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-12)
    np.testing.assert_allclose((y ** 2).mean(1), 1, atol=1e-12)


def test_conv1x1_and_gelu():
    rng = _rng("cv")
    x = rng.standard_normal((2, 8, 5, 6))
    W, b = rng.standard_normal((4, 8, 1, 1)), rng.standard_normal(4)
    ref = F.conv2d(torch.from_numpy(x), torch.from_numpy(W), torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(O.conv1x1(x, W, b), ref, atol=1e-12)
    np.testing.assert_allclose(O.gelu(x), F.gelu(torch.from_numpy(x)).numpy(), atol=1e-12)
    assert O.gelu(np.array(0.0)) == 0.0
    np.testing.assert_allclose(O.gelu(np.array([10.0, -10.0])), [10.0, 0.0], atol=1e-20)
