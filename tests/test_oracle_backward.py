"""Pins the oracle's module-path backward (oracle.converse_oracle.converse2d_module_backward):
against torch autograd in fp64 of the reference op sequence restated in torch (the reference gets
its gradients the same way: converse2d.cpp:223-227 registers the op CompositeImplicitAutograd), and
against central finite differences of the oracle forward."""
import numpy as np
import pytest
import torch

from conversenet_amd import composite
from oracle import converse_oracle as O

CASES = [
    # (s, mode, k, p, psf_batch, H, W)
    (1, "circular", 3, 2, 1, 7, 6),
    (1, "constant", 4, 2, 2, 6, 7),
    (1, "reflect", 5, 2, 1, 8, 9),
    (2, "reflect", 3, 1, 1, 7, 6),
    (2, "circular", 5, 2, 2, 6, 6),
    (3, "replicate", 3, 1, 1, 5, 7),
    (3, "reflect", 4, 2, 1, 6, 5),
    (4, "circular", 7, 0, 2, 5, 6),
    (2, "replicate", 2, 1, 2, 6, 6),
]


def _inputs(rng, s, k, pb, H, W, B=2, C=3):
    x = rng.standard_normal((B, C, H, W))
    w = rng.random((pb, C, k, k))
    w /= w.sum(axis=(2, 3), keepdims=True)
    b = 0.5 * rng.standard_normal((1, C, 1, 1))
    g = rng.standard_normal((B, C, H * s, W * s))
    return x, w, b, g


@pytest.mark.parametrize("s,mode,k,p,pb,H,W", CASES)
def test_backward_matches_torch_autograd_fp64(s, mode, k, p, pb, H, W):
    rng = np.random.default_rng(100 + 7 * s + k)
    x, w, b, g = _inputs(rng, s, k, pb, H, W)
    xt, wt, bt = (torch.tensor(a, requires_grad=True) for a in (x, w, b))
    out = composite.converse2d_module(xt, wt, bt, s, p, mode, 1e-3)
    (out * torch.tensor(g)).sum().backward()
    dx, dw, db = O.converse2d_module_backward(x, w, b, g, s, p, mode, 1e-3)
    for mine, ref in ((dx, xt.grad), (dw, wt.grad), (db, bt.grad)):
        ref = ref.numpy()
        assert np.abs(mine - ref).max() <= 1e-10 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("s,mode,k,p,pb,H,W", CASES[:5])
def test_backward_matches_finite_differences(s, mode, k, p, pb, H, W):
    rng = np.random.default_rng(200 + s + k)
    x, w, b, g = _inputs(rng, s, k, pb, H, W, B=2, C=2)
    dx, dw, db = O.converse2d_module_backward(x, w, b, g, s, p, mode, 1e-2)

    def loss(x_, w_, b_):
        return float((O.converse2d_module(x_, w_, b_, s, p, mode, 1e-2) * g).sum())

    e = 1e-6
    for which, arr, grad in ((0, x, dx), (1, w, dw), (2, b, db)):
        for _ in range(4):
            idx = tuple(int(rng.integers(0, n)) for n in arr.shape)
            a1, a2 = arr.copy(), arr.copy()
            a1[idx] += e
            a2[idx] -= e
            args1, args2 = [x, w, b], [x, w, b]
            args1[which], args2[which] = a1, a2
            fd = (loss(*args1) - loss(*args2)) / (2 * e)
            assert abs(fd - grad[idx]) <= 1e-5 * max(1.0, abs(grad[idx]))


def test_pad_adjoint_is_the_transpose_of_padding():
    rng = np.random.default_rng(5)
    for mode in O.PAD_MODES:
        for p in (1, 2, 3):
            x = rng.standard_normal((2, 5, 6))
            dy = rng.standard_normal((2, 5 + 2 * p, 6 + 2 * p))
            lhs = (O.pad_nchw(x, p, mode) * dy).sum()
            rhs = (x * O.pad_adjoint(dy, p, mode, 5, 6)).sum()
            assert abs(lhs - rhs) <= 1e-12 * max(1.0, abs(lhs))
