"""Transfer-table kernels (the split-DFT form of k_phi_tile) across their edge geometries, through the
module path (util_converse.py:142-192) and the operator path (converse2d.cpp:165-209), against the
fp64 oracle (max-abs <= 1e-4): psf sizes 1 to 48 (one to four 16-row tap groups, odd and even, square
and not), HR sides that are multiples of 16 but not powers of two, rectangular planes, odd LR widths
(the Hermitian column classes at s > 1), column chunks that end part-way, scales 1, 2 and 4,
per-sample and shared psfs."""
import numpy as np
import pytest
import torch

from oracle import converse_oracle as O
from tests.conftest import seeded

pytestmark = pytest.mark.gpu
TOL = 1e-4

# (B, C, H, W, kh, kw, s, pad, psf batch); (H + 2 pad) s is a multiple of 16
MODULE = [
    (2, 3, 44, 36, 1, 1, 1, 2, 1),      # 48 x 40, 1 x 1 psf
    (1, 2, 48, 80, 2, 4, 1, 0, 1),      # even psf sizes
    (2, 2, 92, 60, 17, 17, 1, 2, 2),    # 96 x 64, two tap groups, per-sample psf
    (1, 3, 112, 40, 33, 9, 1, 0, 1),    # three tap groups, non-square psf
    (1, 2, 140, 140, 48, 48, 1, 2, 1),  # 144 x 144 (not a power of two), four tap groups
    (2, 2, 24, 20, 5, 7, 2, 0, 2),      # s = 2: 48 x 40
    (1, 2, 24, 19, 5, 5, 2, 0, 1),      # s = 2, odd LR width (19 column classes, 10 evaluated)
    (1, 3, 28, 36, 16, 16, 2, 2, 1),    # s = 2: 64 x 80, padded
    (2, 2, 16, 12, 25, 25, 4, 0, 2),    # s = 4: 64 x 48, per-sample 25 x 25
    (1, 2, 16, 9, 3, 3, 4, 0, 1),       # s = 4, odd LR width
    (1, 2, 18, 22, 3, 11, 4, 1, 1),     # s = 4: 80 x 96, padded
]


@pytest.mark.parametrize("B,C,H,W,kh,kw,s,p,pb", MODULE)
def test_module_tables_edge_geometries(B, C, H, W, kh, kw, s, p, pb):
    from conversenet_amd import _lib
    from conversenet_amd import functional as Fh
    lib = _lib.load()
    assert lib.cvn_converse2d_route(B, C, H, W, pb, kh, kw, s, p) == _lib.ROUTE_GENERIC
    rng = seeded("tables-module", B, C, H, W, kh, kw, s, p, pb)
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = rng.standard_normal((pb, C, kh * kw))
    w = np.exp(w - w.max(axis=-1, keepdims=True))
    w = (w / w.sum(axis=-1, keepdims=True)).reshape(pb, C, kh, kw).astype(np.float32)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    dev = torch.device("cuda")
    got = Fh.converse2d_fused(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                              torch.from_numpy(b).to(dev).reshape(-1), s, p, "circular", 1e-3,
                              cache=False).cpu().numpy()
    ref = O.converse2d_module(x, w, b, s, p, "circular", 1e-3)
    err = float(np.abs(got - ref).max())
    print(f"module tables B{B} C{C} {H}x{W} psf {kh}x{kw} s{s} p{p} pb{pb}: max-abs {err:.3e}")
    assert err <= TOL


# (B, C, h, w, kh, kw, s) on padded planes, random x0
OP = [(1, 2, 48, 40, 7, 7, 1), (2, 3, 32, 24, 17, 5, 2), (1, 2, 16, 20, 25, 25, 4), (1, 2, 36, 36, 4, 6, 4)]


@pytest.mark.parametrize("B,C,h,w,kh,kw,s", OP)
def test_op_tables_edge_geometries(B, C, h, w, kh, kw, s):
    from conversenet_amd import functional as Fh
    rng = seeded("tables-op", B, C, h, w, kh, kw, s)
    x = rng.standard_normal((B, C, h, w)).astype(np.float32)
    x0 = rng.standard_normal((B, C, h * s, w * s)).astype(np.float32)
    wt = rng.standard_normal((1, C, kh * kw))
    wt = np.exp(wt - wt.max(axis=-1, keepdims=True))
    wt = (wt / wt.sum(axis=-1, keepdims=True)).reshape(1, C, kh, kw).astype(np.float32)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    dev = torch.device("cuda")
    got = Fh.converse2d_op(*(torch.from_numpy(a).to(dev) for a in (x, x0, wt, b)), s, 1e-5,
                           cache=False).cpu().numpy()
    ref = O.converse2d_op(x, x0, wt, b, s, 1e-5)
    err = float(np.abs(got - ref).max())
    print(f"op tables B{B} C{C} {h}x{w} psf {kh}x{kw} s{s}: max-abs {err:.3e}")
    assert err <= TOL
