"""HIP backward of the module path (cvn_converse2d_bwd_f32 and the autograd Function built on it)
against the fp64 oracle backward (oracle.converse_oracle.converse2d_module_backward, itself pinned
against torch autograd of the reference op sequence and finite differences)."""
import numpy as np
import pytest
import torch

from oracle import converse_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

CASES = [
    # (B, C, H, W, k, s, p, mode, psf_batch)
    (2, 3, 16, 18, 3, 1, 2, "circular", 1),
    (2, 2, 20, 17, 5, 1, 2, "reflect", 1),
    (2, 2, 15, 16, 4, 1, 3, "replicate", 1),
    (1, 3, 18, 18, 2, 1, 1, "constant", 1),
    (2, 3, 12, 14, 3, 2, 1, "circular", 1),
    (2, 2, 10, 12, 5, 3, 2, "reflect", 1),
    (2, 2, 8, 9, 7, 4, 0, "circular", 2),
    (3, 2, 16, 16, 5, 1, 2, "circular", 3),
    (2, 3, 256, 256, 5, 1, 2, "circular", 1),   # cfg3 plane size (260^2)
    (1, 2, 256, 256, 7, 1, 6, "circular", 1),   # cfg4 plane size (268^2)
    (2, 2, 64, 64, 25, 4, 0, "circular", 2),    # ConvReverseDataNet data step (per-sample 25x25 psf)
    (1, 2, 24, 26, 3, 1, 20, "replicate", 1),   # wide replicate border: many samples fold onto the edge
    (1, 2, 21, 19, 5, 2, 9, "reflect", 1),
]


def _inputs(B, C, H, W, k, s, pb, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = rng.random((pb, C, k, k)).astype(np.float32)
    w /= w.sum(axis=(2, 3), keepdims=True)
    b = (0.5 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    g = rng.standard_normal((B, C, H * s, W * s)).astype(np.float32)
    return x, w, b, g


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _close(got, ref, rel, what):
    err = float(np.abs(got - ref).max())
    scale = max(1.0, float(np.abs(ref).max()))
    print(f"{what}: max-abs {err:.3e} (|ref| max {scale:.3e})")
    assert err <= rel * scale, what


@pytest.mark.parametrize("B,C,H,W,k,s,p,mode,pb", CASES)
def test_backward_vs_oracle(B, C, H, W, k, s, p, mode, pb):
    from conversenet_amd import functional as Fh
    x, w, b, g = _inputs(B, C, H, W, k, s, pb, 17 + H + k + s)
    eps = 1e-3 if pb > 1 else 1e-5
    gx, gw, gb = Fh.converse2d_backward(_t(g), _t(x), _t(w), _t(b), s, p, mode, eps)
    torch.cuda.synchronize()
    rx, rw, rb = O.converse2d_module_backward(x, w, b, g, s, p, mode, eps)
    _close(gx.cpu().numpy(), rx, 1e-4, "grad_x")
    _close(gw.cpu().numpy(), rw, 2e-4, "grad_weight")
    _close(gb.cpu().numpy(), rb, 2e-4, "grad_bias")


def test_backward_x_only_and_weights_only():
    from conversenet_amd import functional as Fh
    x, w, b, g = _inputs(2, 3, 20, 22, 5, 2, 1, 3)
    rx, rw, rb = O.converse2d_module_backward(x, w, b, g, 2, 2, "reflect", 1e-5)
    gx, gw, gb = Fh.converse2d_backward(_t(g), _t(x), _t(w), _t(b), 2, 2, "reflect", 1e-5, True, False, False)
    assert gw is None and gb is None
    _close(gx.cpu().numpy(), rx, 1e-4, "grad_x only")
    gx, gw, gb = Fh.converse2d_backward(_t(g), _t(x), _t(w), _t(b), 2, 2, "reflect", 1e-5, False, True, True)
    assert gx is None
    _close(gw.cpu().numpy(), rw, 2e-4, "grad_weight only")
    _close(gb.cpu().numpy(), rb, 2e-4, "grad_bias only")


@pytest.mark.parametrize("need", [(True, False, False), (False, True, True)])
def test_backward_partial_scale1(need):
    """Scale 1, the column pass's register path: grad_x alone (no input column transforms, no dPhi)
    and the weight gradients alone."""
    from conversenet_amd import functional as Fh
    x, w, b, g = _inputs(2, 3, 30, 26, 5, 1, 1, 5)
    rx, rw, rb = O.converse2d_module_backward(x, w, b, g, 1, 2, "circular", 1e-5)
    gx, gw, gb = Fh.converse2d_backward(_t(g), _t(x), _t(w), _t(b), 1, 2, "circular", 1e-5, *need)
    if need[0]:
        assert gw is None and gb is None
        _close(gx.cpu().numpy(), rx, 1e-4, "grad_x only")
    else:
        assert gx is None
        _close(gw.cpu().numpy(), rw, 2e-4, "grad_weight only")
        _close(gb.cpu().numpy(), rb, 2e-4, "grad_bias only")


CT_CASES = [
    # (B, C, H, W, k, p, mode, psf_batch, need): scale 1 on the column lengths with a compile-time plan
    (3, 2, 128, 128, 5, 2, "circular", 1, (True, True, True)),    # 132: three planes per column block
    (4, 1, 252, 252, 5, 2, "reflect", 1, (True, False, False)),   # 256, grad_x only (no input columns)
    (3, 2, 256, 256, 3, 2, "circular", 1, (False, True, True)),   # 260, weight gradients only
    (2, 2, 256, 256, 5, 0, "circular", 2, (True, True, True)),    # 256, one plane per block (per-sample psf)
]


@pytest.mark.parametrize("B,C,H,W,k,p,mode,pb,need", CT_CASES)
def test_backward_compile_time_columns(B, C, H, W, k, p, mode, pb, need):
    """The column pass at 132, 256 and 260 points, whose blocks copy each plane's columns into LDS
    asynchronously while the previous plane is transformed: several planes per block, with and
    without the input columns of the weight gradients, and one plane per block."""
    from conversenet_amd import functional as Fh
    x, w, b, g = _inputs(B, C, H, W, k, 1, pb, 29 + H + k)
    eps = 1e-3 if pb > 1 else 1e-5
    rx, rw, rb = O.converse2d_module_backward(x, w, b, g, 1, p, mode, eps)
    gx, gw, gb = Fh.converse2d_backward(_t(g), _t(x), _t(w), _t(b), 1, p, mode, eps, *need)
    torch.cuda.synchronize()
    if need[0]:
        _close(gx.cpu().numpy(), rx, 1e-4, "grad_x")
    if need[1]:
        _close(gw.cpu().numpy(), rw, 2e-4, "grad_weight")
        _close(gb.cpu().numpy(), rb, 2e-4, "grad_bias")


def test_backward_scale1_plane_past_register_path():
    """A 2100-sample padded side at scale 1: one column class per block holds 2100 elements, more than
    the 4 x 512 register slots, so the column pass reads conj(Phi') per element instead.  grad_x only:
    the weight gradient's own transfer-function pass does not take planes this large."""
    from conversenet_amd import functional as Fh
    x, w, b, g = _inputs(1, 1, 2096, 2096, 3, 1, 1, 11)
    rx, _, _ = O.converse2d_module_backward(x, w, b, g, 1, 2, "circular", 1e-5)
    gx, gw, gb = Fh.converse2d_backward(_t(g), _t(x), _t(w), _t(b), 1, 2, "circular", 1e-5, True, False, False)
    torch.cuda.synchronize()
    assert gw is None and gb is None
    _close(gx.cpu().numpy(), rx, 1e-4, "grad_x")


def test_autograd_through_module():
    """Converse2D on HIP tensors that require grad runs the library's forward and backward; loss.backward()
    fills x.grad, weight.grad and bias.grad as the oracle says."""
    from conversenet_amd.util_converse import Converse2D
    torch.manual_seed(0)
    m = Converse2D(3, 3, 5, scale=1, padding=2, padding_mode="circular").to(DEV)
    with torch.no_grad():
        m.bias.copy_(0.3 * torch.randn(1, 3, 1, 1))
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 3, 24, 20)).astype(np.float32)
    g = rng.standard_normal((2, 3, 24, 20)).astype(np.float32)
    xt = _t(x).requires_grad_(True)
    out = m(xt)
    (out * _t(g)).sum().backward()
    rx, rw, rb = O.converse2d_module_backward(x, m.weight.detach().cpu().numpy(), m.bias.detach().cpu().numpy(), g,
                                              1, 2, "circular", 1e-5)
    _close(xt.grad.cpu().numpy(), rx, 1e-4, "x.grad")
    _close(m.weight.grad.cpu().numpy(), rw, 2e-4, "weight.grad")
    _close(m.bias.grad.cpu().numpy(), rb, 2e-4, "bias.grad")
