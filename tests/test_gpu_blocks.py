"""HIP LayerNorm / 1x1 (MFMA) / fused LN-MLP kernels, ConverseBlock, the two models, and full-size
properties of the Converse2D path, all through the library's C ABI, against the fp64 oracle."""
import numpy as np
import pytest
import torch

from oracle import converse_oracle as O
from tests.conftest import seeded, softmax_psf

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
TOL = 1e-4


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _n(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def psnr(a, ref):
    """utils_image.py:626-641 with peak = dynamic range of the reference output."""
    mse = float(np.mean((a.astype(np.float64) - ref) ** 2))
    return 10 * np.log10((ref.max() - ref.min()) ** 2 / mse) if mse > 0 else np.inf


# ------------------------------------------------------------------------------------------------
# a13 LayerNorm (channels first)
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("B,C,H,W,eps", [(2, 64, 32, 40, 1e-6), (1, 128, 16, 18, 1e-5), (3, 5, 7, 9, 1e-5),
                                         (2, 16, 33, 31, 1e-6), (1, 1, 4, 4, 1e-6)])
def test_layernorm_cf(B, C, H, W, eps):
    from conversenet_amd import functional as Fh
    rng = seeded("ln", B, C, H, W)
    x = (3 * rng.standard_normal((B, C, H, W)) + 1).astype(np.float32)
    w = rng.standard_normal(C).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    got = _n(Fh.layernorm_cf(_t(x), _t(w), _t(b), eps))
    ref = O.layernorm_cf(x, w, b, eps)
    assert np.abs(got - ref).max() <= TOL


# ------------------------------------------------------------------------------------------------
# a14 1x1 conv (+ GELU, + residual, + LN prologue) on MFMA, and the generic fallback shapes
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("cin,cout", [(64, 64), (64, 128), (128, 64), (128, 128), (32, 64), (16, 64), (64, 16),
                                      (3, 64), (64, 3), (1, 64), (64, 1)])
@pytest.mark.parametrize("act", [None, "gelu"])
def test_conv1x1(cin, cout, act):
    from conversenet_amd import functional as Fh
    rng = seeded("c11", cin, cout, act)
    B, H, W = 2, 24, 20
    x = rng.standard_normal((B, cin, H, W)).astype(np.float32)
    w = (rng.standard_normal((cout, cin, 1, 1)) / np.sqrt(cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    got = _n(Fh.conv1x1(_t(x), _t(w), _t(b), act=act))
    ref = O.conv1x1(x, w, b)
    if act == "gelu":
        ref = O.gelu(ref)
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("cin,cout", [(1, 64), (64, 1), (3, 64), (64, 3), (2100, 3)])
@pytest.mark.parametrize("HW,res", [((15, 17), False), ((16, 16), True), ((15, 17), True)])
def test_conv1x1_generic_kernel_paths(cin, cout, HW, res):
    """The VALU 1x1 kernel for channel counts without an MFMA tile: four pixels per thread (float4)
    when HW % 4 == 0, one otherwise; with and without a scaled residual; up to 2100 input channels."""
    from conversenet_amd import functional as Fh
    rng = seeded("c11-any", cin, cout, HW, res)
    B = 2
    x = rng.standard_normal((B, cin) + HW).astype(np.float32)
    w = (rng.standard_normal((cout, cin, 1, 1)) / np.sqrt(cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    r = rng.standard_normal((B, cout) + HW).astype(np.float32)
    a = rng.standard_normal(cout).astype(np.float32)
    if res:
        got = _n(Fh.conv1x1(_t(x), _t(w), _t(b), residual=_t(r), res_scale=_t(a)))
        ref = a[None, :, None, None] * O.conv1x1(x, w, b) + r
    else:
        got = _n(Fh.conv1x1(_t(x), _t(w), _t(b), act="gelu"))
        ref = O.gelu(O.conv1x1(x, w, b))
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("HW", [(16, 16), (15, 17)])  # vector (HW % 4 == 0) and scalar paths
def test_conv1x1_residual_scale_and_ln_prologue(HW):
    from conversenet_amd import functional as Fh
    rng = seeded("c11r", HW)
    B, C = 2, 64
    H, W = HW
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    r = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = (rng.standard_normal((C, C, 1, 1)) / 8).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    a = rng.standard_normal(C).astype(np.float32)
    lw, lb = rng.standard_normal(C).astype(np.float32), rng.standard_normal(C).astype(np.float32)
    got = _n(Fh.conv1x1(_t(x), _t(w), _t(b), residual=_t(r), res_scale=_t(a)))
    ref = a[None, :, None, None] * O.conv1x1(x, w, b) + r
    assert np.abs(got - ref).max() <= TOL
    if (H * W) % 4 == 0:
        got = _n(Fh.conv1x1(_t(x), _t(w), _t(b), act="gelu", ln=(_t(lw), _t(lb), 1e-5)))
        ref = O.gelu(O.conv1x1(O.layernorm_cf(x, lw, lb, 1e-5), w, b))
        assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("C,mid", [(64, 128), (32, 64)])
@pytest.mark.parametrize("alpha", [False, True])
def test_ln_mlp_residual(C, mid, alpha):
    """ConverseBlock.conv2 plus its residual in one kernel (util_converse.py:285-292, :321-322)."""
    from conversenet_amd import functional as Fh
    rng = seeded("mlp", C, mid, alpha)
    B, H, W = 2, 20, 24
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    lw, lb = rng.standard_normal(C).astype(np.float32), rng.standard_normal(C).astype(np.float32)
    w1 = (rng.standard_normal((mid, C, 1, 1)) / np.sqrt(C)).astype(np.float32)
    b1 = rng.standard_normal(mid).astype(np.float32)
    w2 = (rng.standard_normal((C, mid, 1, 1)) / np.sqrt(mid)).astype(np.float32)
    b2 = rng.standard_normal(C).astype(np.float32)
    a = rng.standard_normal(C).astype(np.float32) if alpha else None
    got = _n(Fh.ln_mlp_residual(_t(x), _t(lw), _t(lb), 1e-5, _t(w1), _t(b1), _t(w2), _t(b2),
                                res_scale=_t(a) if alpha else None))
    t = O.conv1x1(O.gelu(O.conv1x1(O.layernorm_cf(x, lw, lb, 1e-5), w1, b1)), w2, b2)
    ref = (a[None, :, None, None] * t if alpha else t) + x
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("alpha", [False, True])
@pytest.mark.parametrize("inplace", [False, True])
def test_conv_ln_mlp_residual_tail(alpha, inplace):
    """ConverseBlock tail in one kernel: x + s1 (W0 t + b0), then its LN-MLP branch and residual
    (util_converse.py:279-293, :309-323); against the oracle and the two-kernel sequence."""
    from conversenet_amd import functional as Fh
    rng = seeded("tail", alpha, inplace)
    B, C, Ct, mid, H, W = 2, 64, 128, 128, 20, 26  # 520 pixels: a partial last tile
    t = rng.standard_normal((B, Ct, H, W)).astype(np.float32)
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w0 = (rng.standard_normal((C, Ct, 1, 1)) / np.sqrt(Ct)).astype(np.float32)
    b0 = rng.standard_normal(C).astype(np.float32)
    lw, lb = rng.standard_normal(C).astype(np.float32), rng.standard_normal(C).astype(np.float32)
    w1 = (rng.standard_normal((mid, C, 1, 1)) / np.sqrt(C)).astype(np.float32)
    b1 = rng.standard_normal(mid).astype(np.float32)
    w2 = (rng.standard_normal((C, mid, 1, 1)) / np.sqrt(mid)).astype(np.float32)
    b2 = rng.standard_normal(C).astype(np.float32)
    s1 = rng.standard_normal(C).astype(np.float32) if alpha else None
    s2 = rng.standard_normal(C).astype(np.float32) if alpha else None
    xt = _t(x)
    got = _n(Fh.conv_ln_mlp_residual(_t(t), xt, _t(w0), _t(b0), _t(lw), _t(lb), 1e-5, _t(w1), _t(b1), _t(w2),
                                     _t(b2), _t(s1) if alpha else None, _t(s2) if alpha else None,
                                     out=xt if inplace else None))
    u = O.conv1x1(t, w0, b0)
    y1 = (s1[None, :, None, None] * u if alpha else u) + x
    v = O.conv1x1(O.gelu(O.conv1x1(O.layernorm_cf(y1, lw, lb, 1e-5), w1, b1)), w2, b2)
    ref = (s2[None, :, None, None] * v if alpha else v) + y1
    assert np.abs(got - ref).max() <= TOL
    two = Fh.conv1x1(_t(t), _t(w0), _t(b0), residual=_t(x), res_scale=_t(s1) if alpha else None)
    two = _n(Fh.ln_mlp_residual(two, _t(lw), _t(lb), 1e-5, _t(w1), _t(b1), _t(w2), _t(b2),
                                res_scale=_t(s2) if alpha else None))
    assert np.abs(got - two).max() <= TOL


@pytest.mark.parametrize("scale", [1e-3, 3e5])
def test_tail_split_fp16_range(scale):
    """The tail's 1x1 products run as split fp16 on the matrix cores: tiny activations (fp16 low parts
    below the normal range) keep their accuracy, and activations beyond fp16's range (65504) take the
    fp32 matrix cores for their k-chunk; both against the fp64 oracle, relative to the output scale."""
    from conversenet_amd import functional as Fh
    rng = seeded("tail-range", scale)
    B, C, Ct, mid, H, W = 1, 64, 128, 128, 16, 20
    f = lambda *sh, sc=1.0: (rng.standard_normal(sh) * sc).astype(np.float32)
    t, x = f(B, Ct, H, W, sc=scale), f(B, C, H, W)
    if scale > 1:
        t[:, :, :8] *= 1e-5  # mixed: half the pixels in fp16 range, half far beyond it
    w0, b0 = f(C, Ct, 1, 1, sc=Ct ** -0.5), f(C)
    lw, lb, w1, b1 = f(C), f(C), f(mid, C, 1, 1, sc=C ** -0.5), f(mid)
    w2, b2 = f(C, mid, 1, 1, sc=mid ** -0.5), f(C)
    got = _n(Fh.conv_ln_mlp_residual(_t(t), _t(x), _t(w0), _t(b0), _t(lw), _t(lb), 1e-5, _t(w1), _t(b1), _t(w2),
                                     _t(b2), None, None))
    y1 = O.conv1x1(t, w0, b0) + x
    ref = O.conv1x1(O.gelu(O.conv1x1(O.layernorm_cf(y1, lw, lb, 1e-5), w1, b1)), w2, b2) + y1
    err = np.abs(got - ref).max()
    print(f"tail split-fp16 scale {scale:g}: max-abs {err:.3e}, max |ref| {np.abs(ref).max():.3e}")
    assert err <= max(TOL, 2e-6 * np.abs(ref).max())  # fp32 accumulation at |ref| ~ 1e6: ~1e-6 relative


def test_conv_ln_mlp_head_fused():
    """Block tail plus the next block's LN -> 1x1 -> GELU (util_converse.py:278-280) in one kernel."""
    from conversenet_amd import functional as Fh
    rng = seeded("tail-head")
    B, C, Ct, mid, H, W = 2, 64, 128, 128, 18, 30
    f = lambda *sh, sc=1.0: (rng.standard_normal(sh) * sc).astype(np.float32)
    t, x = f(B, Ct, H, W), f(B, C, H, W)
    w0, b0 = f(C, Ct, 1, 1, sc=Ct ** -0.5), f(C)
    lw, lb, w1, b1 = f(C), f(C), f(mid, C, 1, 1, sc=C ** -0.5), f(mid)
    w2, b2, s1, s2 = f(C, mid, 1, 1, sc=mid ** -0.5), f(C), f(C), f(C)
    hlw, hlb, wh, bh = f(C), f(C), f(Ct, C, 1, 1, sc=C ** -0.5), f(Ct)
    xt = _t(x)
    y, tn = Fh.conv_ln_mlp_residual(_t(t), xt, _t(w0), _t(b0), _t(lw), _t(lb), 1e-5, _t(w1), _t(b1), _t(w2),
                                    _t(b2), _t(s1), _t(s2), out=xt, head=(_t(hlw), _t(hlb), 1e-6, _t(wh), _t(bh)))
    y1 = s1[None, :, None, None] * O.conv1x1(t, w0, b0) + x
    ref = s2[None, :, None, None] * O.conv1x1(O.gelu(O.conv1x1(O.layernorm_cf(y1, lw, lb, 1e-5), w1, b1)), w2, b2) + y1
    tref = O.gelu(O.conv1x1(O.layernorm_cf(ref, hlw, hlb, 1e-6), wh, bh))
    assert np.abs(_n(y) - ref).max() <= TOL
    assert np.abs(_n(tn) - tref).max() <= TOL


@pytest.mark.parametrize("head", [False, True])
def test_conv_ln_mlp_gelu_on_input(head):
    """t_act='gelu': the tail applies the block's GELU to t as it loads it (the 268 path's Converse2D
    then stores its output without GELU), against the oracle on GELU(t)."""
    from conversenet_amd import functional as Fh
    rng = seeded("tail-gelu-in", head)
    B, C, Ct, mid, H, W = 2, 64, 128, 128, 20, 26
    f = lambda *sh, sc=1.0: (rng.standard_normal(sh) * sc).astype(np.float32)
    t, x = f(B, Ct, H, W, sc=2.0), f(B, C, H, W)
    w0, b0 = f(C, Ct, 1, 1, sc=Ct ** -0.5), f(C)
    lw, lb, w1, b1 = f(C), f(C), f(mid, C, 1, 1, sc=C ** -0.5), f(mid)
    w2, b2, s1, s2 = f(C, mid, 1, 1, sc=mid ** -0.5), f(C), f(C), f(C)
    hlw, hlb, wh, bh = f(C), f(C), f(Ct, C, 1, 1, sc=C ** -0.5), f(Ct)
    hd = (_t(hlw), _t(hlb), 1e-6, _t(wh), _t(bh)) if head else None
    got = Fh.conv_ln_mlp_residual(_t(t), _t(x), _t(w0), _t(b0), _t(lw), _t(lb), 1e-5, _t(w1), _t(b1), _t(w2),
                                  _t(b2), _t(s1), _t(s2), head=hd, t_act="gelu")
    y, tn = got if head else (got, None)
    y1 = s1[None, :, None, None] * O.conv1x1(O.gelu(t), w0, b0) + x
    ref = s2[None, :, None, None] * O.conv1x1(O.gelu(O.conv1x1(O.layernorm_cf(y1, lw, lb, 1e-5), w1, b1)), w2, b2) + y1
    err = np.abs(_n(y) - ref).max()
    print(f"tail with GELU on its input, head {head}: max-abs {err:.3e}")
    assert err <= TOL
    if head:
        tref = O.gelu(O.conv1x1(O.layernorm_cf(ref, hlw, hlb, 1e-6), wh, bh))
        assert np.abs(_n(tn) - tref).max() <= TOL


# ------------------------------------------------------------------------------------------------
# a15 ConverseBlock / ConverseBlockAlphaVariant (fused block path on the GPU)
# ------------------------------------------------------------------------------------------------
def _sd(m):
    return {k: v.detach().double().cpu().numpy() for k, v in m.state_dict().items()}


@pytest.mark.parametrize("alpha", [False, True])
@pytest.mark.parametrize("C,k,p,mode", [(64, 3, 2, "circular"), (32, 5, 2, "replicate"), (64, 7, 6, "circular")])
def test_converse_block(alpha, C, k, p, mode):
    from conversenet_amd import util_converse as U
    torch.manual_seed(11)
    cls = U.ConverseBlockAlphaVariant if alpha else U.ConverseBlock
    blk = cls(C, C, kernel_size=k, padding=p, padding_mode=mode)
    if alpha:
        with torch.no_grad():
            blk.alpha1.normal_(0, 0.5)
            blk.alpha2.normal_(0, 0.5)
    rng = seeded("blk", alpha, C, k, p, mode)
    x = rng.standard_normal((2, C, 36, 40)).astype(np.float32)
    ref = O.converse_block(x, _sd(blk), "", k, 1, p, mode, 1e-5, alpha)
    blk = blk.to(DEV).eval()
    with torch.no_grad():
        got = _n(blk(_t(x)))
    err = np.abs(got - ref).max()
    print(f"block C{C} k{k} {mode} alpha={alpha}: max-abs {err:.3e} psnr {psnr(got, ref):.1f}")
    assert err <= 1e-3 and psnr(got, ref) >= 60


# ------------------------------------------------------------------------------------------------
# a16 / a17 models (reduced spatial size; same layer shapes and channel counts as cfg4 / cfg5)
# ------------------------------------------------------------------------------------------------
def test_converse_dncnn():
    from conversenet_amd.converse_dncnn import ConverseDnCNN
    torch.manual_seed(4)
    m = ConverseDnCNN().eval()
    rng = seeded("dncnn")
    x = (rng.random((2, 1, 48, 56)) + 0.1 * rng.standard_normal((2, 1, 48, 56))).astype(np.float32)
    ref = O.converse_dncnn(x, _sd(m))
    with torch.no_grad():
        got = _n(m.to(DEV)(_t(x)))
    print(f"ConverseDnCNN psnr {psnr(got, ref):.1f} dB")
    assert psnr(got, ref) >= 60


def test_converse_usrnet():
    from conversenet_amd.converse_usrnet import ConverseUSRNet
    torch.manual_seed(5)
    m = ConverseUSRNet().eval()
    with torch.no_grad():
        for p in (m.d.alpha, *[b.alpha1 for b in m.p.m_body], *[b.alpha2 for b in m.p.m_body]):
            p.normal_(0, 0.1)
    rng = seeded("usrnet")
    x = rng.random((2, 3, 12, 12)).astype(np.float32)
    k = rng.random((2, 1, 7, 7)).astype(np.float32)
    k /= k.sum(axis=(2, 3), keepdims=True)
    ref = O.converse_usrnet(x, k, 4, _sd(m), 7)
    with torch.no_grad():
        got = _n(m.to(DEV)(_t(x), _t(k), 4))
    print(f"ConverseUSRNet psnr {psnr(got, ref):.1f} dB")
    assert psnr(got, ref) >= 60


def test_converse_msrresnet():
    """ConverseMSRResNet (models/converse_srresnet.py:50-82) at its default width and depth: replicate
    k5 p4 ConverseBlocks and the k2 s2 p2 replicate upsamplers (eps 1e-3) on HIP."""
    from conversenet_amd.converse_srresnet import ConverseMSRResNet
    torch.manual_seed(6)
    m = ConverseMSRResNet().eval()
    with torch.no_grad():
        for mod in (m.up1, m.up2):
            mod.bias.normal_(0, 0.5)
    rng = seeded("msrresnet")
    x = rng.random((1, 3, 16, 18)).astype(np.float32)
    ref = O.converse_msrresnet(x, _sd(m))
    with torch.no_grad():
        got = _n(m.to(DEV)(_t(x)))
    print(f"ConverseMSRResNet psnr {psnr(got, ref):.1f} dB")
    assert psnr(got, ref) >= 60


def test_converse_up_msrresnet():
    from conversenet_amd.converse_srresnet import ConverseUpMSRResNet
    torch.manual_seed(7)
    m = ConverseUpMSRResNet(num_blocks=4).eval()
    rng = seeded("upmsrresnet")
    x = rng.random((2, 3, 12, 12)).astype(np.float32)
    ref = O.converse_up_msrresnet(x, _sd(m), 4)
    with torch.no_grad():
        got = _n(m.to(DEV)(_t(x)))
    print(f"ConverseUpMSRResNet psnr {psnr(got, ref):.1f} dB")
    assert psnr(got, ref) >= 60


# ------------------------------------------------------------------------------------------------
# Full cfg3 size (B16 C64 256^2 k5 p2 circular): oracle on a plane sample, plus size-free identities
# ------------------------------------------------------------------------------------------------
def _cfg3():
    g0 = torch.Generator().manual_seed(0)
    x = torch.randn(16, 64, 256, 256, generator=g0)
    g1 = torch.Generator().manual_seed(1)
    w = torch.softmax(torch.randn(1, 64, 25, generator=g1), dim=-1).reshape(1, 64, 5, 5)
    return x, w


def test_cfg3_full_size_planes_vs_oracle():
    from conversenet_amd import functional as Fh
    x, w = _cfg3()
    b = torch.zeros(64)
    got = Fh.converse2d_fused(x.to(DEV), w.to(DEV), b.to(DEV), 1, 2, "circular", 1e-5)
    torch.cuda.synchronize()
    # one plane per channel, batch index cycling, so every channel's table and every batch slot is hit
    idx = [(c % 16, c) for c in range(64)]
    xs = np.stack([x[bb, c].numpy() for bb, c in idx])[None]          # (1, 64, 256, 256)
    ws = np.stack([w[0, c].numpy() for _, c in idx])[None]
    ref = O.converse2d_module(xs, ws, np.zeros((1, 64, 1, 1), np.float32), 1, 2, "circular", 1e-5)
    g = np.stack([got[bb, c].cpu().numpy() for bb, c in idx])[None]
    err = np.abs(g - ref).max()
    print(f"cfg3 64-plane sample: max-abs {err:.3e}")
    assert err <= TOL


def test_cfg3_full_size_layernorm_and_conv1x1_gelu_vs_oracle():
    """The rest of the cfg3 workload at its full shape (B16 C64 256x256): channels-first LayerNorm
    (eps 1e-6, non-trivial affine) and the 1x1 conv 64 -> 64 + GELU on its output, each against the
    fp64 oracle on the same inputs."""
    from conversenet_amd import functional as Fh
    x, _ = _cfg3()
    g = torch.Generator().manual_seed(5)
    lw, lb = 1 + 0.1 * torch.randn(64, generator=g), 0.1 * torch.randn(64, generator=g)
    cw, cb = torch.randn(64, 64, 1, 1, generator=g) / 8, 0.1 * torch.randn(64, generator=g)
    xd = x.to(DEV)
    ln = Fh.layernorm_cf(xd, lw.to(DEV), lb.to(DEV), 1e-6)
    y = Fh.conv1x1(ln, cw.to(DEV), cb.to(DEV), act="gelu")
    torch.cuda.synchronize()
    ln_ref = O.layernorm_cf(x.numpy(), lw.numpy(), lb.numpy(), 1e-6)
    e_ln = float(np.abs(ln.cpu().numpy() - ln_ref).max())
    y_ref = O.gelu(O.conv1x1(ln.cpu().numpy(), cw.numpy(), cb.numpy()))  # same input as the kernel saw
    e_y = float(np.abs(y.cpu().numpy() - y_ref).max())
    print(f"cfg3 LayerNorm max-abs {e_ln:.3e}, 1x1+GELU max-abs {e_y:.3e}")
    assert e_ln <= TOL and e_y <= TOL


def test_cfg3_full_size_linearity_and_identity():
    """The solve is linear in x for fixed psf and bias; a centred delta psf makes it the identity
    (K = 1, so (conj K + lambda) / (|K|^2 + lambda) = 1)."""
    from conversenet_amd import functional as Fh
    x, w = _cfg3()
    b = torch.zeros(64, device=DEV)
    x1 = x.to(DEV)
    x2 = torch.roll(x1, shifts=(3, 5), dims=(2, 3)).flip(0)
    w = w.to(DEV)
    f = lambda t: Fh.converse2d_fused(t, w, b, 1, 2, "circular", 1e-5)
    lhs = f(0.75 * x1 - 1.5 * x2)
    rhs = 0.75 * f(x1) - 1.5 * f(x2)
    # each of the three evaluations is within 1e-4 of its exact value: 1e-4 (1 + 0.75 + 1.5) bounds the gap
    assert float((lhs - rhs).abs().max()) <= 3.25e-4
    delta = torch.zeros(1, 64, 5, 5, device=DEV)
    delta[..., 2, 2] = 1.0
    y = Fh.converse2d_fused(x1, delta, b, 1, 2, "circular", 1e-5)
    assert float((y - x1).abs().max()) <= 5e-5


# ------------------------------------------------------------------------------------------------
# Edge cases: empty batch, single channel, ragged shapes, a large plane, non-contiguous input
# ------------------------------------------------------------------------------------------------
def test_empty_batch():
    from conversenet_amd import functional as Fh
    x = torch.zeros(0, 4, 16, 16, device=DEV)
    w = torch.full((1, 4, 3, 3), 1 / 9, device=DEV)
    y = Fh.converse2d_fused(x, w, torch.zeros(4, device=DEV), 2, 1, "circular", 1e-5)
    assert tuple(y.shape) == (0, 4, 32, 32)
    y = torch.ops.converse2d.forward(x, torch.zeros(0, 4, 16, 16, device=DEV), w, torch.zeros(1, 4, 1, 1, device=DEV),
                                     1, 1e-5)
    assert tuple(y.shape) == (0, 4, 16, 16)


@pytest.mark.parametrize("B,C,H,W,k,s,p,mode", [(1, 1, 1, 1, 1, 1, 0, "circular"),
                                                 (1, 1, 3, 50, 3, 2, 1, "reflect"),
                                                 (2, 3, 37, 1, 1, 3, 0, "replicate"),
                                                 (1, 1, 1000, 1000, 5, 1, 2, "circular"),
                                                 (1, 2, 61, 67, 6, 2, 3, "constant")])
def test_ragged_and_large(B, C, H, W, k, s, p, mode):
    from conversenet_amd import functional as Fh
    rng = seeded("rag", B, C, H, W, k, s, p, mode)
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    got = _n(Fh.converse2d_fused(_t(x), _t(w), _t(b).reshape(-1), s, p, mode, 1e-5))
    ref = O.converse2d_module(x, w, b, s, p, mode, 1e-5)
    assert np.abs(got - ref).max() <= TOL


def test_module_non_contiguous_input():
    from conversenet_amd.util_converse import Converse2D
    torch.manual_seed(6)
    m = Converse2D(8, 8, 5, scale=1, padding=2).to(DEV)
    base = torch.randn(2, 16, 40, 36, device=DEV)
    x = base[:, ::2]  # channel-strided view
    with torch.no_grad():
        got = _n(m(x))
    ref = O.converse2d_module(x.cpu().numpy(), m.weight.detach().cpu().numpy(), m.bias.detach().cpu().numpy(), 1,
                              2, "circular", 1e-5)
    assert np.abs(got - ref).max() <= TOL


def test_block_chain_matches_block_by_block():
    """run_blocks (each tail kernel also computing the next block's head) against the same blocks
    called one by one, and against the fp64 oracle, for a chain of alpha-variant blocks."""
    from conversenet_amd import util_converse as U
    torch.manual_seed(21)
    blocks = [U.ConverseBlockAlphaVariant(64, 64, kernel_size=3, padding=2, padding_mode="circular")
              for _ in range(3)]
    with torch.no_grad():
        for b in blocks:
            b.alpha1.normal_(0, 0.5)
            b.alpha2.normal_(0, 0.5)
    rng = seeded("chain")
    x = rng.standard_normal((2, 64, 28, 36)).astype(np.float32)
    ref = x.astype(np.float64)
    for b in blocks:
        ref = O.converse_block(ref, _sd(b), "", 3, 1, 2, "circular", 1e-5, True)
    blocks = [b.to(DEV).eval() for b in blocks]
    with torch.no_grad():
        chain = _n(U.run_blocks(blocks, _t(x)))
        one = _t(x)
        for b in blocks:
            one = b(one)
        one = _n(one)
    assert np.abs(chain - one).max() <= 1e-4
    assert np.abs(chain - ref).max() <= 1e-3 and psnr(chain, ref) >= 60


class _OracleDnCNN(torch.nn.Module):
    """The fp64 oracle's Converse-DnCNN behind the model call the evaluation loop makes (no
    parameters: the loop then feeds it tensors on the default device, which it reads back to the host)."""

    def __init__(self, sd):
        super().__init__()
        self.sd = sd

    def forward(self, x):
        return torch.from_numpy(O.converse_dncnn(x.detach().cpu().numpy(), self.sd)).to(x.device)


class _Recorder(torch.nn.Module):
    """Passes the call through and keeps each float output (the loop itself keeps only uint8 images)."""

    def __init__(self, model):
        super().__init__()
        self.model = model
        self.outs = []

    def forward(self, x):
        y = self.model(x)
        self.outs.append(y.detach().double().cpu().numpy())
        return y


def test_evaluate_dncnn_loop_on_hip_matches_oracle(tmp_path):
    """The evaluation loop (main_test_converse_dncnn.py:110-171: noisy image -> model -> uint8 ->
    PSNR / SSIM) through the HIP model against the same loop through the fp64 oracle's Converse-DnCNN
    (random-init weights, two synthetic 64x64 gray images).  The model outputs agree to >= 60 dB PSNR
    (the full-model gate) and max-abs <= 2e-4 (0.05 of a uint8 level); the uint8 images may differ by one
    level only where the oracle's value lies within 0.05 levels of a rounding boundary; PSNR and SSIM
    follow."""
    from PIL import Image
    from conversenet_amd import evaluate as E
    from conversenet_amd.converse_dncnn import ConverseDnCNN
    rng = seeded("eval")
    yy, xx = np.mgrid[0:64, 0:64]
    for name, (fx, fy) in (("a.png", (5.0, 7.0)), ("b.png", (3.0, 11.0))):
        img = (127 + 60 * np.sin(xx / fx) * np.cos(yy / fy) + rng.normal(0, 5, (64, 64))).clip(0, 255)
        Image.fromarray(img.astype(np.uint8)).save(str(tmp_path / name))
    paths = E.get_image_paths(str(tmp_path))
    torch.manual_seed(5)
    m = ConverseDnCNN().eval()
    for p in m.parameters():
        p.requires_grad_(False)
    oracle = _Recorder(_OracleDnCNN(_sd(m)))
    hip = _Recorder(m.to(DEV))
    out_h, out_o = tmp_path / "hip", tmp_path / "oracle"
    out_h.mkdir()
    out_o.mkdir()
    res_h = E.eval_dncnn(paths, hip, 25, str(out_h))
    res_o = E.eval_dncnn(paths, oracle, 25, str(out_o))
    for (n_h, p_h, s_h), (n_o, p_o, s_o), fh, fo in zip(res_h, res_o, hip.outs, oracle.outs):
        assert n_h == n_o
        err = float(np.abs(fh - fo).max())
        ih = np.asarray(Image.open(str(out_h / n_h)), dtype=np.int16)
        io = np.asarray(Image.open(str(out_o / n_o)), dtype=np.int16)
        lv = np.clip(fo.squeeze(), 0, 1) * 255.0
        near = np.abs(lv - np.floor(lv) - 0.5) < 0.05  # within 0.05 levels of a rounding boundary
        diff = np.abs(ih - io)
        print(f"eval {n_h}: output max-abs {err:.2e}; PSNR HIP {p_h:.4f} / oracle {p_o:.4f} dB, SSIM {s_h:.5f} / "
              f"{s_o:.5f}; pixels off by one level {int((diff > 0).sum())} ({int(near.sum())} near a boundary); "
              f"model output PSNR {psnr(fh, fo):.1f} dB")
        assert psnr(fh, fo) >= 60 and err <= 2e-4
        assert diff.max() <= 1 and not np.any((diff > 0) & ~near)
        assert abs(p_h - p_o) < 0.01 and abs(s_h - s_o) < 1e-3
