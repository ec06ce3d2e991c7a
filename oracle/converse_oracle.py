"""CPU oracle for the Converse2D forward path -- TEST INFRASTRUCTURE ONLY.

This module is a numpy/scipy restatement of the reference ConverseNet algorithms.  It is imported
only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg, and only as the
checker.  The product (``conversenet_amd``) never imports it.

Every function cites the reference file:line it restates (paths relative to the reference
repository root).  All functions take numpy arrays (NCHW) and a ``dtype`` selecting the evaluation
precision: ``np.float64`` (the parity truth: the reference op sequence evaluated in fp64 on the same
fp32 inputs) or ``np.float32`` (the reference's own fp32 rounding behaviour, reproduced up to FFT
implementation differences).

How each function is pinned (checked by tests/test_oracle.py and tests/test_oracle_ref.py):
  pad_nchw            F.pad index maps (closed forms) + the compiled reference op's inputs
  upsample_zero       closed form I1 (tiled spectrum)
  nearest             closed form I2 (nearest-hold spectrum)
  p2o                 closed form I3 (direct DFT of the taps)
  converse2d_op       the reference's own compiled C++ op (oracle/_ref, fp64 and fp32), I4, I6, I7
  converse2d_module   the compiled reference op + F.pad + crop; I6 normal equations; I7; I8
  converse2d_op_stable   algebraic identity I5 against converse2d_op in fp64
  converse2d_module_backward   central finite differences of converse2d_module in fp64, and torch
                      autograd (fp64) of the reference op sequence restated in torch
  layernorm_cf        zero mean / unit biased variance closed form; torch F.layer_norm
  conv1x1, gelu       einsum definition; erf special values; torch F.conv2d / F.gelu
  converse_block, converse_dncnn, conv_reverse_datanet, kernelnet, converse_usrnet, converse_net,
  converse_msrresnet, converse_up_msrresnet
                      outputs of the reference's own model classes (imported in the build
                      container by tests/golden/make_model_golden.py) on seeded state dicts:
                      tests/test_oracle_models.py, with planted mistakes that must fail
  conv3x3, bilinear_upsample
                      torch F.conv2d / F.interpolate(bilinear) on the CPU
"""
from __future__ import annotations

import math
import os
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np
from scipy import fft as sfft
from scipy import special as sspecial

# Host threads for the large cases (the model-size checks): independent planes, or independent rows
# of pixels, are evaluated on a thread pool with the same per-element arithmetic as a serial call.
_WORKERS = max(1, min(16, os.cpu_count() or 1))
_POOL = None
_TLS = threading.local()


def _pool():
    global _POOL
    if _POOL is None:
        _POOL = ThreadPoolExecutor(_WORKERS)
    return _POOL


def _parallel_ok(size):
    return _WORKERS > 1 and size >= (1 << 20) and not getattr(_TLS, "inside", False)


def _in_worker(fn):
    def run(*a):
        _TLS.inside = True
        try:
            return fn(*a)
        finally:
            _TLS.inside = False
    return run


def _rows_map(fn, x):
    """fn applied to row blocks of a (B,C,H,W) array and concatenated; fn must act per pixel."""
    if x.ndim != 4 or x.shape[2] < 2 or not _parallel_ok(x.size):
        return fn(x)
    parts = np.array_split(x, min(x.shape[2], 2 * _WORKERS), axis=2)
    return np.concatenate(list(_pool().map(_in_worker(fn), parts)), axis=2)

PAD_MODES = ("constant", "reflect", "replicate", "circular")


def _cdtype(dtype):
    return np.complex128 if np.dtype(dtype) == np.float64 else np.complex64


def _fft_workers(workers):
    return workers or (1 if getattr(_TLS, "inside", False) else _WORKERS)


def fft2(a, workers=None):
    return sfft.fftn(a, axes=(-2, -1), workers=_fft_workers(workers))


def ifft2(a, workers=None):
    return sfft.ifftn(a, axes=(-2, -1), workers=_fft_workers(workers))


# ------------------------------------------------------------------------------------------------
# a2: padding -- models/util_converse.py:144-145 (F.pad(x, [p]*4, mode, value=0))
# ------------------------------------------------------------------------------------------------
def pad_index(i, n, p, mode):
    """Source index in [0, n) for padded index i in [0, n + 2p), or -1 for a zero (constant mode).

    Textbook F.pad index maps: circular (i-p) mod n; reflect mirrors about the edge sample without
    repeating it; replicate clamps; constant yields zero outside.
    """
    j = i - p
    if 0 <= j < n:
        return j
    if mode == "constant":
        return -1
    if mode == "circular":
        return j % n
    if mode == "replicate":
        return 0 if j < 0 else n - 1
    if mode == "reflect":
        if j < 0:
            return -j
        return 2 * (n - 1) - j
    raise ValueError(mode)


def pad_nchw(x, p, mode):
    """F.pad over the last two dims with pad p on every side (util_converse.py:145)."""
    if p == 0:
        return x.copy()
    if mode not in PAD_MODES:
        raise ValueError(mode)
    H, W = x.shape[-2:]
    if mode == "reflect" and (p >= H or p >= W):
        raise ValueError("reflect padding must be < input size")
    if mode == "circular" and (p > H or p > W):
        raise ValueError("circular padding must be <= input size")
    ih = np.array([pad_index(i, H, p, mode) for i in range(H + 2 * p)])
    iw = np.array([pad_index(i, W, p, mode) for i in range(W + 2 * p)])
    out = x[..., np.clip(ih, 0, None)[:, None], np.clip(iw, 0, None)[None, :]]
    if mode == "constant":
        mask = (ih[:, None] >= 0) & (iw[None, :] >= 0)
        out = out * mask
    return out.astype(x.dtype, copy=False)


# ------------------------------------------------------------------------------------------------
# a5/a6/a7: upsample, nearest, p2o
# ------------------------------------------------------------------------------------------------
def upsample_zero(x, s):
    """s-fold zero insertion at offset 0 (util_converse.py:237-245; converse2d.cpp:104-119)."""
    if s == 1:
        return x.copy()
    z = np.zeros(x.shape[:-2] + (x.shape[-2] * s, x.shape[-1] * s), dtype=x.dtype)
    z[..., ::s, ::s] = x
    return z


def nearest(x, s):
    """F.interpolate(scale_factor=s, mode='nearest'): out[i, j] = in[i // s, j // s]
    (util_converse.py:172-173)."""
    if s == 1:
        return x.copy()
    return np.repeat(np.repeat(x, s, axis=-2), s, axis=-1)


def p2o(psf, shape):
    """psf -> OTF (util_converse.py:218-235; converse2d.cpp:80-84): zero-pad the taps at the top-left
    to `shape`, roll by (-int(kh/2), -int(kw/2)), 2-D FFT."""
    kh, kw = psf.shape[-2:]
    otf = np.zeros(psf.shape[:-2] + tuple(shape), dtype=psf.dtype)
    otf[..., :kh, :kw] = psf
    otf = np.roll(otf, (-int(kh / 2), -int(kw / 2)), axis=(-2, -1))
    return fft2(otf)


def splits_mean(a, s):
    """Mean over the s*s frequency blocks (util_converse.py:194-215 + torch.mean(dim=-1);
    converse2d.cpp:121-163): view (..., s, W/s, s, H/s), permute to (..., W/s, H/s, s, s), mean."""
    *lead, W, H = a.shape
    b = a.reshape(*lead, s, W // s, s, H // s)
    nl = len(lead)
    b = b.transpose(*range(nl), nl + 1, nl + 3, nl, nl + 2)
    return b.reshape(*lead, W // s, H // s, s * s).mean(axis=-1)


def lam(bias, eps, dtype=np.float64):
    """lambda = sigmoid(bias - 9) + eps (util_converse.py:147; converse2d.cpp:186)."""
    b = bias.astype(dtype)
    return (1.0 / (1.0 + np.exp(-(b - dtype(9.0))))).astype(dtype) + dtype(eps)


# ------------------------------------------------------------------------------------------------
# a8-a11: the op (x already padded, arbitrary x0, uncropped output)
# ------------------------------------------------------------------------------------------------
def converse2d_op(x, x0, weight, bias, scale, eps, dtype=np.float64):
    """Reference op order (converse2d.cpp:165-209, identical to util_converse.py:170-187).

    x (B,C,h,w) padded input; x0 (B,C,h*s,w*s); weight (1 or B, C, kh, kw); bias (1,C,1,1).
    Returns Re(ifft2(FX)) of shape (B,C,h*s,w*s).
    """
    s = int(scale)
    x = x.astype(dtype)
    x0 = x0.astype(dtype)
    w_ = weight.astype(dtype)
    lmb = lam(bias, eps, dtype)
    h, w = x.shape[-2:]
    STy = upsample_zero(x, s)
    FB = p2o(w_, (h * s, w * s)).astype(_cdtype(dtype))
    FBC = np.conj(FB)
    F2B = (np.abs(FB) ** 2).astype(dtype)
    FBFy = FBC * fft2(STy)
    FR = FBFy + fft2(lmb * x0)
    x1 = FB * FR
    FBR = splits_mean(x1, s)
    invW = splits_mean(F2B, s)
    invWBR = FBR / (invW + lmb)
    FCBinvWBR = FBC * np.tile(invWBR, (1, 1, s, s))
    FX = (FR - FCBinvWBR) / lmb
    return np.real(ifft2(FX)).astype(dtype)


def converse2d_op_stable(x, x0, weight, bias, scale, eps, dtype=np.float64):
    """Cancellation-free algebraic rewrite of converse2d_op (identity I5):

        FX = X0 + conj(K) * (Ytile - M(K X0)) / (M(|K|^2) + lambda)

    where M is the s*s alias-group mean tiled back.  Equal to converse2d_op in exact arithmetic."""
    s = int(scale)
    x = x.astype(dtype)
    x0 = x0.astype(dtype)
    lmb = lam(bias, eps, dtype)
    h, w = x.shape[-2:]
    K = p2o(weight.astype(dtype), (h * s, w * s))
    Y = fft2(x)
    Yt = np.tile(Y, (1, 1, s, s))
    X0 = fft2(x0)
    MK = np.tile(splits_mean(K * X0, s), (1, 1, s, s))
    D = np.tile(splits_mean(np.abs(K) ** 2, s), (1, 1, s, s)) + lmb
    FX = X0 + np.conj(K) * (Yt - MK) / D
    return np.real(ifft2(FX)).astype(dtype)


def converse2d_module(x, weight, bias, scale=1, padding=2, padding_mode="circular", eps=1e-5,
                      dtype=np.float64):
    """Converse2D.forward (util_converse.py:142-192): pad, x0 = nearest(padded), op, crop."""
    s = int(scale)
    C = x.shape[1]
    bias = np.asarray(bias)
    if C > 1 and bias.size == C and _parallel_ok(x.size * s * s):
        # channels are independent planes: evaluate channel slices on the thread pool
        b4 = bias.reshape(1, C, 1, 1)
        slices = [slice(c[0], c[-1] + 1) for c in np.array_split(np.arange(C), min(C, 2 * _WORKERS))]
        job = _in_worker(lambda sl: converse2d_module(x[:, sl], weight[:, sl], b4[:, sl], s, padding, padding_mode,
                                                      eps, dtype))
        return np.concatenate(list(_pool().map(job, slices)), axis=1)
    y = pad_nchw(x, padding, padding_mode) if padding > 0 else x
    x0 = nearest(y, s)
    out = converse2d_op(y, x0, weight, bias, s, eps, dtype)
    if padding > 0:
        ps = padding * s
        out = out[..., ps:-ps, ps:-ps]
    return np.ascontiguousarray(out)


# ------------------------------------------------------------------------------------------------
# Backward of the module path (the reference differentiates util_converse.py:142-192 through torch
# autograd: converse2d.cpp:223-227 registers the op as CompositeImplicitAutograd; gradients are
# compared in test/test_error.py:51-54,73-76).  Explicit spectral adjoint, fp64.
# ------------------------------------------------------------------------------------------------
def hold(s, n):
    """Nearest-hold response H_s(u; n) = sum_{a<s} exp(-2 pi i u a / n) for u in [0, n) (identity I2)."""
    u = np.arange(n)[:, None]
    return np.exp(-2j * np.pi * u * np.arange(s)[None, :] / n).sum(axis=1)


def pad_adjoint(dy, p, mode, H, W):
    """Adjoint of pad_nchw: every padded sample's gradient is added to the source sample it copies
    (constant-mode padding samples are dropped)."""
    if p == 0:
        return dy.copy()
    ih = [pad_index(i, H, p, mode) for i in range(H + 2 * p)]
    iw = [pad_index(i, W, p, mode) for i in range(W + 2 * p)]
    rows = np.zeros(dy.shape[:-2] + (H, dy.shape[-1]), dtype=dy.dtype)
    for i, si in enumerate(ih):
        if si >= 0:
            rows[..., si, :] += dy[..., i, :]
    out = np.zeros(dy.shape[:-2] + (H, W), dtype=dy.dtype)
    for j, sj in enumerate(iw):
        if sj >= 0:
            out[..., sj] += rows[..., j]
    return out


def module_transfer(weight, bias, scale, h, w, eps):
    """The module path's transfer function, in the form the backward differentiates:
    out_full = Re ifft2(Phi * tile_s(fft2(y))) with Phi = Hn + conj(K) g, g = (1 - M(K Hn)) / D,
    D = M(|K|^2) + lambda (M = alias-class mean tiled back; this is the reference solve
    util_converse.py:176-187 with x0 = nearest(y), whose spectrum is Hn tile(Y)).
    Returns (K, Hn, g, D, Phi) with K, g, D, Phi of shape (Pb, C, Hs, Ws)."""
    s = int(scale)
    Hs, Ws = h * s, w * s
    K = p2o(weight.astype(np.float64), (Hs, Ws))
    Hn = hold(s, Hs)[:, None] * hold(s, Ws)[None, :]
    C = weight.shape[1]
    lmb = lam(np.asarray(bias, np.float64).reshape(1, C, 1, 1), eps)

    def mt(a):
        return np.tile(splits_mean(a, s), (1, 1, s, s))

    D = mt(np.abs(K) ** 2) + lmb
    g = (1.0 - mt(K * Hn)) / D
    return K, Hn, g, D, Hn + np.conj(K) * g


def converse2d_module_backward(x, weight, bias, gout, scale=1, padding=2, padding_mode="circular", eps=1e-5):
    """Gradients (dx, dweight, dbias) of sum(gout * converse2d_module(x, weight, bias, ...)), fp64.

    x (B,C,H,W); weight (1 or B, C, kh, kw); bias (1,C,1,1) or (C,); gout (B,C,H*s,W*s).
    Chain: dX = fft2(uncrop(gout)) / (Hs Ws); dx = pad^T(Re F*_{hw}(alias_sum(conj(Phi) dX)));
    dPhi = sum over the samples sharing a psf of conj(tile Y) dX; per alias class, with
    P = sum_m dPhi_m K_m and rho = -Re(conj(P) g) / D:
      dK_m = conj(dPhi_m) g - P conj(Hn_m) / (s^2 D) + 2 rho K_m / s^2,   dlambda = sum rho;
    dweight[i, j] = Re sum_{u,v} dK[u,v] exp(+2 pi i (u (i - kh//2) / Hs + v (j - kw//2) / Ws));
    dbias = dlambda * sigmoid'(bias - 9)."""
    s, p = int(scale), int(padding)
    x = np.asarray(x, np.float64)
    B, C, H, W = x.shape
    y = pad_nchw(x, p, padding_mode) if p > 0 else x
    h, w = y.shape[-2:]
    Hs, Ws = h * s, w * s
    kh, kw = weight.shape[-2:]
    K, Hn, g, D, Phi = module_transfer(weight, bias, s, h, w, eps)
    Gf = np.zeros((B, C, Hs, Ws))
    ps = p * s
    Gf[..., ps:ps + H * s, ps:ps + W * s] = np.asarray(gout, np.float64)
    dX = fft2(Gf) / (Hs * Ws)
    # dx
    dT = np.conj(Phi) * dX
    dY = splits_mean(dT, s) * (s * s)
    dy = np.real(ifft2(dY)) * (h * w)
    dx = pad_adjoint(dy, p, padding_mode, H, W)
    # dPhi (summed over the samples that share a psf)
    T = np.tile(fft2(y), (1, 1, s, s))
    dPhi = np.conj(T) * dX
    if weight.shape[0] == 1:
        dPhi = dPhi.sum(axis=0, keepdims=True)
    Pm = np.tile(splits_mean(dPhi * K, s), (1, 1, s, s)) * (s * s)
    rho = -np.real(np.conj(Pm) * g) / D
    dK = np.conj(dPhi) * g - Pm * np.conj(Hn) / (s * s * D) + 2.0 * rho * K / (s * s)
    dlmb = rho.sum(axis=(-2, -1)) / (s * s)                         # (Pb, C)
    full = ifft2(dK) * (Hs * Ws)                                     # sum dK exp(+...)
    mi = (np.arange(kh) - kh // 2) % Hs
    nj = (np.arange(kw) - kw // 2) % Ws
    dweight = np.real(full[..., mi[:, None], nj[None, :]])
    b = np.asarray(bias, np.float64).reshape(C)
    sig = 1.0 / (1.0 + np.exp(-(b - 9.0)))
    dbias = (dlmb.sum(axis=0) * sig * (1.0 - sig)).reshape(1, C, 1, 1)
    return dx, dweight, dbias


# ------------------------------------------------------------------------------------------------
# a13/a14: LayerNorm(channels_first), 1x1 conv, GELU
# ------------------------------------------------------------------------------------------------
def layernorm_cf(x, weight, bias, eps, dtype=np.float64):
    """LayerNorm channels_first (util_converse.py:63-68): biased variance over dim 1."""
    def ln(x):
        x = x.astype(dtype)
        u = x.mean(axis=1, keepdims=True)
        v = ((x - u) ** 2).mean(axis=1, keepdims=True)
        y = (x - u) / np.sqrt(v + dtype(eps))
        return weight.astype(dtype)[None, :, None, None] * y + bias.astype(dtype)[None, :, None, None]
    return _rows_map(ln, x)


def gelu(x):
    """Exact GELU 0.5 x (1 + erf(x / sqrt 2)) (nn.GELU() default, util_converse.py:280)."""
    return _rows_map(lambda x: 0.5 * x * (1.0 + sspecial.erf(x / math.sqrt(2.0))), x)


def conv1x1(x, weight, bias, dtype=np.float64):
    """nn.Conv2d(cin, cout, 1, 1, 0): y[b,o,p] = sum_c W[o,c] x[b,c,p] + bias[o]."""
    x = x.astype(dtype)
    Wm = weight.reshape(weight.shape[0], -1).astype(dtype)
    B, C, H, W = x.shape
    y = np.matmul(Wm[None], x.reshape(B, C, H * W))
    if bias is not None:
        y = y + bias.astype(dtype)[None, :, None]
    return y.reshape(B, Wm.shape[0], H, W)


# ------------------------------------------------------------------------------------------------
# a15-a17: blocks and models (state dicts use the reference's key names)
# ------------------------------------------------------------------------------------------------
def converse_block(x, sd, prefix, kernel_size, scale, padding, padding_mode, eps=1e-5,
                   alpha=False, dtype=np.float64):
    """ConverseBlock (util_converse.py:253-293) / ConverseBlockAlphaVariant (:296-323).

    conv1 = LN -> 1x1 (C->2C) -> GELU -> Converse2D(2C) -> GELU -> 1x1 (2C->C)
    conv2 = LN -> 1x1 (C->2C) -> GELU -> 1x1 (2C->C); each branch residual (alpha-scaled)."""
    g = lambda k: sd[prefix + k]
    t = layernorm_cf(x, g("conv1.0.weight"), g("conv1.0.bias"), 1e-5, dtype)
    t = gelu(conv1x1(t, g("conv1.1.weight"), g("conv1.1.bias"), dtype))
    t = converse2d_module(t, g("conv1.3.weight"), g("conv1.3.bias"), scale, padding, padding_mode,
                          eps, dtype)
    t = conv1x1(gelu(t), g("conv1.5.weight"), g("conv1.5.bias"), dtype)
    x = (g("alpha1").astype(dtype) * t if alpha else t) + x
    t = layernorm_cf(x, g("conv2.0.weight"), g("conv2.0.bias"), 1e-5, dtype)
    t = gelu(conv1x1(t, g("conv2.1.weight"), g("conv2.1.bias"), dtype))
    t = conv1x1(t, g("conv2.3.weight"), g("conv2.3.bias"), dtype)
    x = (g("alpha2").astype(dtype) * t if alpha else t) + x
    return x


def converse_dncnn(x, sd, kernel_size=7, padding=6, padding_mode="circular", num_blocks=20,
                   dtype=np.float64):
    """ConverseDnCNN.forward (models/converse_dncnn.py:11-35): head 1x1, 20 ConverseBlocks, tail."""
    x = conv1x1(x, sd["m_head.0.weight"], sd["m_head.0.bias"], dtype)
    for i in range(num_blocks):
        x = converse_block(x, sd, f"m_body.{i}.", kernel_size, 1, padding, padding_mode, 1e-5,
                           False, dtype)
    return conv1x1(x, sd["m_tail.0.weight"], sd["m_tail.0.bias"], dtype)


def conv_reverse_datanet(x, k, sf, alpha, eps=1e-3, padding=0, padding_mode="circular", dtype=np.float64):
    """ConvReverseDataNet.forward (models/converse_usrnet.py:41-68): pad, the op with a per-sample psf
    k (B,C,kh,kw), lambda from alpha, x0 = nearest(padded x), crop."""
    return converse2d_module(x, k, alpha, sf, padding, padding_mode, eps, dtype)


def kernelnet(k, sd, prefix, kernel_size, dtype=np.float64):
    """KernelNet.forward (models/converse_usrnet.py:133-142)."""
    b = k.shape[0]
    t = k.reshape(b, -1).astype(dtype)
    lin = lambda t, n: t @ sd[prefix + n + ".weight"].astype(dtype).T + sd[prefix + n + ".bias"]
    t = gelu(lin(t, "fc1"))
    t = gelu(lin(t, "fc2"))
    t = lin(t, "fc3")
    return t.reshape(b, 16, kernel_size, kernel_size)


def converse_net(x, sd, num_iterations=5, num_blocks=7, dtype=np.float64):
    """ConverseNet.forward (models/converse_usrnet.py:150-169): 1x1 3->64, the same
    MultiConverseBlock (k3, padding 2, circular) applied num_iterations times, 1x1 64->3."""
    x = conv1x1(x, sd["conv1.weight"], sd["conv1.bias"], dtype)
    for _ in range(num_iterations):
        for j in range(num_blocks):
            x = converse_block(x, sd, f"p.m_body.{j}.", 3, 1, 2, "circular", 1e-5, False, dtype)
    return conv1x1(x, sd["conv2.weight"], sd["conv2.bias"], dtype)


def converse_usrnet(x, k, sf, sd, kernel_size, num_iterations=5, num_blocks=7, dtype=np.float64):
    """ConverseUSRNet.forward (models/converse_usrnet.py:192-214)."""
    b = k.shape[0]
    kk = kernelnet(k, sd, "kernelnet.", kernel_size, dtype)
    x = conv1x1(x, sd["conv1.weight"], sd["conv1.bias"], dtype)

    def body(x):
        for j in range(num_blocks):
            x = converse_block(x, sd, f"p.m_body.{j}.", 3, 1, 2, "circular", 1e-5, True, dtype)
        return x

    for i in range(num_iterations):
        k_ = conv1x1(kk, sd[f"convs.{i}.weight"], sd[f"convs.{i}.bias"], dtype)
        k_ = k_.reshape(b, 64, kernel_size, kernel_size)
        x = conv_reverse_datanet(x, k_, sf if i == 0 else 1, sd["d.alpha"], 1e-3, dtype=dtype)
        x = body(x)
    return conv1x1(x, sd["conv2.weight"], sd["conv2.bias"], dtype)


# ------------------------------------------------------------------------------------------------
# SRResNet family (models/converse_srresnet.py) and the plain layers it uses
# ------------------------------------------------------------------------------------------------
def conv3x3(x, weight, bias, dtype=np.float64):
    """nn.Conv2d(cin, cout, 3, 1, 1) (zero padding 1): y[b,o,i,j] = sum_{c,a,d} W[o,c,a,d] x[b,c,i+a-1,j+d-1]."""
    x = x.astype(dtype)
    B, C, H, W = x.shape
    xp = np.zeros((B, C, H + 2, W + 2), dtype)
    xp[:, :, 1:-1, 1:-1] = x
    y = np.zeros((B, weight.shape[0], H, W), dtype)
    for a in range(3):
        for d in range(3):
            y += np.einsum("oc,bchw->bohw", weight[:, :, a, d].astype(dtype), xp[:, :, a:a + H, d:d + W])
    if bias is not None:
        y += bias.astype(dtype)[None, :, None, None]
    return y


def bilinear_upsample(x, s):
    """F.interpolate(scale_factor=s, mode='bilinear', align_corners=False): source coordinate
    (dst + 0.5) / s - 0.5 clamped at 0, linear weights between floor and floor + 1 (clamped to the
    last sample), separably along rows and columns."""
    def axis_weights(n):
        dst = np.arange(n * s)
        src = np.maximum((dst + 0.5) / s - 0.5, 0.0)
        i0 = np.floor(src).astype(int)
        i1 = np.minimum(i0 + 1, n - 1)
        lam1 = src - i0
        return i0, i1, lam1
    H, W = x.shape[-2:]
    r0, r1, lr = axis_weights(H)
    c0, c1, lc = axis_weights(W)
    rows = x[..., r0, :] * (1 - lr)[:, None] + x[..., r1, :] * lr[:, None]
    return rows[..., c0] * (1 - lc) + rows[..., c1] * lc


def residual_block(x, sd, prefix, dtype=np.float64):
    """ResidualBlock (util_converse.py:328-342): x + conv2(relu(conv1(x)))."""
    t = np.maximum(conv3x3(x, sd[prefix + "conv1.weight"], sd[prefix + "conv1.bias"], dtype), 0.0)
    return x + conv3x3(t, sd[prefix + "conv2.weight"], sd[prefix + "conv2.bias"], dtype)


def converse_msrresnet(x, sd, num_blocks=16, upscale=4, dtype=np.float64):
    """ConverseMSRResNet.forward (models/converse_srresnet.py:72-82): 1x1 head + GELU, ConverseBlocks
    (k5, padding 4, replicate), two ConverseBlock + Converse2D(k2, s2, padding 2, replicate, eps 1e-3)
    + GELU upsamplers, ConverseBlock + GELU, 1x1 tail without bias, plus the bilinear-upsampled input."""
    x = x.astype(dtype)
    blk = lambda t, name: converse_block(t, sd, name + ".", 5, 1, 4, "replicate", 1e-5, False, dtype)  # noqa: E731
    x1 = gelu(conv1x1(x, sd["conv_first.weight"], sd["conv_first.bias"], dtype))
    for i in range(num_blocks):
        x1 = blk(x1, f"conv_body.{i}")
    for up in ("1", "2"):
        x1 = blk(x1, "upconv" + up)
        x1 = gelu(converse2d_module(x1, sd[f"up{up}.weight"], sd[f"up{up}.bias"], 2, 2, "replicate", 1e-3, dtype))
    x1 = gelu(blk(x1, "conv_hres"))
    x1 = conv1x1(x1, sd["conv_last.weight"], None, dtype)
    return x1 + bilinear_upsample(x, upscale)


def converse_up_msrresnet(x, sd, num_blocks=16, upscale=4, dtype=np.float64):
    """ConverseUpMSRResNet.forward (models/converse_srresnet.py:107-119): 3x3 head + GELU, residual
    blocks, two (3x3 conv -> Converse2D(k2, s2, padding 2, circular) -> GELU) upsamplers, 3x3 tail,
    plus the bilinear-upsampled input."""
    x = x.astype(dtype)
    x1 = gelu(conv3x3(x, sd["conv_first.weight"], sd["conv_first.bias"], dtype))
    for i in range(num_blocks):
        x1 = residual_block(x1, sd, f"conv_body.{i}.", dtype)
    for k in ("1", "2"):
        x1 = conv3x3(x1, sd[f"conv{k}.weight"], sd[f"conv{k}.bias"], dtype)
        x1 = gelu(converse2d_module(x1, sd[f"reverse{k}.weight"], sd[f"reverse{k}.bias"], 2, 2, "circular", 1e-5,
                                    dtype))
    x1 = conv3x3(gelu(conv3x3(x1, sd["conv_hres.weight"], sd["conv_hres.bias"], dtype)), sd["conv_last.weight"],
                 sd["conv_last.bias"], dtype)
    return x1 + bilinear_upsample(x, upscale)


# ------------------------------------------------------------------------------------------------
# Closed forms and brute force used to pin the functions above (identities I1-I8)
# ------------------------------------------------------------------------------------------------
def otf_direct(psf, shape):
    """I3: K[u,v] = sum_{a,b} psf[a,b] exp(-2 pi i (u (a - kh//2)/Hs + v (b - kw//2)/Ws))."""
    kh, kw = psf.shape[-2:]
    Hs, Ws = shape
    u = np.arange(Hs)[:, None]
    v = np.arange(Ws)[:, None]
    ea = np.exp(-2j * np.pi * u * (np.arange(kh)[None, :] - kh // 2) / Hs)  # (Hs, kh)
    eb = np.exp(-2j * np.pi * v * (np.arange(kw)[None, :] - kw // 2) / Ws)  # (Ws, kw)
    return np.einsum("ua,...ab,vb->...uv", ea, psf.astype(np.float64), eb)


def normal_equation_solve(y, x0, psf, lmb, s):
    """I6: the minimiser of ||y - S(K (*) x)||^2 + lambda ||x - x0||^2 on the (h s, w s) torus,
    solved as a dense linear system in fp64 (tiny planes only).  y (h,w), x0 (hs,ws), psf (kh,kw)."""
    h, w = y.shape
    Hs, Ws = h * s, w * s
    kh, kw = psf.shape
    n = Hs * Ws
    Kmat = np.zeros((n, n))
    for i in range(Hs):
        for j in range(Ws):
            row = i * Ws + j
            for a in range(kh):
                for b in range(kw):
                    # circular convolution with the psf centred at (kh//2, kw//2)
                    ii = (i - (a - kh // 2)) % Hs
                    jj = (j - (b - kw // 2)) % Ws
                    Kmat[row, ii * Ws + jj] += psf[a, b]
    S = np.zeros((h * w, n))
    for i in range(h):
        for j in range(w):
            S[i * w + j, (i * s) * Ws + j * s] = 1.0
    A = S @ Kmat
    lhs = A.T @ A + lmb * np.eye(n)
    rhs = A.T @ y.reshape(-1) + lmb * x0.reshape(-1)
    return np.linalg.solve(lhs, rhs).reshape(Hs, Ws)
