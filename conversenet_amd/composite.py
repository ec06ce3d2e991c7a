"""The PyTorch (torch.fft) composition of the Converse2D solve: the `backend="pytorch"` path.

The reference offers the same pure-PyTorch path (models/util_converse.py:170-187) and registers its
op as CompositeImplicitAutograd (Converse2D/torch_converse2d/converse2d.cpp:223-227), so CPU tensors,
float64 and autograd all work through torch's own differentiable ops.  This module keeps that
behaviour for the cases the forward-only fp32 HIP kernels do not take: CPU tensors, other dtypes,
and inputs that require grad.  The op order is the reference's (including its division by lambda),
so gradients and CPU results follow the reference exactly.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def p2o(psf, shape):
    """util_converse.py:218-235 (zeros created on the psf's device instead of CPU + copy)."""
    otf = torch.zeros(psf.shape[:-2] + tuple(shape), dtype=psf.dtype, device=psf.device)
    otf[..., : psf.shape[-2], : psf.shape[-1]].copy_(psf)
    otf = torch.roll(otf, (-int(psf.shape[-2] / 2), -int(psf.shape[-1] / 2)), dims=(-2, -1))
    return torch.fft.fftn(otf, dim=(-2, -1))


def upsample(x, scale):
    """util_converse.py:237-245."""
    if scale == 1:
        return x
    z = torch.zeros((x.shape[0], x.shape[1], x.shape[2] * scale, x.shape[3] * scale), dtype=x.dtype,
                    device=x.device)
    z[..., ::scale, ::scale].copy_(x)
    return z


def splits(a, scale):
    """util_converse.py:194-215."""
    *lead, W, H = a.size()
    Ws, Hs = W // scale, H // scale
    b = a.view(*lead, scale, Ws, scale, Hs)
    n = len(lead)
    b = b.permute(*range(n), n + 1, n + 3, n, n + 2).contiguous()
    return b.view(*lead, Ws, Hs, scale * scale)


def solve(x, x0, weight, lmb, scale):
    """The closed-form solve on an already padded x, reference op order (converse2d.cpp:186-207)."""
    s = int(scale)
    h, w = x.shape[-2:]
    STy = upsample(x, s)
    FB = p2o(weight, (h * s, w * s))
    FBC = torch.conj(FB)
    F2B = torch.pow(torch.abs(FB), 2)
    FBFy = FBC * torch.fft.fftn(STy, dim=(-2, -1))
    FR = FBFy + torch.fft.fftn(lmb * x0, dim=(-2, -1))
    x1 = FB.mul(FR)
    FBR = torch.mean(splits(x1, s), dim=-1, keepdim=False)
    invW = torch.mean(splits(F2B, s), dim=-1, keepdim=False)
    invWBR = FBR.div(invW + lmb)
    FCBinvWBR = FBC * invWBR.repeat(1, 1, s, s)
    FX = (FR - FCBinvWBR) / lmb
    return torch.real(torch.fft.ifftn(FX, dim=(-2, -1)))


def check_op_args(x, x0, weight, bias, scale):
    """The reference op's argument checks (converse2d.cpp:167-172), raising RuntimeError."""
    if x.dim() != 4:
        raise RuntimeError("x must be (B,C,H,W)")
    if x0.dim() != 4:
        raise RuntimeError("x0 must be (B,C,Hs,Ws)")
    if weight.dim() != 4 or weight.size(0) != 1:
        raise RuntimeError("weight must be (1,C,kh,kw)")
    if bias.dim() != 4 or bias.size(0) != 1 or bias.size(2) != 1 or bias.size(3) != 1:
        raise RuntimeError("bias must be (1,C,1,1)")
    if not (x.device == x0.device == weight.device == bias.device):
        raise RuntimeError("tensors on same device")
    if int(scale) < 1:
        raise RuntimeError("scale must be >= 1")


def converse2d_op(x, x0, weight, bias, scale, eps=1e-5):
    """converse2d::forward semantics (converse2d.cpp:165-209)."""
    check_op_args(x, x0, weight, bias, scale)
    return solve(x, x0, weight, torch.sigmoid(bias - 9.0) + eps, scale)


def converse2d_module(x, weight, bias, scale, padding, padding_mode, eps):
    """Converse2D.forward pure-PyTorch branch (util_converse.py:144-192)."""
    if padding > 0:
        x = F.pad(x, pad=[padding] * 4, mode=padding_mode, value=0)
    lmb = torch.sigmoid(bias - 9.0) + eps
    x0 = x if scale == 1 else F.interpolate(x, scale_factor=scale, mode="nearest")
    out = solve(x, x0, weight, lmb, scale)
    if padding > 0:
        ps = padding * scale
        out = out[..., ps:-ps, ps:-ps]
    return out
