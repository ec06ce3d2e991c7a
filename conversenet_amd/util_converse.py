"""Drop-in replacement for the reference's models/util_converse.py, backed by the HIP library.

Same public names, constructor signatures, parameter shapes and state-dict keys as the reference
(models/util_converse.py): LayerNorm (:42-68), sequential (:71-91), Converse2D (:98-245),
ConverseBlock (:253-293), ConverseBlockAlphaVariant (:296-323), ResidualBlock (:328-342).

Dispatch (mirrors the reference's backend selection, util_converse.py:150-169):
  * backend "auto": fp32 HIP tensors without a pending gradient run the fused HIP kernels (an
    ImportError if the library is not built: there is no silent fallback for HIP tensors);
    anything else runs the PyTorch composition (the reference's own pure-PyTorch path).
  * backend "cuda": requires the HIP library and a HIP tensor (RuntimeError otherwise, as :156-158).
  * backend "pytorch": always the PyTorch composition.
  * $CONVERSE2D_BACKEND overrides the module's backend (:150).
A forward that autograd must differentiate runs the library's forward and backward kernels
(functional.Converse2DFunction) where the backward supports the configuration, and the composition
otherwise; the LayerNorm / 1x1 kernels are forward-only (the composition runs under autograd).
"""
from __future__ import annotations

import os
from collections import OrderedDict

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib, composite, functional
from . import op_registry  # noqa: F401  (registers torch.ops.converse2d)

_HAS_CONVERSE2D_EXT = _lib.available()

converse2d_CUDA = torch.ops.converse2d.forward

# (Cin, Cout) tiles the MFMA 1x1 kernels are instantiated for; (C, Cmid) for the fused branch
MFMA_SHAPES = {(64, 64), (64, 128), (128, 64), (128, 128), (16, 64), (64, 16), (32, 32), (32, 64), (64, 32)}
MLP_SHAPES = {(64, 128), (32, 64)}


def _backend(default: str) -> str:
    return (os.environ.get("CONVERSE2D_BACKEND", "") or default).lower()


def _hip_eligible(*ts) -> bool:
    """True when the forward-only fp32 HIP kernels serve these tensors.  HIP tensors never fall back
    to the PyTorch composition because the library is missing: that raises instead."""
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda or t.dtype != torch.float32:
            return False
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts):
        return False
    _lib.load()  # ImportError when libcvn_hip.so is not built
    return True


def _converse_hip(x, weight, bias, scale, padding) -> bool:
    """True when the library's forward serves this Converse2D call: fp32 HIP tensors, no pending
    gradient, and a geometry inside the library's limits (cvn_converse2d_supported; e.g. padded planes
    up to 4096 samples a side).  Other geometries run the PyTorch composition, which has no limits."""
    return _hip_eligible(x, weight, bias) and functional.supported(x, weight, scale, padding)


def _hip_grad_eligible(x, weight, bias, scale, padding, padding_mode) -> bool:
    """True when a forward that autograd must differentiate can run on the library's forward and
    backward kernels (fp32 HIP tensors, and a geometry the forward and the requested backward support,
    per cvn_converse2d_supported); otherwise the composition runs under autograd."""
    ts = (x, weight, bias)
    if not all(t.is_cuda and t.dtype == torch.float32 for t in ts):
        return False
    if not (torch.is_grad_enabled() and any(t.requires_grad for t in ts)):
        return False
    _lib.load()
    return functional.supported(x, weight, scale, padding, x.requires_grad, weight.requires_grad or bias.requires_grad)


"""
# --------------------------------------------
# LayerNorm for Vision Normalization
# --------------------------------------------
"""


class LayerNorm(nn.Module):
    """LayerNorm over channels_last (F.layer_norm) or channels_first (util_converse.py:42-68)."""

    def __init__(self, normalized_shape, eps=1e-6, data_format="channels_last"):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(normalized_shape))
        self.bias = nn.Parameter(torch.zeros(normalized_shape))
        self.eps = eps
        self.data_format = data_format
        if self.data_format not in ["channels_last", "channels_first"]:
            raise NotImplementedError
        self.normalized_shape = (normalized_shape,)

    def forward(self, x):
        if self.data_format == "channels_last":
            return F.layer_norm(x, self.normalized_shape, self.weight, self.bias, self.eps)
        if _hip_eligible(x, self.weight, self.bias) and x.dim() >= 2:
            return functional.layernorm_cf(x, self.weight, self.bias, self.eps)
        u = x.mean(1, keepdim=True)
        s = (x - u).pow(2).mean(1, keepdim=True)
        x = (x - u) / torch.sqrt(s + self.eps)
        x = self.weight[:, None, None] * x + self.bias[:, None, None]
        return x


def sequential(*args):
    """nn.Sequential that flattens nested Sequentials (util_converse.py:71-91)."""
    if len(args) == 1:
        if isinstance(args[0], OrderedDict):
            raise NotImplementedError("sequential does not support OrderedDict input.")
        return args[0]
    modules = []
    for module in args:
        if isinstance(module, nn.Sequential):
            for submodule in module.children():
                modules.append(submodule)
        elif isinstance(module, nn.Module):
            modules.append(module)
    return nn.Sequential(*modules)


"""
# --------------------------------------------
# Converse2D operator
# --------------------------------------------
"""


class Converse2D(nn.Module):
    """Depthwise reverse convolution (util_converse.py:98-245).

    Args match the reference: in_channels == out_channels (depthwise), kernel_size, scale (upsampling
    factor), padding, padding_mode ('reflect' | 'replicate' | 'circular' | 'constant'), eps, backend
    ('auto' | 'cuda' | 'pytorch').  Output (N, C, H*scale, W*scale).  Parameters: weight
    (1, C, k, k), initialised as a softmax over the k*k taps of a standard normal draw; bias
    (1, C, 1, 1) zeros; lambda = sigmoid(bias - 9) + eps is stored in self.biaseps on forward.
    """

    def __init__(self, in_channels, out_channels, kernel_size, scale=1, padding=2, padding_mode="circular",
                 eps=1e-5, backend: str = "auto"):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = kernel_size
        self.scale = scale
        self.padding = padding
        self.padding_mode = padding_mode
        self.eps = eps
        self.backend = backend.lower()
        if self.backend not in ("auto", "cuda", "pytorch"):
            raise ValueError(f"backend must be 'auto' | 'cuda' | 'pytorch', got: {self.backend}")
        assert self.out_channels == self.in_channels
        self.weight = nn.Parameter(torch.randn(1, self.in_channels, self.kernel_size, self.kernel_size))
        self.bias = nn.Parameter(torch.zeros(1, self.in_channels, 1, 1))
        self.weight.data = nn.functional.softmax(self.weight.data.view(1, self.in_channels, -1), dim=-1).view(
            1, self.in_channels, self.kernel_size, self.kernel_size)

    def _use_hip(self, x) -> bool:
        backend = _backend(self.backend)
        if backend == "cuda":
            if not (_HAS_CONVERSE2D_EXT and x.is_cuda):
                raise RuntimeError("Converse2D backend='cuda' but CUDA extension is unavailable.")
        elif backend == "pytorch":
            return False
        return _converse_hip(x, self.weight, self.bias, self.scale, self.padding)

    @property
    def biaseps(self):
        """lambda = sigmoid(bias - 9) + eps, as the reference's forward stores it (util_converse.py:150).
        The HIP path evaluates lambda inside the transfer-table kernel and computes this tensor only
        when it is read."""
        v = self.__dict__.get("_biaseps")
        return torch.sigmoid(self.bias - 9.0) + self.eps if v is None else v

    @biaseps.setter
    def biaseps(self, v):
        self.__dict__["_biaseps"] = v

    def _use_hip_grad(self, x) -> bool:
        if _backend(self.backend) == "pytorch":
            return False
        return _hip_grad_eligible(x, self.weight, self.bias, self.scale, self.padding, self.padding_mode)

    def forward(self, x, act=None):
        """act='gelu' applies exact GELU to the output (fused on store on the HIP path)."""
        if self._use_hip(x):
            self.biaseps = None  # read lazily from the current bias
            return functional.converse2d_fused(x, self.weight, self.bias.reshape(-1), self.scale, self.padding,
                                               self.padding_mode, self.eps, act)
        if self._use_hip_grad(x):
            self.biaseps = None
            out = functional.converse2d_train(x, self.weight, self.bias, self.scale, self.padding, self.padding_mode,
                                              self.eps)
            return F.gelu(out) if act == "gelu" else out
        self.biaseps = torch.sigmoid(self.bias - 9.0) + self.eps
        out = composite.converse2d_module(x, self.weight, self.bias, self.scale, self.padding, self.padding_mode,
                                          self.eps)
        return F.gelu(out) if act == "gelu" else out

    # reference helpers kept for API parity (util_converse.py:194-245)
    def splits(self, a, scale):
        return composite.splits(a, scale)

    def p2o(self, psf, shape):
        return composite.p2o(psf, shape)

    def upsample(self, x, scale=3):
        return composite.upsample(x, scale)


"""
# --------------------------------------------
# Converse Blocks
# --------------------------------------------
"""


def _block_parts(blk):
    """The layers of a ConverseBlock(AlphaVariant) the fused path needs, or None when a shape is
    outside the instantiated HIP tiles."""
    ln1, c11, _, cv, _, c15 = blk.conv1
    ln2, c21, _, c23 = blk.conv2
    C = c11.in_channels
    mid = c11.out_channels
    if (C, mid) not in MFMA_SHAPES or (mid, C) not in MFMA_SHAPES or (C, c21.out_channels) not in MLP_SHAPES:
        return None
    if not isinstance(cv, Converse2D) or _backend(cv.backend) == "pytorch" or cv.scale != 1:
        return None
    alphas = (blk.alpha1.reshape(-1), blk.alpha2.reshape(-1)) if hasattr(blk, "alpha1") else (None, None)
    return ln1, c11, cv, c15, ln2, c21, c23, alphas


def _block_head(parts, x):
    """LN -> 1x1 -> GELU (the first branch's first layer)."""
    ln1, c11 = parts[0], parts[1]
    return functional.conv1x1(x, c11.weight, c11.bias, act="gelu", ln=(ln1.weight, ln1.bias, ln1.eps))


def _block_converse(parts, t, act="gelu"):
    cv = parts[2]
    cv.biaseps = None  # read lazily from the current bias
    return functional.converse2d_fused(t, cv.weight, cv.bias.reshape(-1), cv.scale, cv.padding, cv.padding_mode,
                                       cv.eps, act=act)


def _gelu_in_tail(parts, t_shape, x):
    """Whether the block's GELU after its Converse2D (util_converse.py:281) is applied as the fused
    tail loads its input instead of as the Converse2D stores its output: on the 268 path, whose
    inverse row pass is bound by VALU issue at three waves per SIMD (there the GELU costs about 24 us
    of a 0.47 ms layer at Converse-DnCNN's shape; in the tail, about 10 us)."""
    _, _, cv, c15, _, c21, _, _ = parts
    if (c15.in_channels, c15.out_channels, c21.out_channels) not in functional.TAIL_SHAPES or x.data_ptr() % 16:
        return False
    return functional.module_route(t_shape, cv.weight, cv.scale, cv.padding) == _lib.ROUTE_PFA268


def _block_tail(parts, t, x, next_parts=None, t_act=None):
    """1x1 + residual and the LN-MLP branch + residual; with next_parts also the next block's head.
    t_act='gelu': t is the Converse2D output before the block's GELU.
    Returns (block output, next block's Converse2D input or None)."""
    _, _, _, c15, ln2, c21, c23, (s1, s2) = parts
    mid, C = c15.in_channels, c15.out_channels
    aligned = t.data_ptr() % 16 == 0 and x.data_ptr() % 16 == 0
    if (mid, C, c21.out_channels) in functional.TAIL_SHAPES and aligned:
        if next_parts is not None and next_parts[1].out_channels == mid:
            nln, nc11 = next_parts[0], next_parts[1]
            return functional.conv_ln_mlp_residual(t, x, c15.weight, c15.bias, ln2.weight, ln2.bias, ln2.eps,
                                                   c21.weight, c21.bias, c23.weight, c23.bias, s1, s2,
                                                   head=(nln.weight, nln.bias, nln.eps, nc11.weight, nc11.bias),
                                                   t_act=t_act)
        y = functional.conv_ln_mlp_residual(t, x, c15.weight, c15.bias, ln2.weight, ln2.bias, ln2.eps,
                                            c21.weight, c21.bias, c23.weight, c23.bias, s1, s2, t_act=t_act)
        return y, None
    if t_act == "gelu":
        t = torch.nn.functional.gelu(t)
    x = functional.conv1x1(t, c15.weight, c15.bias, residual=x, res_scale=s1)
    y = functional.ln_mlp_residual(x, ln2.weight, ln2.bias, ln2.eps, c21.weight, c21.bias, c23.weight, c23.bias,
                                   res_scale=s2, out=x)
    return y, None


def _parts_supported(parts, x):
    """The block's Converse2D input is (B, 2C, H, W): inside the library's limits?"""
    cv = parts[2]
    return functional.supported(None, cv.weight, cv.scale, cv.padding,
                                shape=(x.shape[0], cv.in_channels, x.shape[2], x.shape[3]))


def _fused_block_forward(blk, x, alpha1=None, alpha2=None):
    """LN+1x1+GELU -> Converse2D+GELU -> 1x1+residual and the LN-MLP branch + residual.
    Returns None when a shape is outside the instantiated HIP tiles or the library's limits."""
    parts = _block_parts(blk)
    if parts is None or (x.shape[2] * x.shape[3]) % 4 != 0 or not _parts_supported(parts, x):
        return None
    t = _block_head(parts, x)
    gin = _gelu_in_tail(parts, t.shape, x)
    return _block_tail(parts, _block_converse(parts, t, None if gin else "gelu"), x, t_act="gelu" if gin else None)[0]


def run_blocks(blocks, x):
    """A chain of ConverseBlocks (util_converse.py:253-323 applied in sequence, as in the bodies of
    converse_dncnn.py:24 and converse_usrnet.py:19-33).  On the HIP path each block's tail kernel
    also computes the next block's LN -> 1x1 -> GELU, so a block's output is read once; otherwise the
    blocks run one by one."""
    blocks = list(blocks)
    if not blocks:
        return x
    parts = [_block_parts(b) if _hip_eligible(x, *_block_params(b)) else None for b in blocks]
    if (any(p is None for p in parts) or (x.shape[2] * x.shape[3]) % 4 != 0
            or not all(_parts_supported(p, x) for p in parts)):
        for b in blocks:
            x = b(x)
        return x
    t = _block_head(parts[0], x)
    for i, p in enumerate(parts):
        gin = _gelu_in_tail(p, t.shape, x)
        t = _block_converse(p, t, None if gin else "gelu")
        x, t_next = _block_tail(p, t, x, parts[i + 1] if i + 1 < len(parts) else None, "gelu" if gin else None)
        t = t_next if t_next is not None else (_block_head(parts[i + 1], x) if i + 1 < len(parts) else None)
    return x


def _block_params(blk):
    return [p for p in blk.parameters()]


class ConverseBlock(nn.Module):
    """LN -> 1x1 -> GELU -> Converse2D -> GELU -> 1x1 (+x); LN -> 1x1 -> GELU -> 1x1 (+x)
    (util_converse.py:253-293)."""

    def __init__(self, in_channels, out_channels, kernel_size=3, scale=1, padding=2, padding_mode="replicate",
                 eps=1e-5):
        super().__init__()
        self.conv1 = nn.Sequential(LayerNorm(in_channels, eps=1e-5, data_format="channels_first"),
                                   nn.Conv2d(in_channels, 2 * out_channels, 1, 1, 0),
                                   nn.GELU(),
                                   Converse2D(2 * out_channels, 2 * out_channels, kernel_size, scale=scale,
                                              padding=padding, padding_mode=padding_mode, eps=eps),
                                   nn.GELU(),
                                   nn.Conv2d(2 * out_channels, out_channels, 1, 1, 0))
        self.conv2 = nn.Sequential(LayerNorm(in_channels, eps=1e-5, data_format="channels_first"),
                                   nn.Conv2d(out_channels, 2 * out_channels, 1, 1, 0),
                                   nn.GELU(),
                                   nn.Conv2d(2 * out_channels, out_channels, 1, 1, 0))

    def forward(self, x):
        if _hip_eligible(x, *_block_params(self)) and self.conv1[3].scale == 1:
            y = _fused_block_forward(self, x)
            if y is not None:
                return y
        x = self.conv1(x) + x
        x = self.conv2(x) + x
        return x


class ConverseBlockAlphaVariant(nn.Module):
    """ConverseBlock with per-channel alpha scaling of both residual branches
    (util_converse.py:296-323); alpha1/alpha2 initialise to zero."""

    def __init__(self, in_channels, out_channels, kernel_size=3, scale=1, padding=2, padding_mode="replicate",
                 eps=1e-5):
        super().__init__()
        self.alpha1 = nn.Parameter(torch.zeros((1, out_channels, 1, 1)), requires_grad=True)
        self.alpha2 = nn.Parameter(torch.zeros((1, out_channels, 1, 1)), requires_grad=True)
        self.conv1 = nn.Sequential(LayerNorm(in_channels, eps=1e-5, data_format="channels_first"),
                                   nn.Conv2d(in_channels, 2 * out_channels, 1, 1, 0),
                                   nn.GELU(),
                                   Converse2D(2 * out_channels, 2 * out_channels, kernel_size, scale=scale,
                                              padding=padding, padding_mode=padding_mode, eps=eps),
                                   nn.GELU(),
                                   nn.Conv2d(2 * out_channels, out_channels, 1, 1, 0))
        self.conv2 = nn.Sequential(LayerNorm(in_channels, eps=1e-5, data_format="channels_first"),
                                   nn.Conv2d(out_channels, 2 * out_channels, 1, 1, 0),
                                   nn.GELU(),
                                   nn.Conv2d(2 * out_channels, out_channels, 1, 1, 0))

    def forward(self, x):
        if _hip_eligible(x, *_block_params(self)) and self.conv1[3].scale == 1:
            y = _fused_block_forward(self, x, self.alpha1, self.alpha2)
            if y is not None:
                return y
        x = self.alpha1 * self.conv1(x) + x
        x = self.alpha2 * self.conv2(x) + x
        return x


class ResidualBlock(nn.Module):
    """---Conv-ReLU-Conv-+- (util_converse.py:328-342); plain torch convolutions."""

    def __init__(self, num_features=64):
        super().__init__()
        self.conv1 = nn.Conv2d(num_features, num_features, 3, 1, 1, bias=True)
        self.conv2 = nn.Conv2d(num_features, num_features, 3, 1, 1, bias=True)

    def forward(self, x):
        out = F.relu(self.conv1(x), inplace=True)
        out = self.conv2(out)
        return x + out
