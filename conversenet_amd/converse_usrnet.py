"""Converse-USRNet family (models/converse_usrnet.py): MultiConverseBlock (:10-16),
MultiConverseBlockAlphaVariant (:19-25), ConvReverseDataNet (:33-117), KernelNet (:125-142),
ConverseNet (:150-169), ConverseUSRNet (:178-214).

Same class names, constructor defaults, module trees and state-dict keys as the reference.  One
addition: ConverseUSRNet(kernel_size=7) forwards its kernel_size to KernelNet; the reference
hard-codes KernelNet() (7x7 blur kernels only, converse_usrnet.py:186).
"""
import torch
import torch.nn as nn

from . import composite, functional
from .util_converse import (_converse_hip, _hip_grad_eligible, ConverseBlock, ConverseBlockAlphaVariant,
                            _hip_eligible, run_blocks, sequential)


class MultiConverseBlock(nn.Module):
    def __init__(self, in_channels=64, num_blocks=7, kernel_size=3, scale=1, padding=2, padding_mode="circular"):
        super().__init__()
        self.m_body = sequential(*[ConverseBlock(in_channels, in_channels, kernel_size, scale, padding, padding_mode)
                                   for _ in range(num_blocks)])

    def forward(self, x):
        return run_blocks(self.m_body, x)


class MultiConverseBlockAlphaVariant(nn.Module):
    def __init__(self, in_channels=64, num_blocks=7, kernel_size=3, scale=1, padding=2, padding_mode="circular"):
        super().__init__()
        self.m_body = sequential(*[ConverseBlockAlphaVariant(in_channels, in_channels, kernel_size, scale, padding,
                                                             padding_mode) for _ in range(num_blocks)])

    def forward(self, x):
        return run_blocks(self.m_body, x)


class ConvReverseDataNet(nn.Module):
    """Converse2D solve with a per-sample psf k (B,64,kh,kw), lambda from alpha, eps 1e-3
    (converse_usrnet.py:33-104)."""

    def __init__(self, eps=1e-3):
        super().__init__()
        self.alpha = nn.Parameter(torch.zeros(1, 64, 1, 1))
        self.eps = eps

    @property
    def biaseps(self):
        """sigmoid(alpha - 9) + eps as the reference's forward stores it (converse_usrnet.py:46); the HIP
        path computes this tensor only when it is read."""
        v = self.__dict__.get("_biaseps")
        return torch.sigmoid(self.alpha - 9.0) + self.eps if v is None else v

    @biaseps.setter
    def biaseps(self, v):
        self.__dict__["_biaseps"] = v

    def forward(self, x, k, sf, padding=0, padding_mode="circular"):
        if _converse_hip(x, k, self.alpha, sf, padding):
            self.biaseps = None  # read lazily from the current alpha
            # k is an activation computed anew on every forward: its table is never reused, so not cached
            return functional.converse2d_fused(x, k, self.alpha.reshape(-1), sf, padding, padding_mode, self.eps,
                                               cache=False)
        if k.dim() == 4 and _hip_grad_eligible(x, k, self.alpha, sf, padding, padding_mode):
            self.biaseps = None
            return functional.converse2d_train(x, k, self.alpha, sf, padding, padding_mode, self.eps)
        self.biaseps = torch.sigmoid(self.alpha - 9.0) + self.eps
        return composite.converse2d_module(x, k, self.alpha, sf, padding, padding_mode, self.eps)

    def splits(self, a, scale):
        return composite.splits(a, scale)

    def p2o(self, psf, shape):
        return composite.p2o(psf, shape)

    def upsample(self, x, scale=3):
        return composite.upsample(x, scale)


class KernelNet(nn.Module):
    def __init__(self, kernel_size=7):
        super().__init__()
        self.kernel_size = kernel_size
        self.fc1 = nn.Linear(kernel_size ** 2, 64)
        self.fc2 = nn.Linear(64, 64)
        self.fc3 = nn.Linear(64, 16 * (kernel_size ** 2))
        self.gelu = nn.GELU()

    def forward(self, k):
        k = k.to(torch.float)
        b, _, _, _ = k.shape
        k = k.view(b, -1)
        k = self.gelu(self.fc1(k))
        k = self.gelu(self.fc2(k))
        k = self.fc3(k)
        return k.view(b, 16, self.kernel_size, self.kernel_size)


class ConverseNet(nn.Module):
    def __init__(self, num_iterations=5, in_channels=64, num_blocks=7):
        super().__init__()
        self.p = MultiConverseBlock(in_channels=in_channels, num_blocks=num_blocks)
        self.conv1 = nn.Conv2d(3, in_channels, 1, 1, 0)
        self.conv2 = nn.Conv2d(in_channels, 3, 1, 1, 0)
        self.num_iterations = num_iterations

    def forward(self, x):
        x = self.conv1(x)
        for _ in range(self.num_iterations):
            x = self.p(x)
        return self.conv2(x)


def _conv(m, x):
    if _hip_eligible(x, m.weight, m.bias):
        return functional.conv1x1(x, m.weight, m.bias)
    return m(x)


def _psf_maps(model, k, b, h, w):
    """Every iteration's psf convs[i](k).view(b, 64, h, w) (converse_usrnet.py:203-211 computes each in
    its loop; they depend on k only).  On HIP the 1x1 convolutions (16 -> 64 channels on psf-sized maps,
    a few microseconds of work each, bound by launch and memory latency) run as one launch with the
    weights stacked (kept while the parameters are unchanged), and one transposing copy lays the
    output out iteration-major, so that each iteration's psf is a contiguous (b, 64, h, w) view."""
    convs = model.convs
    if all(_hip_eligible(k, m.weight, m.bias) for m in convs):
        params = [t for m in convs for t in (m.weight, m.bias)]
        key = tuple((t.data_ptr(), t._version) for t in params)
        cached = getattr(model, "_psf_stack", None)
        if cached is None or cached[0] != key:
            cached = (key, torch.cat([m.weight for m in convs]), torch.cat([m.bias for m in convs]))
            model._psf_stack = cached
        n, m_ = convs[0].weight.shape[0], len(convs)
        y = functional.conv1x1(k, cached[1], cached[2])  # (b, m n, kh, kw)
        z = y.view(b, m_, n * y.shape[2] * y.shape[3]).transpose(0, 1).contiguous()
        return [z[i].view(b, n, h, w) for i in range(m_)]
    return [_conv(m, k).view(b, 64, h, w) for m in convs]


class ConverseUSRNet(nn.Module):
    def __init__(self, num_iterations=5, in_channels=64, num_blocks=7, kernel_size=7):
        super().__init__()
        self.d = ConvReverseDataNet()
        self.p = MultiConverseBlockAlphaVariant(in_channels=in_channels, num_blocks=num_blocks)
        self.conv1 = nn.Conv2d(3, 64, 1, 1, 0)
        self.conv2 = nn.Conv2d(64, 3, 1, 1, 0)
        self.kernelnet = KernelNet(kernel_size)
        self.num_iterations = num_iterations
        self.convs = nn.ModuleList([nn.Conv2d(16, 64, 1, 1, 0) for _ in range(num_iterations)])

    def forward(self, x, k, sf):
        b, c, h, w = k.shape
        k = self.kernelnet(k)
        x = _conv(self.conv1, x)
        ks = _psf_maps(self, k, b, h, w)
        x = self.d(x, ks[0], sf)
        x = self.p(x)
        for i in range(1, self.num_iterations):
            x = self.d(x, ks[i], 1)
            x = self.p(x)
        return _conv(self.conv2, x)
