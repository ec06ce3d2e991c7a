"""Converse SRResNet variants (models/converse_srresnet.py): ConverseMSRResNet (:50-82) and
ConverseUpMSRResNet (:85-119).  The plain MSRResNet (:7-46) has no Converse2D layer and is not part
of this library.

Same class names, constructor defaults, module trees and state-dict keys as the reference, so the
reference checkpoint (model_zoo/converse_srresnet.pth, a ConverseMSRResNet) loads with strict=True.
ConverseMSRResNet runs its ConverseBlocks fused (k5, padding 4, replicate), the two x2 Converse2D
upsamplers (k2, padding 2, replicate, eps 1e-3) with GELU on store, and its 1x1 convolutions on the
library's kernels (the last one adds the bilinear-upsampled input as its residual).
ConverseUpMSRResNet keeps its 3x3 convolutions and residual blocks in torch; its Converse2D
upsamplers run on the library.
"""
import torch.nn as nn
import torch.nn.functional as F

from . import functional
from .util_converse import Converse2D, ConverseBlock, ResidualBlock, _hip_eligible


class ConverseMSRResNet(nn.Module):
    """MSRResNet with ConverseBlocks and Converse2D x2 upsamplers (converse_srresnet.py:50-82)."""

    def __init__(self, in_channels=3, out_channels=3, num_features=64, num_blocks=16, upscale=4):
        super().__init__()
        self.upscale = upscale
        self.conv_first = nn.Conv2d(in_channels, num_features, 1, 1, 0, bias=True)
        self.conv_body = nn.Sequential(*[ConverseBlock(num_features, num_features, 5, 1, 4, padding_mode="replicate",
                                                       eps=1e-5) for _ in range(num_blocks)])
        self.upconv1 = ConverseBlock(num_features, num_features, 5, 1, 4, padding_mode="replicate", eps=1e-5)
        self.up1 = Converse2D(num_features, num_features, 2, 2, 2, padding_mode="replicate", eps=1e-3)
        self.upconv2 = ConverseBlock(num_features, num_features, 5, 1, 4, padding_mode="replicate", eps=1e-5)
        self.up2 = Converse2D(num_features, num_features, 2, 2, 2, padding_mode="replicate", eps=1e-3)
        self.conv_hres = ConverseBlock(num_features, num_features, 5, 1, 4, padding_mode="replicate", eps=1e-5)
        self.conv_last = nn.Conv2d(num_features, out_channels, 1, 1, 0, bias=False)
        self.gelu = nn.GELU()

    def forward(self, x):
        cf, cl = self.conv_first, self.conv_last
        if _hip_eligible(x, cf.weight, cf.bias, cl.weight):
            x1 = functional.conv1x1(x, cf.weight, cf.bias, act="gelu")
            x1 = self.conv_body(x1)
            x1 = self.up1(self.upconv1(x1), act="gelu")
            x1 = self.up2(self.upconv2(x1), act="gelu")
            x1 = self.gelu(self.conv_hres(x1))
            xu = F.interpolate(x, scale_factor=self.upscale, mode="bilinear", align_corners=False)
            return functional.conv1x1(x1, cl.weight, None, residual=xu)
        x1 = self.gelu(self.conv_first(x))
        x1 = self.conv_body(x1)
        x1 = self.gelu(self.up1(self.upconv1(x1)))
        x1 = self.gelu(self.up2(self.upconv2(x1)))
        x1 = self.conv_last(self.gelu(self.conv_hres(x1)))
        x = F.interpolate(x, scale_factor=self.upscale, mode="bilinear", align_corners=False)
        return x1 + x


class ConverseUpMSRResNet(nn.Module):
    """MSRResNet upsampling with Converse2D (converse_srresnet.py:85-119)."""

    def __init__(self, in_channels=3, out_channels=3, num_features=64, num_blocks=16, upscale=4):
        super().__init__()
        self.upscale = upscale
        self.conv_first = nn.Conv2d(in_channels, num_features, 3, 1, 1, bias=True)
        self.conv_body = nn.Sequential(*[ResidualBlock(num_features) for _ in range(num_blocks)])
        self.conv1 = nn.Conv2d(num_features, num_features, 3, 1, 1)
        self.reverse1 = Converse2D(num_features, num_features, 2, scale=2)
        self.conv2 = nn.Conv2d(num_features, num_features, 3, 1, 1)
        self.reverse2 = Converse2D(num_features, num_features, 2, scale=2)
        self.conv_hres = nn.Conv2d(num_features, num_features, 3, 1, 1, bias=True)
        self.conv_last = nn.Conv2d(num_features, out_channels, 3, 1, 1, bias=True)
        self.gelu = nn.GELU()

    def forward(self, x):
        x1 = self.gelu(self.conv_first(x))
        x1 = self.conv_body(x1)
        x1 = self.reverse1(self.conv1(x1), act="gelu")  # GELU fused on store on the HIP path
        x1 = self.reverse2(self.conv2(x1), act="gelu")
        x1 = self.conv_last(self.gelu(self.conv_hres(x1)))
        x = F.interpolate(x, scale_factor=self.upscale, mode="bilinear", align_corners=False)
        return x1 + x
