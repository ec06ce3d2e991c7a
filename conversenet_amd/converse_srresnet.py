"""SRResNet family (models/converse_srresnet.py): MSRResNet (:7-47), ConverseMSRResNet (:50-82) and
ConverseUpMSRResNet (:85-119).

Same class names, constructor defaults, module trees and state-dict keys as the reference, so the
reference checkpoint (model_zoo/converse_srresnet.pth, a ConverseMSRResNet) loads with strict=True.
ConverseMSRResNet runs its ConverseBlocks fused (k5, padding 4, replicate), the two x2 Converse2D
upsamplers (k2, padding 2, replicate, eps 1e-3) with GELU on store, and its 1x1 convolutions on the
library's kernels (the last one adds the bilinear-upsampled input as its residual).  MSRResNet and
ConverseUpMSRResNet keep their 3x3 convolutions, pixel shuffle and residual blocks in torch; the
Converse2D upsamplers of ConverseUpMSRResNet run on the library.
"""
import torch.nn as nn
import torch.nn.functional as F

from . import functional
from .util_converse import Converse2D, ConverseBlock, ResidualBlock, _hip_eligible


class MSRResNet(nn.Module):
    """Modified SRResNet (converse_srresnet.py:7-47): no Converse2D layers."""

    def __init__(self, in_channels=3, out_channels=3, num_features=64, num_blocks=16, upscale=4):
        super().__init__()
        self.upscale = upscale
        self.conv_first = nn.Conv2d(in_channels, num_features, 3, 1, 1, bias=True)
        self.conv_body = nn.Sequential(*[ResidualBlock(num_features) for _ in range(num_blocks)])
        if self.upscale in [2, 3]:
            self.upconv1 = nn.Conv2d(num_features, num_features * (upscale ** 2), 3, 1, 1, bias=True)
            self.pixel_shuffle = nn.PixelShuffle(upscale)
        elif self.upscale == 4:
            self.upconv1 = nn.Conv2d(num_features, num_features * 4, 3, 1, 1, bias=True)
            self.upconv2 = nn.Conv2d(num_features, num_features * 4, 3, 1, 1, bias=True)
            self.pixel_shuffle = nn.PixelShuffle(2)
        self.conv_hres = nn.Conv2d(num_features, num_features, 3, 1, 1, bias=True)
        self.conv_last = nn.Conv2d(num_features, out_channels, 3, 1, 1, bias=True)
        self.lrelu = nn.LeakyReLU(negative_slope=0.1, inplace=True)

    def forward(self, x):
        x1 = self.lrelu(self.conv_first(x))
        x1 = self.conv_body(x1)
        if self.upscale == 4:
            x1 = self.lrelu(self.pixel_shuffle(self.upconv1(x1)))
            x1 = self.lrelu(self.pixel_shuffle(self.upconv2(x1)))
        elif self.upscale in [2, 3]:
            x1 = self.lrelu(self.pixel_shuffle(self.upconv1(x1)))
        x1 = self.conv_last(self.lrelu(self.conv_hres(x1)))
        x = F.interpolate(x, scale_factor=self.upscale, mode="bilinear", align_corners=False)
        return x1 + x


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
