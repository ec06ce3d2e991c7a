"""Converse-DnCNN (models/converse_dncnn.py:11-35): 1x1 head, 20 ConverseBlocks, 1x1 tail.

Same constructor defaults, module tree and state-dict keys as the reference, so reference
checkpoints load with strict=True.  The 1x1 head (1->64) and tail (64->1) run on the library's VALU
1x1 kernel; the blocks run fused (conversenet_amd.util_converse.ConverseBlock).
"""
import torch.nn as nn

from . import functional
from .util_converse import ConverseBlock, _hip_eligible, run_blocks


class ConverseDnCNN(nn.Module):
    def __init__(self, in_channels=1, kernel_size=7, num_features=64, padding=6, padding_mode="circular", eps=1e-5,
                 num_blocks=20):
        super().__init__()
        self.num_features = num_features
        self.kernel_size = kernel_size
        self.padding = padding
        self.padding_mode = padding_mode
        self.eps = eps
        self.num_blocks = num_blocks
        # the reference builds exactly 20 blocks regardless of num_blocks (converse_dncnn.py:24)
        self.m_head = nn.Sequential(nn.Conv2d(in_channels, num_features, 1, 1, 0))
        self.m_body = nn.Sequential(*[ConverseBlock(num_features, num_features, kernel_size=self.kernel_size, scale=1,
                                                    padding=padding, padding_mode=padding_mode, eps=1e-5)
                                      for _ in range(20)])
        self.m_tail = nn.Sequential(nn.Conv2d(num_features, in_channels, 1, 1, 0))

    def forward(self, x):
        h, t = self.m_head[0], self.m_tail[0]
        if _hip_eligible(x, h.weight, h.bias, t.weight, t.bias):
            x = functional.conv1x1(x, h.weight, h.bias)
            x = run_blocks(self.m_body, x)
            return functional.conv1x1(x, t.weight, t.bias)
        x = self.m_head(x)
        x = self.m_body(x)
        x = self.m_tail(x)
        return x
