"""KADConv, DSC and LCSA modules with the reference's public API.

Class names, constructor arguments, forward signatures and parameter names
follow KAD-Conv/kadconv/kad_conv.py:18-121 so that state dicts (and KAD-CNet
checkpoints, whose KADC4/DCN_RCA/RCA layers use the same names) load
unchanged.  The module tree is therefore the same as the reference's; the
forward passes are written here independently.

``forward`` is the plain composition of torch ops the reference describes.
The deformable convolution inside it is ``kadconv.ops.deform_conv2d``: the
gfx950 HIP kernel for GPU tensors, and torchvision's operator for CPU tensors
when torchvision is importable.  ``enable_fast_inference`` (kadconv.fast)
replaces the forward of eval-mode layers by the fused HIP pipeline in
kadconv.fused.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops

# YOLO-style BatchNorm settings of KAD-CNet training (kad_conv.py:13-15).
BN_EPS = 1e-3
BN_MOMENTUM = 0.03


def _bn(c):
    return nn.BatchNorm2d(c, eps=BN_EPS, momentum=BN_MOMENTUM)


class LCSA(nn.Module):
    """Low-Cost Spatial Attention (kad_conv.py:18-39): row and column means,
    added by broadcasting, then a depthwise 1xk conv, BN, ReLU, a depthwise kx1
    conv and a 1x1 projection to ``out_channels`` mask logits (pre-sigmoid)."""

    def __init__(self, in_channels, out_channels, band_kernel_size=11):
        super().__init__()
        k = band_kernel_size
        self.pool_h = nn.AdaptiveAvgPool2d((None, 1))
        self.pool_w = nn.AdaptiveAvgPool2d((1, None))
        self.excite = nn.Sequential(
            nn.Conv2d(in_channels, in_channels, (1, k), padding=(0, k // 2), groups=in_channels),
            _bn(in_channels),
            nn.ReLU(inplace=True),
            nn.Conv2d(in_channels, in_channels, (k, 1), padding=(k // 2, 0), groups=in_channels),
            nn.Conv2d(in_channels, out_channels, 1),
        )

    def forward(self, x):
        return self.excite(self.pool_h(x) + self.pool_w(x))


class DSC(nn.Module):
    """Deformable Spatial Convolution (kad_conv.py:42-67): DCNv2 whose offsets
    come from a 3x3 conv and whose modulation mask is sigmoid(LCSA(x))."""

    def __init__(self, in_channels, out_channels, kernel_size=3, stride=1, padding=1):
        super().__init__()
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size = kernel_size
        self.mask = True
        self.stride = (stride, stride)
        self.padding = padding
        kk = kernel_size * kernel_size
        self.weight = nn.Parameter(torch.empty(out_channels, in_channels, kernel_size, kernel_size))
        self.bias = nn.Parameter(torch.zeros(out_channels))
        self.conv_offset = nn.Conv2d(in_channels, 2 * kk, kernel_size, stride=stride, padding=padding)
        self.RCA_mask = LCSA(in_channels, kk)
        bound = 1.0 / math.sqrt(in_channels * kk)
        nn.init.uniform_(self.weight, -bound, bound)
        nn.init.zeros_(self.conv_offset.weight)
        nn.init.zeros_(self.conv_offset.bias)

    def forward(self, x):
        offset = self.conv_offset(x)
        mask = torch.sigmoid(self.RCA_mask(x)) if getattr(self, 'mask', True) else None
        return ops.deform_conv2d(x, offset, self.weight, self.bias, stride=self.stride, padding=self.padding,
                                 mask=mask)


class _Scale(nn.Module):
    """Learnable per-channel branch weight (kad_conv.py:70-78)."""

    def __init__(self, dims):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(*dims))

    def forward(self, x):
        return x * self.weight


def branch_widths(dim, n):
    """Channels per branch: the remainder goes to branch 0 (kad_conv.py:99)."""
    return [dim - (dim // n) * (n - 1)] + [dim // n] * (n - 1)


class KADConv(nn.Module):
    """Kernel Adaptive Deformable Convolution (kad_conv.py:81-121).

    ``n`` branches at relative resolutions 1, 1/2, ..., 1/2^(n-1); branch i is
    avg-pool 2^i -> 1x1 projection -> DSC -> BN -> ReLU -> per-channel scale ->
    channel attention, upsampled back (bilinear, align_corners=False); the
    branches are concatenated and the input is added.  Shape-preserving.
    """

    def __init__(self, dim, n=3, se_min_hidden=32):
        super().__init__()
        self.n = n
        widths = branch_widths(dim, n)
        self.convs = nn.ModuleList(
            nn.Sequential(nn.Conv2d(dim, c, 1), DSC(c, c), _bn(c), nn.ReLU(inplace=True)) for c in widths)
        self.fc = nn.ModuleList(
            nn.Sequential(nn.Linear(c, max(se_min_hidden, c)), nn.ReLU(),
                          nn.Linear(max(se_min_hidden, c), c), nn.Sigmoid()) for c in widths)
        self.weight = nn.ModuleList(nn.Sequential(_Scale([1, c, 1, 1])) for c in widths)

    def forward(self, x):
        outs = []
        size = x.shape[2:]
        for i in range(self.n):
            y = F.avg_pool2d(x, kernel_size=2 ** i) if i > 0 else x
            y = self.weight[i](self.convs[i](y))
            att = self.fc[i](y.mean(dim=(2, 3)))
            y = y * att.view(x.shape[0], -1, 1, 1)
            if i > 0:
                y = F.interpolate(y, size=size, mode='bilinear', align_corners=False)
            outs.append(y)
        return torch.cat(outs, dim=1) + x
