"""KAD-CNet building blocks with the reference's class names, constructor
arguments and attribute names (KAD-CNet/models/common.py), so that state dicts
and module trees line up with the reference's DetectionModel.  Forward passes
are the plain PyTorch compositions the reference defines; they run on CPU or
GPU.  The HIP network forward lives in kadcnet.fast.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F


def make_divisible(x, divisor):
    """Round x up to a multiple of divisor (KAD-CNet/utils/general.py:660-664)."""
    return math.ceil(x / divisor) * divisor


def autopad(k, p=None, d=1):
    """'same' padding for an odd kernel (common.py:34-40)."""
    if d > 1:
        k = d * (k - 1) + 1 if isinstance(k, int) else [d * (x - 1) + 1 for x in k]
    if p is None:
        p = k // 2 if isinstance(k, int) else [x // 2 for x in k]
    return p


class Conv(nn.Module):
    """conv (no bias) -> BatchNorm -> SiLU (common.py:43-57).  After ``fuse``
    the BN is folded into a biased conv and ``forward_fuse`` runs."""
    default_act = nn.SiLU()

    def __init__(self, c1, c2, k=1, s=1, p=None, g=1, d=1, act=True):
        super().__init__()
        self.conv = nn.Conv2d(c1, c2, k, s, autopad(k, p, d), groups=g, dilation=d, bias=False)
        self.bn = nn.BatchNorm2d(c2)
        self.act = self.default_act if act is True else act if isinstance(act, nn.Module) else nn.Identity()

    def forward(self, x):
        return self.act(self.bn(self.conv(x)))

    def forward_fuse(self, x):
        return self.act(self.conv(x))


class AConv(nn.Module):
    """2x2 / stride-1 average pool, then a 3x3 stride-2 Conv (common.py:60-67)."""

    def __init__(self, c1, c2):
        super().__init__()
        self.cv1 = Conv(c1, c2, 3, 2, 1)

    def forward(self, x):
        return self.cv1(F.avg_pool2d(x, 2, 1, 0, False, True))


class SP(nn.Module):
    """Max pool, stride 1, 'same' padding (common.py:187-193)."""

    def __init__(self, k=3, s=1):
        super().__init__()
        self.m = nn.MaxPool2d(kernel_size=k, stride=s, padding=k // 2)

    def forward(self, x):
        return self.m(x)


class Concat(nn.Module):
    def __init__(self, dimension=1):
        super().__init__()
        self.d = dimension

    def forward(self, x):
        return torch.cat(x, self.d)


class SPPELAN(nn.Module):
    """cv1, three chained 5x5 max pools, concat of all four, cv5 (common.py:563-577)."""

    def __init__(self, c1, c2, c3):
        super().__init__()
        self.c = c3
        self.cv1 = Conv(c1, c3, 1, 1)
        self.cv2 = SP(5)
        self.cv3 = SP(5)
        self.cv4 = SP(5)
        self.cv5 = Conv(4 * c3, c2, 1, 1)

    def forward(self, x):
        y = [self.cv1(x)]
        y.extend(m(y[-1]) for m in [self.cv2, self.cv3, self.cv4])
        return self.cv5(torch.cat(y, 1))


class ELAN1(nn.Module):
    """cv1 split in two halves; cv2, cv3 chained on the second; concat; cv4 (common.py:580-598)."""

    def __init__(self, c1, c2, c3, c4):
        super().__init__()
        self.c = c3 // 2
        self.cv1 = Conv(c1, c3, 1, 1)
        self.cv2 = Conv(c3 // 2, c4, 3, 1)
        self.cv3 = Conv(c4, c4, 3, 1)
        self.cv4 = Conv(c3 + (2 * c4), c2, 1, 1)

    def forward(self, x):
        y = list(self.cv1(x).chunk(2, 1))
        y.extend(m(y[-1]) for m in [self.cv2, self.cv3])
        return self.cv4(torch.cat(y, 1))


class DFL(nn.Module):
    """Distribution focal loss integral: softmax over c1 bins, expectation of the
    bin index (common.py:232-244)."""

    def __init__(self, c1=17):
        super().__init__()
        self.conv = nn.Conv2d(c1, 1, 1, bias=False).requires_grad_(False)
        self.conv.weight.data[:] = torch.arange(c1, dtype=torch.float).view(1, c1, 1, 1)
        self.c1 = c1

    def forward(self, x):
        b, _, a = x.shape
        return self.conv(x.view(b, 4, self.c1, a).transpose(2, 1).softmax(1)).view(b, 4, a)


def fuse_conv_and_bn(conv, bn):
    """A biased conv equal to bn(conv(x)) in eval mode (KAD-CNet/utils/torch_utils.py:244-265)."""
    fused = nn.Conv2d(conv.in_channels, conv.out_channels, kernel_size=conv.kernel_size, stride=conv.stride,
                      padding=conv.padding, dilation=conv.dilation, groups=conv.groups,
                      bias=True).requires_grad_(False).to(conv.weight.device, conv.weight.dtype)
    scale = bn.weight.detach() / torch.sqrt(bn.running_var + bn.eps)
    fused.weight.copy_(conv.weight.detach() * scale.view(-1, 1, 1, 1))
    b = conv.bias.detach() if conv.bias is not None else torch.zeros_like(bn.running_mean)
    fused.bias.copy_((b - bn.running_mean) * scale + bn.bias.detach())
    return fused
