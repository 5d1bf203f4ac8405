"""KAD-CNet building blocks.

What has to match the reference (KAD-CNet/models/common.py) is the module tree: class names,
constructor arguments, attribute names and the order submodules are created in (so state dicts,
class-name discovery and seeded initialisation line up).  The forwards are written here from the
blocks' math:

  Conv     act(BN(conv_k,s,g,d(x))), 'same' padding d (k - 1) / 2; after fusion BN is gone
  AConv    Conv_3x3,s2(mean over each 2 x 2 window, stride 1, no padding)
  SPPELAN  t0 = cv1(x), t_{i+1} = maxpool_5x5,s1,pad2(t_i) for i < 3, cv5([t0 t1 t2 t3])
  ELAN1    h = cv1(x) split into halves a | b (a the larger for odd widths, as torch.chunk),
           c = cv2(b), d = cv3(c), cv4([a b c d])
  DFL      expected bin index under a softmax over each side's c1 logits

The HIP network forward lives in kadcnet.fast.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F


def make_divisible(x, divisor):
    """The smallest multiple of divisor that is >= x (KAD-CNet/utils/general.py:660-664)."""
    return int(math.ceil(x / divisor)) * divisor


def _same_padding(k, p, d):
    """Explicit padding p, or the padding that keeps the size at stride 1: half the dilated
    kernel extent d (k - 1) (per dimension for a tuple k)."""
    if p is not None:
        return p
    if isinstance(k, int):
        return d * (k - 1) // 2
    return [d * (e - 1) // 2 for e in k]


def _activation(act):
    if act is True:
        return nn.SiLU()
    return act if isinstance(act, nn.Module) else nn.Identity()


class Conv(nn.Module):
    """Convolution without bias, BatchNorm, activation (SiLU unless act says otherwise).
    DetectionModel.fuse folds the BatchNorm into a biased convolution and removes ``bn``."""

    def __init__(self, c1, c2, k=1, s=1, p=None, g=1, d=1, act=True):
        super().__init__()
        self.conv = nn.Conv2d(c1, c2, k, stride=s, padding=_same_padding(k, p, d), dilation=d, groups=g,
                              bias=False)
        self.bn = nn.BatchNorm2d(c2)
        self.act = _activation(act)

    def forward(self, x):
        y = self.conv(x)
        bn = getattr(self, 'bn', None)
        return self.act(y if bn is None else bn(y))


class AConv(nn.Module):
    """Downsampler: 2 x 2 window mean at stride 1, then a 3 x 3 stride-2 Conv."""

    def __init__(self, c1, c2):
        super().__init__()
        self.cv1 = Conv(c1, c2, 3, 2, 1)

    def forward(self, x):
        return self.cv1(F.avg_pool2d(x, kernel_size=2, stride=1))


class SP(nn.Module):
    """Max pool, stride 1, 'same' padding."""

    def __init__(self, k=3, s=1):
        super().__init__()
        self.m = nn.MaxPool2d(kernel_size=k, stride=s, padding=k // 2)

    def forward(self, x):
        return self.m(x)


class Concat(nn.Module):
    """Concatenation of a list of maps along dimension ``d``."""

    def __init__(self, dimension=1):
        super().__init__()
        self.d = dimension

    def forward(self, x):
        return torch.cat(list(x), dim=self.d)


class SPPELAN(nn.Module):
    """Spatial pyramid pooling: cv1, three chained 5 x 5 max pools, the four maps side by side, cv5."""

    def __init__(self, c1, c2, c3):
        super().__init__()
        self.c = c3
        self.cv1 = Conv(c1, c3, 1, 1)
        self.cv2 = SP(5)
        self.cv3 = SP(5)
        self.cv4 = SP(5)
        self.cv5 = Conv(4 * c3, c2, 1, 1)

    def forward(self, x):
        t = self.cv1(x)
        pyramid = [t]
        for pool in (self.cv2, self.cv3, self.cv4):
            t = pool(t)
            pyramid.append(t)
        return self.cv5(torch.cat(pyramid, dim=1))


def elan_forward(cv1, stage_a, stage_b, cv4, x):
    """The ELAN pattern shared by ELAN1 and RepNCSPELAN4_KADC: h = cv1(x) split into a | b
    (a = the first ceil(C / 2) channels), c = stage_a(b), d = stage_b(c), cv4([a b c d])."""
    h = cv1(x)
    k = (h.shape[1] + 1) // 2
    a, b = h[:, :k], h[:, k:]
    c = stage_a(b)
    d = stage_b(c)
    return cv4(torch.cat((a, b, c, d), dim=1))


class ELAN1(nn.Module):
    """ELAN with two plain 3 x 3 Convs on the second half of cv1's output."""

    def __init__(self, c1, c2, c3, c4):
        super().__init__()
        self.c = c3 // 2
        self.cv1 = Conv(c1, c3, 1, 1)
        self.cv2 = Conv(c3 // 2, c4, 3, 1)
        self.cv3 = Conv(c4, c4, 3, 1)
        self.cv4 = Conv(c3 + 2 * c4, c2, 1, 1)

    def forward(self, x):
        return elan_forward(self.cv1, self.cv2, self.cv3, self.cv4, x)


class DFL(nn.Module):
    """Box side distance from c1 bin logits: sum_k k softmax(l)_k.  The bin values are the weights
    of a frozen 1 x 1 conv (0, 1, ..., c1 - 1), as in the reference's state dict."""

    def __init__(self, c1=17):
        super().__init__()
        self.c1 = c1
        self.conv = nn.Conv2d(c1, 1, 1, bias=False).requires_grad_(False)
        with torch.no_grad():
            self.conv.weight.copy_(torch.arange(c1, dtype=torch.float32).view(1, c1, 1, 1))

    def forward(self, x):
        """x [B, 4 c1, A] -> [B, 4, A]."""
        b, _, n = x.shape
        p = x.view(b, 4, self.c1, n).softmax(dim=2)
        bins = self.conv.weight.view(1, 1, self.c1, 1).to(p.dtype)
        return (p * bins).sum(dim=2)


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
