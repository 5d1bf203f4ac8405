"""KAD-CNet's KAD-Conv layers and the CSP-ELAN blocks built on them, with the
reference's class names (KAD-CNet/models/module/KADC/module.py:14-111).

KADC4 / KADC4_m are kadconv.KADConv with the reference's class names and
channel-attention widths (hidden >= 32 / >= 64): same parameters, same
state-dict keys (module.py:14-68 has the same module tree as
KAD-Conv/kadconv/kad_conv.py:81-121), so kadconv.enable_fast_inference finds
them by class name.
"""
import torch
import torch.nn as nn

from kadconv import KADConv

from .common import Conv


class KADC4(KADConv):
    """KAD-Conv with channel-attention hidden width max(32, c) (module.py:14-61)."""
    se_min_hidden = 32

    def __init__(self, dim, n=3):
        super().__init__(dim, n=n, se_min_hidden=self.se_min_hidden)


class KADC4_m(KADC4):
    """KAD-Conv with hidden width max(64, c), used by KAD-CNet-S with MGL (module.py:64-68)."""
    se_min_hidden = 64


KAD_CONV_VARIANTS = {'KADC4': KADC4, 'KADC4_m': KADC4_m}


class RepNCSP_KADC(nn.Module):
    """CSP bottleneck over n KAD-Conv layers (module.py:74-89):
    cv3(cat(m(cv1(x)), cv2(x)))."""

    def __init__(self, c1, c2, n=1, shortcut=True, g=1, e=0.5, kadc_variant=None):
        super().__init__()
        c_ = int(c2 * e)
        self.cv1 = Conv(c1, c_, 1, 1)
        self.cv2 = Conv(c1, c_, 1, 1)
        self.cv3 = Conv(2 * c_, c2, 1)
        block = KAD_CONV_VARIANTS[kadc_variant] if isinstance(kadc_variant, str) else (kadc_variant or KADC4)
        if block not in KAD_CONV_VARIANTS.values():
            raise ValueError(f'unsupported KAD-Conv variant: {kadc_variant}')
        self.m = nn.Sequential(*(block(c_) for _ in range(n)))

    def forward(self, x):
        return self.cv3(torch.cat((self.m(self.cv1(x)), self.cv2(x)), 1))


class RepNCSPELAN4_KADC(nn.Module):
    """GELAN block with KAD-Conv in both computational branches (module.py:92-111):
    cv1 split in halves; cv2 = (RepNCSP_KADC, 3x3 Conv) on the second half,
    cv3 = the same on cv2's output; cv4 over the concat of all four."""

    def __init__(self, c1, c2, c3, c4, c5=1, kadc_variant=None):
        super().__init__()
        self.c = c3 // 2
        self.cv1 = Conv(c1, c3, 1, 1)
        self.cv2 = nn.Sequential(RepNCSP_KADC(c3 // 2, c4, c5, kadc_variant=kadc_variant), Conv(c4, c4, 3, 1))
        self.cv3 = nn.Sequential(RepNCSP_KADC(c4, c4, c5, kadc_variant=kadc_variant), Conv(c4, c4, 3, 1))
        self.cv4 = Conv(c3 + (2 * c4), c2, 1, 1)

    def forward(self, x):
        y = list(self.cv1(x).chunk(2, 1))
        y.extend(m(y[-1]) for m in [self.cv2, self.cv3])
        return self.cv4(torch.cat(y, 1))
