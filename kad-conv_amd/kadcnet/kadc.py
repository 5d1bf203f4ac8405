"""KAD-CNet's KAD-Conv layers and the CSP-ELAN blocks built on them, under the reference's class
names (KAD-CNet/models/module/KADC/module.py:14-111).

KADC4 / KADC4_m are kadconv.KADConv with the reference's class names and channel-attention widths
(hidden >= 32 / >= 64): same parameters, same state-dict keys (module.py:14-68 has the module tree
of KAD-Conv/kadconv/kad_conv.py:81-121), so kadconv.enable_fast_inference finds them by class name.

  RepNCSP_KADC       cv3([m(cv1(x)) cv2(x)]), m = n KAD-Conv layers in sequence
  RepNCSPELAN4_KADC  the ELAN pattern (kadcnet.common.elan_forward) with (RepNCSP_KADC, 3 x 3 Conv)
                     as each of its two chained stages
"""
import torch
import torch.nn as nn

from kadconv import KADConv

from .common import Conv, elan_forward


class KADC4(KADConv):
    """KAD-Conv with channel-attention hidden width max(32, c)."""
    se_min_hidden = 32

    def __init__(self, dim, n=3):
        super().__init__(dim, n=n, se_min_hidden=self.se_min_hidden)


class KADC4_m(KADC4):
    """KAD-Conv with hidden width max(64, c) (the MGL configuration of KAD-CNet-S)."""
    se_min_hidden = 64


KAD_CONV_VARIANTS = {'KADC4': KADC4, 'KADC4_m': KADC4_m}


def _kadconv_class(variant):
    """KADC4 for None, else the class named (or given) by ``variant``."""
    if variant is None:
        return KADC4
    cls = KAD_CONV_VARIANTS.get(variant) if isinstance(variant, str) else variant
    if cls not in KAD_CONV_VARIANTS.values():
        raise ValueError(f'RepNCSP_KADC: kadc_variant must be one of {sorted(KAD_CONV_VARIANTS)}, got {variant!r}')
    return cls


class RepNCSP_KADC(nn.Module):
    """CSP block over n KAD-Conv layers of width c2 * e.  ``shortcut`` and ``g`` are accepted for
    the reference's signature; the KAD-Conv layers carry their own residual."""

    def __init__(self, c1, c2, n=1, shortcut=True, g=1, e=0.5, kadc_variant=None):
        super().__init__()
        hidden = int(c2 * e)
        self.cv1 = Conv(c1, hidden, 1, 1)
        self.cv2 = Conv(c1, hidden, 1, 1)
        self.cv3 = Conv(2 * hidden, c2, 1)
        layer = _kadconv_class(kadc_variant)
        self.m = nn.Sequential(*[layer(hidden) for _ in range(n)])

    def forward(self, x):
        t = self.cv1(x)
        for layer in self.m:
            t = layer(t)
        return self.cv3(torch.cat((t, self.cv2(x)), dim=1))


class RepNCSPELAN4_KADC(nn.Module):
    """GELAN block: cv1 (c1 -> c3) split in halves; two chained stages (RepNCSP_KADC with c5 KAD-Conv
    layers, then a 3 x 3 Conv) on the second half; cv4 over all four maps."""

    def __init__(self, c1, c2, c3, c4, c5=1, kadc_variant=None):
        super().__init__()
        self.c = c3 // 2
        self.cv1 = Conv(c1, c3, 1, 1)
        self.cv2 = nn.Sequential(RepNCSP_KADC(c3 // 2, c4, c5, kadc_variant=kadc_variant), Conv(c4, c4, 3, 1))
        self.cv3 = nn.Sequential(RepNCSP_KADC(c4, c4, c5, kadc_variant=kadc_variant), Conv(c4, c4, 3, 1))
        self.cv4 = Conv(c3 + 2 * c4, c2, 1, 1)

    def forward(self, x):
        return elan_forward(self.cv1, self.cv2, self.cv3, self.cv4, x)
