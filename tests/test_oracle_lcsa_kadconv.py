"""Pins the oracle's LCSA, DSC composition, KADConv and KADDown.

LCSA (kad_conv.py:18-39) is checked against its separable closed form written
with explicit numpy loops: with a[h] = mean_w x[h, :], b[w] = mean_h x[:, w],
the 1x11 depthwise conv of a[h] + b[w] equals a[h] * S(w) + B(w) + bias where
S(w) sums the in-image taps and B(w) is the 1-D conv of b.  KADConv is checked
for n=1 against a composition from torch modules built with the reference's
module list (kad_conv.py:100-110) and state-dict keys."""
import math

import numpy as np
import torch
import torch.nn as nn

from oracle import kadconv_oracle as O


def _lcsa_closed_form(sd, prefix, x):
    x = x.numpy()
    N, C, H, W = x.shape
    w1 = sd[prefix + 'excite.0.weight'].numpy().reshape(C, 11)
    b1 = sd[prefix + 'excite.0.bias'].numpy()
    g = sd[prefix + 'excite.1.weight'].numpy()
    be = sd[prefix + 'excite.1.bias'].numpy()
    rm = sd[prefix + 'excite.1.running_mean'].numpy()
    rv = sd[prefix + 'excite.1.running_var'].numpy()
    w3 = sd[prefix + 'excite.3.weight'].numpy().reshape(C, 11)
    b3 = sd[prefix + 'excite.3.bias'].numpy()
    w4 = sd[prefix + 'excite.4.weight'].numpy().reshape(9, C)
    b4 = sd[prefix + 'excite.4.bias'].numpy()
    out = np.zeros((N, 9, H, W))
    for n in range(N):
        u = np.zeros((C, H, W))
        for c in range(C):
            a = x[n, c].mean(axis=1)
            b = x[n, c].mean(axis=0)
            for w in range(W):
                S = sum(w1[c, k] for k in range(11) if 0 <= w + k - 5 < W)
                B = sum(w1[c, k] * b[w + k - 5] for k in range(11) if 0 <= w + k - 5 < W)
                for h in range(H):
                    t = a[h] * S + B + b1[c]
                    t = (t - rm[c]) / math.sqrt(rv[c] + 1e-3) * g[c] + be[c]
                    u[c, h, w] = max(t, 0.0)
        v = np.zeros((C, H, W))
        for c in range(C):
            for h in range(H):
                for k in range(11):
                    hh = h + k - 5
                    if 0 <= hh < H:
                        v[c, h] += w3[c, k] * u[c, hh]
            v[c] += b3[c]
        out[n] = np.einsum('jc,chw->jhw', w4, v) + b4[:, None, None]
    return torch.from_numpy(out)


def test_lcsa_matches_separable_closed_form():
    sd = O.make_dsc_state(6, 6, seed=3, dtype=torch.float64)
    x = torch.randn(2, 6, 13, 9, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    got = O.lcsa_forward(sd, 'RCA_mask.', x)
    ref = _lcsa_closed_form(sd, 'RCA_mask.', x)
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)


class _Scale(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(1, c, 1, 1))

    def forward(self, x):
        return x * self.weight


class _DSCProbe(nn.Module):
    """Holds DSC's parameters under the reference's names; forward uses the oracle's deform."""

    def __init__(self, c):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(c, c, 3, 3))
        self.bias = nn.Parameter(torch.empty(c))
        self.conv_offset = nn.Conv2d(c, 18, 3, padding=1)
        self.RCA_mask = nn.Module()
        self.RCA_mask.excite = nn.Sequential(
            nn.Conv2d(c, c, (1, 11), padding=(0, 5), groups=c), nn.BatchNorm2d(c, eps=1e-3), nn.ReLU(),
            nn.Conv2d(c, c, (11, 1), padding=(5, 0), groups=c), nn.Conv2d(c, 9, 1))

    def forward(self, x):
        off = self.conv_offset(x)
        pooled = nn.AdaptiveAvgPool2d((None, 1))(x) + nn.AdaptiveAvgPool2d((1, None))(x)
        mask = torch.sigmoid(self.RCA_mask.excite(pooled))
        return O.deform_conv2d(x, off, self.weight, self.bias, mask=mask)


def test_kadconv_one_branch_matches_module_composition():
    dim = 5
    sd = O.make_kadconv_state(dim, n=1, se_min_hidden=8, seed=2, dtype=torch.float64)
    conv = nn.Sequential(nn.Conv2d(dim, dim, 1), _DSCProbe(dim), nn.BatchNorm2d(dim, eps=1e-3), nn.ReLU())
    fc = nn.Sequential(nn.Linear(dim, 8), nn.ReLU(), nn.Linear(8, dim), nn.Sigmoid())
    holder = nn.Module()
    holder.convs = nn.ModuleList([conv])
    holder.fc = nn.ModuleList([fc])
    holder.weight = nn.ModuleList([nn.Sequential(_Scale(dim))])
    holder = holder.double().eval()
    missing, unexpected = holder.load_state_dict(sd, strict=False)
    assert not unexpected and all(k.endswith('num_batches_tracked') for k in missing)
    x = torch.randn(2, dim, 7, 6, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    with torch.no_grad():
        y = holder.weight[0](conv(x))
        ref = y * fc(y.mean(dim=(2, 3))).view(2, -1, 1, 1) + x
    got = O.kadconv_forward(sd, x, n=1)
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)


def test_kadconv_state_keys_match_reference_layout():
    sd = O.make_kadconv_state(64)
    assert O.branch_widths(64) == [22, 21, 21]
    assert O.branch_widths(256) == [86, 85, 85]
    for i, c in enumerate([22, 21, 21]):
        assert sd[f'convs.{i}.0.weight'].shape == (c, 64, 1, 1)
        assert sd[f'convs.{i}.1.weight'].shape == (c, c, 3, 3)
        assert sd[f'convs.{i}.1.conv_offset.weight'].shape == (18, c, 3, 3)
        assert sd[f'convs.{i}.1.RCA_mask.excite.0.weight'].shape == (c, 1, 1, 11)
        assert sd[f'convs.{i}.1.RCA_mask.excite.3.weight'].shape == (c, 1, 11, 1)
        assert sd[f'convs.{i}.1.RCA_mask.excite.4.weight'].shape == (9, c, 1, 1)
        assert sd[f'fc.{i}.0.weight'].shape == (max(32, c), c)
        assert sd[f'weight.{i}.0.weight'].shape == (1, c, 1, 1)


def test_kaddown_collapses_to_single_conv_on_blockwise_constant_input():
    # With equal branch weights and an input constant on every 8x8 block, every
    # pyramid level upsamples back to the same map, so the softmax mixture
    # reduces to one 1x1 convolution of the 2x2-pooled input, gated.
    c1, c2 = 4, 6
    sd = O.make_kaddown_state(c1, c2, seed=1, dtype=torch.float64)
    for i in (1, 2):
        sd[f'proj.{i}.weight'] = sd['proj.0.weight'].clone()
        sd[f'proj.{i}.bias'] = sd['proj.0.bias'].clone()
    g = torch.Generator().manual_seed(0)
    base = torch.randn(1, c1, 1, 1, generator=g, dtype=torch.float64)
    x = base.expand(1, c1, 32, 32).clone()
    got = O.kaddown_forward(sd, x)
    ref = torch.nn.functional.conv2d(x[:, :, ::2, ::2], sd['proj.0.weight'], sd['proj.0.bias'])
    ref = ref * torch.sigmoid(sd['gate']).view(1, -1, 1, 1)
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)
