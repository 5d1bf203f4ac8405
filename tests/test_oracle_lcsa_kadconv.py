"""Pins the oracle's LCSA, DSC composition, KADConv and KADDown.

LCSA (kad_conv.py:18-39) is checked against its separable closed form written
with explicit numpy loops: with a[h] = mean_w x[h, :], b[w] = mean_h x[:, w],
the 1x11 depthwise conv of a[h] + b[w] equals a[h] * S(w) + B(w) + bias where
S(w) sums the in-image taps and B(w) is the 1-D conv of b.  KADConv is checked
for n=1 against a composition from torch modules built with the reference's
module list (kad_conv.py:100-110) and state-dict keys.  KADDown (builder-defined)
is pinned on linear inputs: block means and the bilinear resize are exact on
lines, so each branch has a closed form whose border clamping fixes its pool
factor and resize rule; one-hot mixture logits fix the logit / branch pairing."""
import math

import numpy as np
import pytest
import torch
import torch.nn as nn

from kadconv import synthetic as S
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
    sd = S.make_dsc_state(6, 6, seed=3, dtype=torch.float64)
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
    sd = S.make_kadconv_state(dim, n=1, se_min_hidden=8, seed=2, dtype=torch.float64)
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
    sd = S.make_kadconv_state(64)
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
    sd = S.make_kaddown_state(c1, c2, seed=1, dtype=torch.float64)
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


def _sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


@pytest.mark.parametrize('istar', [0, 1, 2])
def test_kaddown_ramp_pins_pool_factor_resize_rule_and_branch_order(istar):
    """Branch i of KADDown averages 2^(i+1) x 2^(i+1) blocks and resizes the result bilinearly
    (align_corners=False) to (H/2, W/2).  On a linear input x_c = a_c + b_c h + d_c w both steps
    are exact on lines: a block mean samples the line at the block centre, and the resize places
    output row j at source position 2 j + 0.5 of the full-resolution grid, clamped to the centre
    range [e_i, H - 1 - e_i] of the pooled samples, e_i = (2^(i+1) - 1) / 2.  So branch i at
    (j, k) is W_i L(clamp(2 j + 0.5, e_i, H - 1 - e_i), clamp(2 k + 0.5, e_i, W - 1 - e_i)) + b_i,
    computed here with numpy.  One-hot mixture logits (+-30) select branch istar, and each branch
    has its own weights: a wrong pool factor (2^i), align_corners=True, a swapped logit / branch
    pairing or a missing gate each move the result by more than the 1e-9 bound."""
    c1, c2, H, W = 3, 4, 32, 40
    sd = S.make_kaddown_state(c1, c2, seed=11, dtype=torch.float64)
    sd['alpha'] = torch.full((3,), -30.0, dtype=torch.float64)
    sd['alpha'][istar] = 30.0
    g = torch.Generator().manual_seed(12)
    a = torch.rand(c1, generator=g, dtype=torch.float64)
    b = torch.rand(c1, generator=g, dtype=torch.float64) * 0.3
    d = torch.rand(c1, generator=g, dtype=torch.float64) * 0.3 - 0.15
    hh = torch.arange(H, dtype=torch.float64).view(1, H, 1)
    ww = torch.arange(W, dtype=torch.float64).view(1, 1, W)
    x = (a.view(c1, 1, 1) + b.view(c1, 1, 1) * hh + d.view(c1, 1, 1) * ww).unsqueeze(0)
    got = O.kaddown_forward(sd, x)[0].numpy()
    e = (2 ** (istar + 1) - 1) / 2
    ph = np.clip(2 * np.arange(H // 2) + 0.5, e, H - 1 - e)
    pw = np.clip(2 * np.arange(W // 2) + 0.5, e, W - 1 - e)
    lines = a.numpy()[:, None, None] + b.numpy()[:, None, None] * ph[None, :, None] + d.numpy()[:, None, None] * pw[None, None, :]
    wi = sd[f'proj.{istar}.weight'].numpy().reshape(c2, c1)
    ref = np.einsum('oc,chw->ohw', wi, lines) + sd[f'proj.{istar}.bias'].numpy()[:, None, None]
    ref = ref / (1.0 + np.exp(-sd['gate'].numpy()))[:, None, None]
    assert got.shape == (c2, H // 2, W // 2)
    assert np.abs(got - ref).max() <= 1e-9, np.abs(got - ref).max()


def test_kadconv_three_branches_zero_dsc_weights_give_constant_branches():
    """n = 3 pin of the concat order and widths, residual, BN, ReLU, branch scale
    and SE MLP: with every DSC weight 0 the DSC returns its bias, so branch i is
    the per-channel constant v_i = scale * relu(bn(bias_i)), gated by
    att_i = sigmoid(W2 relu(W1 v_i + b1) + b2) (the mean of a constant map is the
    constant; its bilinear upsample is the same constant).  Expected output:
    cat_i(v_i * att_i) + x, computed here with numpy from the state dict."""
    dim = 14
    sd = S.make_kadconv_state(dim, seed=5, dtype=torch.float64)
    for i in range(3):
        sd[f'convs.{i}.1.weight'].zero_()
    x = torch.randn(2, dim, 12, 16, generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    got = O.kadconv_forward(sd, x)
    consts = []
    for i, c in enumerate(O.branch_widths(dim)):
        p = f'convs.{i}.'
        n = lambda k: sd[k].numpy().reshape(-1)  # noqa: E731
        t = (n(p + '1.bias') - n(p + '2.running_mean')) / np.sqrt(n(p + '2.running_var') + 1e-3) \
            * n(p + '2.weight') + n(p + '2.bias')
        v = np.maximum(t, 0.0) * n(f'weight.{i}.0.weight')
        hdn = np.maximum(sd[f'fc.{i}.0.weight'].numpy() @ v + n(f'fc.{i}.0.bias'), 0.0)
        att = _sigmoid(sd[f'fc.{i}.2.weight'].numpy() @ hdn + n(f'fc.{i}.2.bias'))
        assert len(v) == c
        consts.append(v * att)
    ref = torch.from_numpy(np.concatenate(consts)).view(1, dim, 1, 1) + x
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)


def test_kadconv_three_branches_pool_factor_and_upsample_rule():
    """n = 3 pin of the per-branch pool factor 2^i and the bilinear upsample
    rule (align_corners=False).  Every stage is made a known positive scaling:
    branch i's projection selects input channels [c_off_i, c_off_i + c_i); the
    DSC has zero offsets, a centre-tap identity weight and a constant mask
    m = sigmoid(b4) (LCSA's last 1x1 weight 0); BN is identity up to
    1/sqrt(1 + eps); the SE weights are 0 so att = sigmoid(b2).  The input is
    linear, x = a + b h + c w > 0.  Average-pooling a linear map by s samples it
    at the block centres s k + (s - 1)/2, and upsampling those samples back
    (src = (j + 0.5)/s - 0.5, clamped to the sample range) reproduces the line
    inside and holds its end values outside, so branch i equals
    a + b clamp(h, e, H - 1 - e) + c clamp(w, e, W - 1 - e), e = (2^i - 1)/2,
    times the stage gains: the border width pins s = 2^i, the clamping pins the
    align_corners=False rule, the channel windows pin the concat order."""
    dim, H, W = 9, 16, 24
    widths = O.branch_widths(dim)
    sd = S.make_kadconv_state(dim, seed=8, dtype=torch.float64)
    gains = []
    c_off = 0
    for i, c in enumerate(widths):
        p = f'convs.{i}.'
        sel = torch.zeros(c, dim, 1, 1, dtype=torch.float64)
        for j in range(c):
            sel[j, c_off + j] = 1.0
        sd[p + '0.weight'], sd[p + '0.bias'] = sel, torch.zeros(c, dtype=torch.float64)
        w = torch.zeros(c, c, 3, 3, dtype=torch.float64)
        for j in range(c):
            w[j, j, 1, 1] = 1.0
        sd[p + '1.weight'], sd[p + '1.bias'] = w, torch.zeros(c, dtype=torch.float64)
        sd[p + '1.conv_offset.weight'].zero_()
        sd[p + '1.conv_offset.bias'].zero_()
        sd[p + '1.RCA_mask.excite.4.weight'].zero_()
        b4 = sd[p + '1.RCA_mask.excite.4.bias'].numpy()
        for k, v in (('weight', 1.0), ('bias', 0.0), ('running_mean', 0.0), ('running_var', 1.0)):
            sd[p + '2.' + k] = torch.full((c,), v, dtype=torch.float64)
        sd[f'fc.{i}.0.weight'].zero_()
        sd[f'fc.{i}.2.weight'].zero_()
        att = _sigmoid(sd[f'fc.{i}.2.bias'].numpy())
        scale = sd[f'weight.{i}.0.weight'].numpy().reshape(-1)
        gains.append(_sigmoid(b4[4]) / math.sqrt(1 + 1e-3) * scale * att)
        c_off += c
    g = torch.Generator().manual_seed(9)
    a = torch.rand(dim, generator=g, dtype=torch.float64) + 0.5
    b = torch.rand(dim, generator=g, dtype=torch.float64) * 0.2
    cc = torch.rand(dim, generator=g, dtype=torch.float64) * 0.2
    hh = torch.arange(H, dtype=torch.float64).view(1, H, 1)
    ww = torch.arange(W, dtype=torch.float64).view(1, 1, W)
    x = (a.view(dim, 1, 1) + b.view(dim, 1, 1) * hh + cc.view(dim, 1, 1) * ww).unsqueeze(0)
    got = O.kadconv_forward(sd, x)
    ref = x.clone()
    c_off = 0
    for i, c in enumerate(widths):
        e = (2 ** i - 1) / 2
        lin = a.view(dim, 1, 1) + b.view(dim, 1, 1) * hh.clamp(e, H - 1 - e) + cc.view(dim, 1, 1) * ww.clamp(e, W - 1 - e)
        ref[0, c_off:c_off + c] += torch.from_numpy(gains[i]).view(c, 1, 1) * lin[c_off:c_off + c]
        c_off += c
    assert torch.allclose(got, ref, atol=1e-12, rtol=0), (got - ref).abs().max()
