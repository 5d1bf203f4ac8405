"""CPU restatement of the reference's plain-PyTorch KAD-Conv forward.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline) -- never as the thing measured or shipped.
The product package (``kad-conv_amd/kadconv``) never imports it.

Everything here is a functional restatement driven by a state dict whose keys
are the reference's parameter names (``KAD-Conv/kadconv/kad_conv.py:18-121``;
the same names are used by ``KAD-CNet/models/module/KADC/module.py:14-68`` and
``KAD-CNet/models/module/ops.py:12-72``).  It runs in whatever floating dtype the
inputs carry (float32 for the baseline, float64 for golden fixtures).

torchvision is absent on both machines, so ``torchvision.ops.deform_conv2d``
(called at ``kad_conv.py:66-67``; pinned torchvision 0.16.2,
``KAD-CNet/README.md:20,25``) is restated from the reference's own description
of its sampling rule at ``acceleration/kadc_dcn_direct.py:57-107`` and
``acceleration/kadc_dcn16_kernel.cu:206-266``.

Pins (see tests/test_oracle_*.py): the deformable convolution is checked
against an independent ``grid_sample`` formulation, a float64 brute-force C
loop (``oracle/dcn_brute.c``) and closed-form special cases (zero offsets with
unit mask equal ``conv2d``; integer offsets equal a shifted ``conv2d``; mask 0
gives the bias; linearity in the mask).  LCSA is checked against its separable
closed form computed with numpy loops.  KADConv with one branch is checked
against a composition written from the module list.  ``kaddown_forward`` (a
builder-defined operator with no counterpart in the reference) is pinned by
its closed-form collapse to a single 1x1 convolution when the branches share
weights and the input is constant per 8x8 block.
"""
import torch
import torch.nn.functional as F

BN_EPS = 1e-3  # KAD-Conv/kadconv/kad_conv.py:14 (and KAD-CNet/utils/torch_utils.py:214)


# --------------------------------------------------------------------------- #
# Modulated deformable convolution (DCNv2), torchvision semantics.
# --------------------------------------------------------------------------- #
def _bilinear_gather(img, py, px):
    """Zero-padded bilinear sample of ``img`` [N, C, H, W] at float positions
    ``py``/``px`` [N, P] -> [N, C, P].

    The rule follows kadc_dcn_direct.py:65-102: a sample whose position is
    ``<= -1`` or ``>= size`` on either axis is 0; otherwise the four corners
    around ``floor(p)`` are blended and corners outside the image read 0.
    """
    N, C, H, W = img.shape
    valid = (py > -1) & (py < H) & (px > -1) & (px < W)
    y0 = torch.floor(py)
    x0 = torch.floor(px)
    ly = py - y0
    lx = px - x0
    hy = 1 - ly
    hx = 1 - lx
    y0 = y0.long()
    x0 = x0.long()
    y1 = y0 + 1
    x1 = x0 + 1
    flat = img.reshape(N, C, H * W)
    out = torch.zeros(N, C, py.shape[1], dtype=img.dtype)
    for yy, xx, wgt in ((y0, x0, hy * hx), (y0, x1, hy * lx), (y1, x0, ly * hx), (y1, x1, ly * lx)):
        ok = valid & (yy >= 0) & (yy < H) & (xx >= 0) & (xx < W)
        idx = (yy.clamp(0, H - 1) * W + xx.clamp(0, W - 1))
        vals = torch.gather(flat, 2, idx.unsqueeze(1).expand(N, C, idx.shape[1]))
        out += vals * (wgt * ok.to(img.dtype)).unsqueeze(1)
    return out


def deform_conv2d(x, offset, weight, bias=None, stride=1, padding=1, dilation=1, mask=None):
    """Restates ``torchvision.ops.deform_conv2d`` for one offset group.

    out[n,co,oy,ox] = bias[co] + sum_{ci,k} W[co,ci,k] * m[n,k,oy,ox] * bil(x[n,ci], py, px)
    with py = oy*s - pad + ky*dil + offset[n,2k], px = ox*s - pad + kx*dil + offset[n,2k+1],
    k = ky*KW + kx (kad_conv.py:66-67; sampling rule kadc_dcn_direct.py:57-107).
    """
    s = (stride, stride) if isinstance(stride, int) else tuple(stride)
    p = (padding, padding) if isinstance(padding, int) else tuple(padding)
    d = (dilation, dilation) if isinstance(dilation, int) else tuple(dilation)
    N, Ci, H, W = x.shape
    Co, Ci_w, KH, KW = weight.shape
    assert Ci_w == Ci, 'one weight group only'
    Ho = (H + 2 * p[0] - d[0] * (KH - 1) - 1) // s[0] + 1
    Wo = (W + 2 * p[1] - d[1] * (KW - 1) - 1) // s[1] + 1
    K = KH * KW
    assert offset.shape == (N, 2 * K, Ho, Wo), offset.shape
    if mask is not None:
        assert mask.shape == (N, K, Ho, Wo), mask.shape
    oy = (torch.arange(Ho, dtype=x.dtype) * s[0] - p[0]).view(1, Ho, 1)
    ox = (torch.arange(Wo, dtype=x.dtype) * s[1] - p[1]).view(1, 1, Wo)
    wmat = weight.reshape(Co, Ci * K)
    out = torch.empty(N, Co, Ho * Wo, dtype=x.dtype)
    for n in range(N):  # one image at a time bounds the column buffer
        cols = torch.empty(Ci, K, Ho * Wo, dtype=x.dtype)
        for k in range(K):
            ky, kx = divmod(k, KW)
            py = (oy + ky * d[0] + offset[n:n + 1, 2 * k]).reshape(1, -1)
            px = (ox + kx * d[1] + offset[n:n + 1, 2 * k + 1]).reshape(1, -1)
            v = _bilinear_gather(x[n:n + 1], py, px)[0]
            if mask is not None:
                v = v * mask[n, k].reshape(1, -1)
            cols[:, k] = v
        out[n] = wmat @ cols.reshape(Ci * K, Ho * Wo)
    if bias is not None:
        out += bias.view(1, Co, 1)
    return out.view(N, Co, Ho, Wo)


def deform_conv2d_gridsample(x, offset, weight, bias=None, stride=1, padding=1, mask=None):
    """Independent formulation through ``F.grid_sample`` (zeros padding,
    align_corners=True maps normalised -1/+1 onto pixel centres 0 and size-1,
    which reproduces the zero-padded bilinear rule above for H, W > 1)."""
    N, Ci, H, W = x.shape
    Co, _, KH, KW = weight.shape
    Ho, Wo = offset.shape[2:]
    oy = torch.arange(Ho, dtype=x.dtype).view(Ho, 1) * stride - padding
    ox = torch.arange(Wo, dtype=x.dtype).view(1, Wo) * stride - padding
    out = torch.zeros(N, Co, Ho, Wo, dtype=x.dtype)
    for k in range(KH * KW):
        ky, kx = divmod(k, KW)
        py = oy + ky + offset[:, 2 * k]
        px = ox + kx + offset[:, 2 * k + 1]
        grid = torch.stack((2 * px / (W - 1) - 1, 2 * py / (H - 1) - 1), dim=-1)
        v = F.grid_sample(x, grid, mode='bilinear', padding_mode='zeros', align_corners=True)
        if mask is not None:
            v = v * mask[:, k:k + 1]
        out += torch.einsum('oc,nchw->nohw', weight[:, :, ky, kx], v)
    if bias is not None:
        out += bias.view(1, Co, 1, 1)
    return out


# --------------------------------------------------------------------------- #
# LCSA, DSC, KADConv (kad_conv.py:18-121)
# --------------------------------------------------------------------------- #
def _bn(x, sd, prefix, eps=BN_EPS):
    return F.batch_norm(x, sd[prefix + 'running_mean'], sd[prefix + 'running_var'],
                        sd[prefix + 'weight'], sd[prefix + 'bias'], False, 0.0, eps)


def lcsa_forward(sd, prefix, x, band=11):
    """LCSA.forward (kad_conv.py:38-39): excite(pool_h(x) + pool_w(x)), pre-sigmoid."""
    C = x.shape[1]
    s = x.mean(dim=3, keepdim=True) + x.mean(dim=2, keepdim=True)   # AdaptiveAvgPool2d((None,1)) + ((1,None))
    t = F.conv2d(s, sd[prefix + 'excite.0.weight'], sd[prefix + 'excite.0.bias'],
                 padding=(0, band // 2), groups=C)                      # kad_conv.py:29-30
    t = torch.relu(_bn(t, sd, prefix + 'excite.1.'))                    # :31-32
    t = F.conv2d(t, sd[prefix + 'excite.3.weight'], sd[prefix + 'excite.3.bias'],
                 padding=(band // 2, 0), groups=C)                      # :33-34
    return F.conv2d(t, sd[prefix + 'excite.4.weight'], sd[prefix + 'excite.4.bias'])  # :35


def dsc_forward(sd, prefix, x, stride=1, padding=1):
    """DSC.forward (kad_conv.py:63-67)."""
    offset = F.conv2d(x, sd[prefix + 'conv_offset.weight'], sd[prefix + 'conv_offset.bias'],
                      stride=stride, padding=padding)
    mask = torch.sigmoid(lcsa_forward(sd, prefix + 'RCA_mask.', x))
    return deform_conv2d(x, offset, sd[prefix + 'weight'], sd[prefix + 'bias'],
                         stride=stride, padding=padding, mask=mask)


def branch_widths(dim, n=3):
    """kad_conv.py:99."""
    return [dim - (dim // n) * (n - 1)] + [dim // n] * (n - 1)


def kadconv_branch(sd, i, x):
    """Branch i of KADConv.forward up to (and including) the channel attention,
    before the upsample (kad_conv.py:115-117)."""
    y = F.avg_pool2d(x, kernel_size=2 ** i) if i > 0 else x
    p = f'convs.{i}.'
    y = F.conv2d(y, sd[p + '0.weight'], sd[p + '0.bias'])
    y = dsc_forward(sd, p + '1.', y)
    y = torch.relu(_bn(y, sd, p + '2.'))
    y = y * sd[f'weight.{i}.0.weight']
    g = y.mean(dim=(2, 3))
    h = torch.relu(F.linear(g, sd[f'fc.{i}.0.weight'], sd[f'fc.{i}.0.bias']))
    a = torch.sigmoid(F.linear(h, sd[f'fc.{i}.2.weight'], sd[f'fc.{i}.2.bias']))
    return y * a.view(x.shape[0], -1, 1, 1)


def kadconv_forward(sd, x, n=3):
    """KADConv.forward (kad_conv.py:112-121)."""
    feats = []
    for i in range(n):
        y = kadconv_branch(sd, i, x)
        if i > 0:
            y = F.interpolate(y, size=x.shape[2:], mode='bilinear', align_corners=False)
        feats.append(y)
    return torch.cat(feats, dim=1) + x


# --------------------------------------------------------------------------- #
# Fused blocks (BASELINE configs 4a/4b)
# --------------------------------------------------------------------------- #
def conv1x1_silu(x, weight, bias):
    """KAD-CNet ``Conv`` after Conv-BN fusion with SiLU (models/common.py:43-57):
    SiLU(W x + b), W [Co, Ci] or [Co, Ci, 1, 1]."""
    w = weight.reshape(weight.shape[0], -1, 1, 1)
    return F.silu(F.conv2d(x, w, bias))


def se_forward(x, w1, b1, w2, b2):
    """Squeeze-excitation as in KADConv's channel attention (kad_conv.py:105-109,117):
    y = x * sigmoid(W2 relu(W1 mean_hw(x) + b1) + b2)."""
    g = x.mean(dim=(2, 3))
    a = torch.sigmoid(F.linear(torch.relu(F.linear(g, w1, b1)), w2, b2))
    return x * a.view(x.shape[0], x.shape[1], 1, 1)


# --------------------------------------------------------------------------- #
# KADDown: builder-defined stride-2 multi-branch downsampling (no counterpart
# in the reference; assembled from KADConv's branch structure, kad_conv.py:112-121,
# the one-pass pyramid pool idea of acceleration/kadc_fused_sm75.py:653-692 and
# the stride-2 downsamplers of KAD-CNet/models/common.py:60-83).
# --------------------------------------------------------------------------- #
def kaddown_forward(sd, x, n=3):
    """y = sigmoid(gate) * sum_i softmax(alpha)_i * up_i(conv1x1_i(avgpool(x, 2^(i+1))))

    up_i is bilinear (align_corners=False) to (H//2, W//2); branch 0 needs none.
    Keys: ``proj.{i}.weight`` [C2,C1,1,1], ``proj.{i}.bias`` [C2], ``alpha`` [n],
    ``gate`` [C2]."""
    Ho, Wo = x.shape[2] // 2, x.shape[3] // 2
    a = torch.softmax(sd['alpha'], dim=0)
    z = None
    for i in range(n):
        p = F.avg_pool2d(x, kernel_size=2 ** (i + 1))
        b = F.conv2d(p, sd[f'proj.{i}.weight'], sd[f'proj.{i}.bias'])
        if b.shape[2:] != (Ho, Wo):
            b = F.interpolate(b, size=(Ho, Wo), mode='bilinear', align_corners=False)
        z = a[i] * b if z is None else z + a[i] * b
    return z * torch.sigmoid(sd['gate']).view(1, -1, 1, 1)
