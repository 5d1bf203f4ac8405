"""Functional operators backed by libkadconv_hip.so.

* ``deform_conv2d`` -- drop-in for ``torchvision.ops.deform_conv2d`` (the call
  at KAD-Conv/kadconv/kad_conv.py:66-67) for 3x3 kernels, one offset group,
  dilation 1.  GPU tensors run the gfx950 HIP kernel; CPU tensors run a
  plain-torch im2col restatement (any kernel size, stride, dilation).
* ``conv1x1`` -- 1x1 conv + bias + optional SiLU, optional input avg-pool
  (north-star piece 3; KAD-CNet ``Conv`` after Conv-BN fusion).
* ``squeeze_excitation`` -- SE block: GAP, FC-ReLU-FC-sigmoid, channel scale.

GPU entry points never fall back to another implementation: if the HIP library
is missing they raise ``kadconv._ext.KadExtensionError``.
"""
import torch
import torch.nn.functional as F

from . import _ext


def _nhwc_view(x):
    """Return (tensor [N,H,W,cs], cs) usable by the DCN kernels, converting with
    the HIP transpose when x is not already channels-last with cs % 8 == 0."""
    N, C, H, W = x.shape
    if x.is_contiguous(memory_format=torch.channels_last) and C % 8 == 0 and C > 1:
        return x.permute(0, 2, 3, 1), C
    cs = (C + 7) // 8 * 8
    out = torch.empty(N, H, W, cs, dtype=x.dtype, device=x.device)
    v = x.permute(0, 2, 3, 1)
    vs = v.stride()
    if (vs[3] == 1 and vs[2] >= C and vs[1] == vs[2] * W and vs[0] == vs[1] * H):
        _ext.nhwc_pad(v, out)        # channels-last (or a channel slice of one): one padding pass
    else:
        _ext.to_nhwc(x.contiguous(), out)
    return out, cs


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def _deform_conv2d_cpu(x, offset, weight, bias, s, p, d, mask):
    """Plain-torch modulated deformable convolution for CPU tensors (the
    reference's CPU path is torchvision's operator, absent here).

    Sampling rule of torchvision (restated at acceleration/kadc_dcn_direct.py:57-107):
    a sample at (py, px) is 0 if py <= -1, py >= H, px <= -1 or px >= W;
    otherwise the four corners around floor(p) are blended and corners
    outside the image read 0.  Here the image is zero-padded by one pixel on
    every side, so for every live sample all four corners (rows floor(py)
    and floor(py) + 1 in [-1, H]) index the padded image and the outside
    corners read the padding: one flat gather per corner, no per-corner
    validity.  The columns [N, Cin * KH * KW, P] then meet the weights in one
    batched matmul (im2col, the torchvision strategy)."""
    N, C, H, W = x.shape
    Co, Ci, KH, KW = weight.shape
    Ho, Wo = offset.shape[2:]
    K = KH * KW
    dt = x.dtype
    xp = F.pad(x, (1, 1, 1, 1)).reshape(N, C, (H + 2) * (W + 2))
    base_y = (torch.arange(Ho, dtype=dt) * s[0] - p[0]).view(1, 1, Ho, 1)
    base_x = (torch.arange(Wo, dtype=dt) * s[1] - p[1]).view(1, 1, 1, Wo)
    ky = (torch.arange(K) // KW).to(dt).view(1, K, 1, 1) * d[0]
    kx = (torch.arange(K) % KW).to(dt).view(1, K, 1, 1) * d[1]
    off = offset.reshape(N, K, 2, Ho, Wo)
    py = base_y + ky + off[:, :, 0]                     # [N, K, Ho, Wo]
    px = base_x + kx + off[:, :, 1]
    live = (py > -1) & (py < H) & (px > -1) & (px < W)
    py = torch.where(live, py, torch.zeros_like(py))    # dead samples: any in-range position, weight 0
    px = torch.where(live, px, torch.zeros_like(px))
    fy, fx = torch.floor(py), torch.floor(px)
    ly, lx = py - fy, px - fx
    r0 = fy.long() + 1                                  # padded row of floor(py), in [0, H]
    c0 = fx.long() + 1
    gain = live.to(dt) if mask is None else live.to(dt) * mask.reshape(N, K, Ho, Wo)
    cols = x.new_zeros(N, C, K * Ho * Wo)
    for dy, dx, wgt in ((0, 0, (1 - ly) * (1 - lx)), (0, 1, (1 - ly) * lx), (1, 0, ly * (1 - lx)), (1, 1, ly * lx)):
        idx = ((r0 + dy) * (W + 2) + (c0 + dx)).reshape(N, 1, -1).expand(N, C, -1)
        cols += torch.gather(xp, 2, idx) * (wgt * gain).reshape(N, 1, -1)
    cols = cols.reshape(N, C * K, Ho * Wo)               # row ci * K + k: weight's [Ci][KH][KW] order
    out = torch.matmul(weight.reshape(Co, Ci * K), cols)
    if bias is not None:
        out = out + bias.view(1, Co, 1)
    return out.reshape(N, Co, Ho, Wo)


def deform_conv2d(input, offset, weight, bias=None, stride=1, padding=0, dilation=1, mask=None):
    """Modulated deformable convolution with torchvision's signature and semantics.
    GPU tensors run the gfx950 HIP kernel; CPU tensors run a plain-torch
    restatement of the same sampling rule (the reference's CPU path is
    torchvision's operator, which this image does not ship)."""
    if not input.is_cuda:
        s, p, d = _pair(stride), _pair(padding), _pair(dilation)
        if input.dim() != 4 or weight.dim() != 4 or weight.shape[1] != input.shape[1]:
            raise ValueError('input [N, C, H, W] and weight [Cout, C, KH, KW] (one weight group) expected')
        KH, KW = weight.shape[2:]
        Ho = (input.shape[2] + 2 * p[0] - d[0] * (KH - 1) - 1) // s[0] + 1
        Wo = (input.shape[3] + 2 * p[1] - d[1] * (KW - 1) - 1) // s[1] + 1
        if tuple(offset.shape) != (input.shape[0], 2 * KH * KW, Ho, Wo):
            raise ValueError(f'offset shape {tuple(offset.shape)} != {(input.shape[0], 2 * KH * KW, Ho, Wo)}')
        if mask is not None and tuple(mask.shape) != (input.shape[0], KH * KW, Ho, Wo):
            raise ValueError(f'mask shape {tuple(mask.shape)} != {(input.shape[0], KH * KW, Ho, Wo)}')
        return _deform_conv2d_cpu(input, offset.to(input.dtype), weight.to(input.dtype),
                                  None if bias is None else bias.to(input.dtype), s, p, d,
                                  None if mask is None else mask.to(input.dtype))
    s, p, d = _pair(stride), _pair(padding), _pair(dilation)
    if input.dim() != 4 or weight.dim() != 4:
        raise ValueError('input and weight must be 4-D')
    N, C, H, W = input.shape
    Co, Ci, KH, KW = weight.shape
    if (KH, KW) != (3, 3) or d != (1, 1) or s[0] != s[1] or p[0] != p[1]:
        raise NotImplementedError('the HIP kernel covers 3x3, dilation 1, equal strides/paddings (DSC\'s case)')
    if Ci != C:
        raise ValueError(f'weight expects {Ci} input channels, input has {C} (one weight group only)')
    Ho = (H + 2 * p[0] - 3) // s[0] + 1
    Wo = (W + 2 * p[1] - 3) // s[1] + 1
    if tuple(offset.shape) != (N, 18, Ho, Wo):
        raise ValueError(f'offset shape {tuple(offset.shape)} != {(N, 18, Ho, Wo)} (one offset group)')
    if mask is not None and tuple(mask.shape) != (N, 9, Ho, Wo):
        raise ValueError(f'mask shape {tuple(mask.shape)} != {(N, 9, Ho, Wo)}')
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (input, offset, weight, bias, mask)):
        raise NotImplementedError('kadconv HIP kernels are inference-only (no backward)')
    dtype = input.dtype
    if N == 0 or Ho <= 0 or Wo <= 0:  # nothing to compute: the empty result, as torchvision returns it
        return input.new_empty(N, Co, max(Ho, 0), max(Wo, 0))
    x, _ = _nhwc_view(input)
    P = Ho * Wo
    off = offset.to(torch.float32).contiguous()
    m = mask.to(torch.float32).contiguous() if mask is not None else None
    wp = _ext.dcn_pack_weights(weight, dtype)
    b = None
    if bias is not None:  # fp32 contiguous biases are used as they are (no per-call copy)
        b = bias if (bias.dtype == torch.float32 and bias.is_contiguous()) else bias.detach().float().contiguous()
    out = torch.empty(N, Co, Ho, Wo, dtype=dtype, device=input.device)
    _ext.dcn_fwd(x, C, off, (18 * P, 1, P), m, (9 * P, 1, P), wp, Co, out, stride=s[0], pad=p[0], bias=b,
                 out_layout=_ext.KAD_NCHW)
    return out


def conv1x1(x, weight, bias=None, act=None, pool=1, wpack=None):
    """act(conv1x1(avg_pool2d(x, pool), weight) + bias) on the GPU; NCHW or
    channels-last input, output in the same memory format."""
    if not x.is_cuda:
        raise ValueError('kadconv.ops.conv1x1 needs a GPU tensor')
    N, C, H, W = x.shape
    Co = weight.shape[0]
    dtype = x.dtype
    if wpack is None:
        wpack = _ext.gemm_pack_weights(weight, dtype)
    b = bias.detach().to(torch.float32).contiguous() if bias is not None else None
    a = {None: 0, 'silu': 1}[act]
    Hp, Wp = H // pool, W // pool
    if N * Hp * Wp == 0:  # nothing to compute: the empty result
        mf = torch.channels_last if x.is_contiguous(memory_format=torch.channels_last) else torch.contiguous_format
        return torch.empty(N, Co, Hp, Wp, dtype=dtype, device=x.device, memory_format=mf)
    if x.is_contiguous(memory_format=torch.channels_last) and not x.is_contiguous():
        out = torch.empty(N, Co, Hp, Wp, dtype=dtype, device=x.device, memory_format=torch.channels_last)
        _ext.gemm1x1_fwd(x.permute(0, 2, 3, 1), _ext.KAD_NHWC, C, wpack, Co, out.permute(0, 2, 3, 1),
                         _ext.KAD_NHWC, bias=b, pool=pool, act=a)
        return out
    out = torch.empty(N, Co, Hp, Wp, dtype=dtype, device=x.device)
    _ext.gemm1x1_fwd(x.contiguous(), _ext.KAD_NCHW, C, wpack, Co, out, _ext.KAD_NCHW, bias=b, pool=pool, act=a)
    return out


def squeeze_excitation(x, w1, b1, w2, b2):
    """x * sigmoid(W2 relu(W1 mean_hw(x) + b1) + b2) on the GPU (NCHW or channels-last)."""
    if not x.is_cuda:
        raise ValueError('kadconv.ops.squeeze_excitation needs a GPU tensor')
    N, C, H, W = x.shape
    if N == 0:  # nothing to compute: the empty result
        return torch.empty_like(x)
    hid = w1.shape[0]
    def f32(t):  # fp32 contiguous tensors are used as they are (no per-call copy)
        return t if (t.dtype == torch.float32 and t.is_contiguous()) else t.detach().float().contiguous()

    nhwc = x.is_contiguous(memory_format=torch.channels_last) and not x.is_contiguous()
    layout = _ext.KAD_NHWC if nhwc else _ext.KAD_NCHW
    xv = x.permute(0, 2, 3, 1) if nhwc else x.contiguous()
    if not nhwc and _ext.se_nchw_fits(N, C, H, W, hid) and x.dtype in (torch.float16, torch.bfloat16, torch.float32):
        att = torch.empty(N, C, dtype=torch.float32, device=x.device)
        return _ext.se_nchw(xv, f32(w1), None if b1 is None else f32(b1), f32(w2), None if b2 is None else f32(b2),
                            att, torch.empty_like(xv))
    tiles = _ext.se_pool_tiles(H, W, layout)
    partial = torch.empty(N, tiles, C, dtype=torch.float32, device=x.device)
    _ext.se_pool(xv, C, layout, partial)
    att = torch.empty(N, C, dtype=torch.float32, device=x.device)
    hidden = torch.empty(N, hid, dtype=torch.float32, device=x.device)
    if not nhwc and C <= 1024 and hid <= 64:
        # hidden layer, then layer 2 inside the channel scale (one launch fewer)
        _ext.se_hidden(partial, tiles, 1.0 / (H * W), f32(w1), f32(b1), hidden, N, C, hid)
        out = torch.empty_like(xv)
        _ext.se_scale(xv, hidden, f32(w2), f32(b2), att, out, hid)
        return out
    _ext.se_mlp_ws(partial, tiles, 1.0 / (H * W), f32(w1), f32(b1), f32(w2), f32(b2), att, N, C, hid, hidden)
    if nhwc:
        out = torch.empty_like(x, memory_format=torch.channels_last)
        _ext.channel_scale(xv, att, out.permute(0, 2, 3, 1), C, layout)
    else:
        out = torch.empty_like(xv)
        _ext.channel_scale(xv, att, out, C, layout)
    return out
