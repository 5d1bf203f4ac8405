"""Functional operators backed by libkadconv_hip.so.

* ``deform_conv2d`` -- drop-in for ``torchvision.ops.deform_conv2d`` (the call
  at KAD-Conv/kadconv/kad_conv.py:66-67) for 3x3 kernels, one offset group,
  dilation 1.  GPU tensors run the gfx950 HIP kernel; CPU tensors are handed to
  torchvision when it is importable (the reference's own CPU path).
* ``conv1x1`` -- 1x1 conv + bias + optional SiLU, optional input avg-pool
  (north-star piece 3; KAD-CNet ``Conv`` after Conv-BN fusion).
* ``squeeze_excitation`` -- SE block: GAP, FC-ReLU-FC-sigmoid, channel scale.

GPU entry points never fall back to another implementation: if the HIP library
is missing they raise ``kadconv._ext.KadExtensionError``.
"""
import torch

from . import _ext


def _nhwc_view(x):
    """Return (tensor [N,H,W,cs], cs) usable by the DCN kernels, converting with
    the HIP transpose when x is not already channels-last with cs % 8 == 0."""
    N, C, H, W = x.shape
    if x.is_contiguous(memory_format=torch.channels_last) and C % 8 == 0 and C > 1:
        return x.permute(0, 2, 3, 1), C
    cs = (C + 7) // 8 * 8
    xc = x.contiguous()
    out = torch.empty(N, H, W, cs, dtype=x.dtype, device=x.device)
    _ext.to_nhwc(xc, out)
    return out, cs


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def deform_conv2d(input, offset, weight, bias=None, stride=1, padding=0, dilation=1, mask=None):
    """Modulated deformable convolution with torchvision's signature and semantics."""
    if not input.is_cuda:
        try:
            import torchvision  # noqa: F401  (the reference's CPU operator)
        except ImportError:
            raise RuntimeError('kadconv.ops.deform_conv2d runs on the GPU (gfx950 HIP kernel); for CPU tensors '
                               'it needs torchvision.ops.deform_conv2d, which is not installed') from None
        import torchvision.ops
        return torchvision.ops.deform_conv2d(input, offset, weight, bias, stride=stride, padding=padding,
                                             dilation=dilation, mask=mask)
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
    tiles = _ext.se_pool_tiles(H, W, layout)
    partial = torch.empty(N, tiles, C, dtype=torch.float32, device=x.device)
    _ext.se_pool(xv, C, layout, partial)
    att = torch.empty(N, C, dtype=torch.float32, device=x.device)
    _ext.se_mlp(partial, tiles, 1.0 / (H * W), f32(w1), f32(b1), f32(w2), f32(b2), att, N, C, hid)
    if nhwc:
        out = torch.empty_like(x, memory_format=torch.channels_last)
        _ext.channel_scale(xv, att, out.permute(0, 2, 3, 1), C, layout)
    else:
        out = torch.empty_like(xv)
        _ext.channel_scale(xv, att, out, C, layout)
    return out
