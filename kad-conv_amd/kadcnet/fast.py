"""Whole-network HIP forward of KAD-CNet-S (the config the reference benchmarks
with KAD-CNet/inference/benchmark_s.py and runs through
kadc_fused_nsmall.patch, KAD-CNet/inference/acceleration/kadc_fused_nsmall.py:524-629).

``KADCNetPlan`` walks a DetectionModel's layer list (the reference's module
tree, found by class name, so a model built by the reference's own
KAD-CNet/models/yolo.py works too) and runs every layer on the gfx950 kernels:

  Conv k=1 (+SiLU)          kad_gemm1x1_fwd, NHWC in / out
  Conv k=3 (+SiLU), s 1/2   kad_conv_fwd (implicit-GEMM 3x3 conv); the first layer on a
                            1-3 channel image: kad_stem_conv_fwd, reading the NCHW input
  AConv                     kad_nhwc_resample (2x2 / s1 average) + kad_conv_fwd s2
  ELAN1, SPPELAN, GELAN     the convs write their channel slice of one concat
                            buffer; chunks are slices of it (no copies)
  KADC4 / KADC4_m           kadconv.fused.KADConvPlan (pyramid, LCSA, fused DSC +
                            SE, merges) on channels-last maps
  nn.Upsample, Concat       kad_nhwc_resample (nearest / copy into slices)
  DDetect                   per level: the two first 3x3 convs as one conv with
                            stacked outputs, the grouped convs as block-diagonal
                            dense weights, the 1x1 outputs written into one
                            [box | cls] map per level; kad_ddetect_decode for
                            DFL + dist2bbox + sigmoid of all levels

Activations stay NHWC in the model's dtype between layers.  Conv + BatchNorm
pairs are folded into one biased conv (KAD-CNet/utils/torch_utils.py:244-265)
whether or not the model was ``fuse()``d.  ``forward`` returns (y, x) as
DDetect does in eval mode: y [N, 4 + nc, anchors] and the per-level head maps
[N, 4 reg_max + nc, h, w] (channels-last views).  Weights are captured when the
plan is built: rebuild it after loading new weights.
"""
import types

import torch
import torch.nn as nn

from kadconv import _ext
from kadconv.fused import KADConvPlan

_KADC_TYPES = {'KADConv', 'KADC4', 'KADC4_m'}


def _act_of(m):
    act = getattr(m, 'act', None)
    if isinstance(act, nn.SiLU):
        return _ext.KAD_ACT_SILU
    if act is None or isinstance(act, nn.Identity):
        return _ext.KAD_ACT_NONE
    if isinstance(act, nn.ReLU):
        return _ext.KAD_ACT_RELU
    raise NotImplementedError(f'activation {type(act).__name__} has no HIP epilogue')


class _ConvOp:
    """One k=1 or k=3 convolution (+ folded BN, + activation) on NHWC maps."""

    def __init__(self, conv, bn=None, act=_ext.KAD_ACT_NONE):
        w = conv.weight.detach().float()
        co, cig, kh, kw = w.shape
        g = conv.groups
        b = conv.bias.detach().float() if conv.bias is not None else torch.zeros(co, device=w.device)
        if bn is not None:
            scale = bn.weight.detach().float() / torch.sqrt(bn.running_var.float() + bn.eps)
            w = w * scale.view(-1, 1, 1, 1)
            b = (b - bn.running_mean.float()) * scale + bn.bias.detach().float()
        if g > 1:  # grouped: block-diagonal dense weights
            dense = torch.zeros(co, cig * g, kh, kw, device=w.device)
            cog = co // g
            for i in range(g):
                dense[i * cog:(i + 1) * cog, i * cig:(i + 1) * cig] = w[i * cog:(i + 1) * cog]
            w = dense
        if kh != kw or kh not in (1, 3) or tuple(conv.dilation) != (1, 1):
            raise NotImplementedError(f'conv {kh}x{kw} dilation {conv.dilation}: the HIP path covers 1x1 and 3x3')
        self.k, self.stride, self.pad = kh, conv.stride[0], conv.padding[0]
        if self.k == 1 and (self.stride != 1 or self.pad != 0):
            raise NotImplementedError('1x1 convs run with stride 1, no padding')
        if self.k == 3 and (self.pad != 1 or self.stride not in (1, 2)):
            raise NotImplementedError('3x3 convs run with padding 1, stride 1 or 2')
        self.cin, self.cout = w.shape[1], co
        self.w = w.contiguous()
        self.b = b.contiguous()
        self.act = act
        self._packed = {}

    @classmethod
    def from_conv_module(cls, m):
        """KAD-CNet's Conv (conv, optional bn, act)."""
        return cls(m.conv, getattr(m, 'bn', None), _act_of(m))

    @classmethod
    def stacked(cls, ops):
        """One conv producing the concatenated outputs of several convs of the same input."""
        first = ops[0]
        op = object.__new__(cls)
        op.k, op.stride, op.pad, op.cin = first.k, first.stride, first.pad, first.cin
        if any((o.k, o.stride, o.pad, o.cin, o.act) != (op.k, op.stride, op.pad, op.cin, first.act) for o in ops):
            raise ValueError('stacked convs must share input, shape and activation')
        op.w = torch.cat([o.w for o in ops]).contiguous()
        op.b = torch.cat([o.b for o in ops]).contiguous()
        op.cout, op.act, op._packed = op.w.shape[0], first.act, {}
        return op

    @classmethod
    def block_diagonal(cls, ops):
        """One 1x1 conv over the concatenated inputs of several 1x1 convs, producing their
        concatenated outputs (each reads only its own input channels)."""
        first = ops[0]
        if any(o.k != 1 or o.act != first.act for o in ops):
            raise ValueError('block-diagonal convs must be 1x1 with one activation')
        op = object.__new__(cls)
        op.k, op.stride, op.pad = 1, 1, 0
        op.cin, op.cout = sum(o.cin for o in ops), sum(o.cout for o in ops)
        op.w = torch.zeros(op.cout, op.cin, 1, 1, device=first.w.device)
        r = c = 0
        for o in ops:
            op.w[r:r + o.cout, c:c + o.cin] = o.w
            r, c = r + o.cout, c + o.cin
        op.b = torch.cat([o.b for o in ops]).contiguous()
        op.act, op._packed = first.act, {}
        return op

    def out_hw(self, h, w):
        if self.k == 1:
            return h, w
        return (h + 2 - 3) // self.stride + 1, (w + 2 - 3) // self.stride + 1

    def packed(self, dtype):
        if dtype not in self._packed:
            if self.k == 1:
                self._packed[dtype] = _ext.gemm_pack_weights(self.w.reshape(self.cout, self.cin), dtype)
            else:
                self._packed[dtype] = _ext.dcn_pack_weights(self.w, dtype)
        return self._packed[dtype]

    def __call__(self, x, out=None):
        N, H, W = x.shape[:3]
        if out is None:
            ho, wo = self.out_hw(H, W)
            out = x.new_empty(N, ho, wo, self.cout)
        wp = self.packed(x.dtype)
        if self.k == 1:
            _ext.gemm1x1_nhwc(x, self.cin, wp, self.cout, out, bias=self.b, act=self.act)
        else:
            _ext.conv_fwd(x, self.cin, wp, self.cout, out, stride=self.stride, pad=1, bias=self.b, act=self.act)
        return out


def _stem_ok(op, x):
    """The first layer can read the NCHW image directly (kad_stem_conv_fwd)."""
    return (isinstance(op, _ConvOp) and op.k == 3 and op.pad == 1 and op.stride in (1, 2) and op.cin <= 3
            and op.cout <= 64 and x.dtype in (torch.float16, torch.bfloat16) and x.shape[3] % 8 == 0)


def _stem(op, x):
    N, _, H, W = x.shape
    ho, wo = op.out_hw(H, W)
    out = x.new_empty(N, ho, wo, op.cout)
    _ext.stem_conv_fwd(x, op.packed(x.dtype), op.cout, out, stride=op.stride, bias=op.b, act=op.act)
    return out


def _copy(src, dst):
    """dst[..., :c] = src (NHWC views, c = src channels)."""
    _ext.nhwc_resample(src, dst, src.shape[3], _ext.KAD_RS_AVG, k=1, s=1, p=0)
    return dst


class _KADConvOp:
    def __init__(self, layer):
        self.plan = KADConvPlan(layer)
        self.dim = self.plan.dim

    def __call__(self, x, out=None):
        """x: NHWC [N, H, W, dim], dense or a channel slice of a wider buffer -> NHWC [N, H, W, dim]
        (dense, or out: an NHWC channel slice of a wider buffer)."""
        y = self.plan.forward(x.permute(0, 3, 1, 2), None if out is None else out.permute(0, 3, 1, 2))
        return y.permute(0, 2, 3, 1)


class _RepNCSP:
    """cv3(cat(m(cv1(x)), cv2(x))) (KAD-CNet/models/module/KADC/module.py:74-89)."""

    def __init__(self, m):
        self.cv1 = _ConvOp.from_conv_module(m.cv1)
        self.cv2 = _ConvOp.from_conv_module(m.cv2)
        self.cv3 = _ConvOp.from_conv_module(m.cv3)
        self.m = [_KADConvOp(b) for b in m.m]
        self.c_ = self.cv1.cout
        # cv1 and cv2 read the same input: one GEMM with stacked weights writes [cv1(x) | cv2(x)]
        # into the concat buffer; the first block reads cv1(x) from there, the last overwrites it
        # (two or more blocks: the last block's input is then another tensor)
        self.cv12 = None
        if len(self.m) >= 2:
            try:
                self.cv12 = _ConvOp.stacked([self.cv1, self.cv2])
            except ValueError:
                self.cv12 = None

    def __call__(self, x, out=None):
        N, H, W = x.shape[:3]
        cat = x.new_empty(N, H, W, 2 * self.c_)
        if self.cv12 is not None:
            self.cv12(x, cat)
            y = cat[..., :self.c_]
        else:
            self.cv2(x, cat[..., self.c_:])
            y = self.cv1(x)
        if not self.m:
            _copy(y, cat)
        for i, blk in enumerate(self.m):  # the last block writes the concat's first half itself
            y = blk(y, cat[..., :self.c_] if i == len(self.m) - 1 else None)
        return self.cv3(cat, out)


class _GELAN:
    """RepNCSPELAN4_KADC (module.py:92-111) and ELAN1 (common.py:580-598): cv1
    into the first c3 channels of the concat buffer, each later stage into its
    slice, cv4 over the buffer."""

    def __init__(self, m):
        self.cv1 = _ConvOp.from_conv_module(m.cv1)
        self.c3 = self.cv1.cout
        if isinstance(m.cv2, nn.Sequential):  # RepNCSPELAN4_KADC: (RepNCSP_KADC, 3x3 Conv)
            self.stages = [(_RepNCSP(s[0]), _ConvOp.from_conv_module(s[1])) for s in (m.cv2, m.cv3)]
        else:  # ELAN1: plain 3x3 Convs
            self.stages = [(None, _ConvOp.from_conv_module(s)) for s in (m.cv2, m.cv3)]
        self.c4 = self.stages[0][1].cout
        self.cv4 = _ConvOp.from_conv_module(m.cv4)

    def __call__(self, x, out=None):
        N, H, W = x.shape[:3]
        ctot = self.c3 + 2 * self.c4
        cat = x.new_empty(N, H, W, ctot)
        self.cv1(x, cat[..., :self.c3])
        src = cat[..., (self.c3 + 1) // 2:self.c3]  # the second half as the module splits it (first = ceil(c3 / 2))
        off = self.c3
        for csp, conv in self.stages:
            t = csp(src) if csp is not None else src
            dst = cat[..., off:off + self.c4]
            conv(t, dst)
            src = dst
            off += self.c4
        return self.cv4(cat, out)


class _AConv:
    def __init__(self, m):
        self.cv1 = _ConvOp.from_conv_module(m.cv1)

    def __call__(self, x, out=None):
        N, H, W, C = x.shape
        p = x.new_empty(N, H - 1, W - 1, C)
        _ext.nhwc_resample(x, p, C, _ext.KAD_RS_AVG, k=2, s=1, p=0)
        return self.cv1(p, out)


class _SPPELAN:
    def __init__(self, m):
        self.cv1 = _ConvOp.from_conv_module(m.cv1)
        self.k = []
        for sp in (m.cv2, m.cv3, m.cv4):
            k, st, pd = (v if isinstance(v, int) else v[0] for v in (sp.m.kernel_size, sp.m.stride, sp.m.padding))
            if st != 1 or pd != k // 2 or k % 2 != 1:
                raise NotImplementedError('SPPELAN: the HIP path covers odd max pools with stride 1 and padding k // 2')
            self.k.append(k)
        self.cv5 = _ConvOp.from_conv_module(m.cv5)

    def __call__(self, x, out=None):
        N, H, W = x.shape[:3]
        c = self.cv1.cout
        cat = x.new_empty(N, H, W, 4 * c)
        self.cv1(x, cat[..., :c])
        ks = self.k
        if ks[0] == ks[1] == ks[2]:  # the three chained pools in one launch
            _ext.nhwc_resample(cat[..., :c], cat[..., c:], c, _ext.KAD_RS_MAX3, k=ks[0], s=1, p=ks[0] // 2)
        else:
            for i, k in enumerate(ks):
                _ext.nhwc_resample(cat[..., i * c:(i + 1) * c], cat[..., (i + 1) * c:(i + 2) * c], c, _ext.KAD_RS_MAX,
                                   k=k, s=1, p=k // 2)
        return self.cv5(cat, out)


class _Upsample:
    def __init__(self, m):
        if m.mode != 'nearest' or m.size is not None:
            raise NotImplementedError('nn.Upsample: the HIP path covers nearest with an integer scale factor')
        sf = m.scale_factor
        sf = sf[0] if isinstance(sf, (tuple, list)) else sf
        if float(sf) != int(sf):
            raise NotImplementedError('nn.Upsample: integer scale factors only')
        self.s = int(sf)

    def __call__(self, x, out=None):
        N, H, W, C = x.shape
        if out is None:
            out = x.new_empty(N, H * self.s, W * self.s, C)
        _ext.nhwc_resample(x, out, C, _ext.KAD_RS_NEAREST, s=self.s)
        return out


class _Concat:
    def __call__(self, xs):
        N, H, W = xs[0].shape[:3]
        out = xs[0].new_empty(N, H, W, sum(t.shape[3] for t in xs))
        off = 0
        for t in xs:
            _copy(t, out[..., off:off + t.shape[3]])
            off += t.shape[3]
        return out


class _DDetect:
    def __init__(self, m):
        self.nc, self.reg_max, self.nl = m.nc, m.reg_max, m.nl
        self.box_ch = 4 * m.reg_max
        self.stride = [float(s) for s in m.stride]
        self.levels = []
        for i in range(m.nl):
            b0, b1, b2 = m.cv2[i]
            c0, c1, c2 = m.cv3[i]
            first = _ConvOp.stacked([_ConvOp.from_conv_module(b0), _ConvOp.from_conv_module(c0)])
            ob1, oc1 = _ConvOp.from_conv_module(b1), _ConvOp.from_conv_module(c1)
            self.levels.append((first, ob1, oc1, _ConvOp.block_diagonal([_ConvOp(b2), _ConvOp(c2)])))
        self.head_cs = (self.box_ch + self.nc + 7) // 8 * 8

    def __call__(self, xs):
        heads = []
        for x, (first, b1, c1, bc2) in zip(xs, self.levels):
            N, H, W = x.shape[:3]
            t = first(x)
            nb = b1.cin
            # the two branches' middle convs write one buffer, whose box and class 1x1 convs run
            # as one block-diagonal GEMM straight into the [box | cls] map
            mid = x.new_empty(N, H, W, b1.cout + c1.cout)
            b1(t[..., :nb], mid[..., :b1.cout])
            c1(t[..., nb:], mid[..., b1.cout:])
            head = x.new_empty(N, H, W, self.head_cs)
            bc2(mid, head[..., :self.box_ch + self.nc])
            heads.append(head)
        A = sum(h.shape[1] * h.shape[2] for h in heads)
        y = heads[0].new_empty(heads[0].shape[0], 4 + self.nc, A)
        _ext.ddetect_decode(heads, self.stride, y, self.nc, reg_max=self.reg_max, box_ch=self.box_ch)
        return y, [h[..., :self.box_ch + self.nc].permute(0, 3, 1, 2) for h in heads]


def _layer_op(m):
    t = type(m).__name__
    if t == 'Conv':
        return _ConvOp.from_conv_module(m)
    if t == 'AConv':
        return _AConv(m)
    if t in ('ELAN1', 'RepNCSPELAN4_KADC'):
        return _GELAN(m)
    if t == 'SPPELAN':
        return _SPPELAN(m)
    if t == 'Upsample':
        return _Upsample(m)
    if t == 'Concat':
        if m.d != 1:
            raise NotImplementedError('Concat along channels only')
        return _Concat()
    if t == 'DDetect':
        return _DDetect(m)
    if t in _KADC_TYPES:
        return _KADConvOp(m)
    raise NotImplementedError(f'no HIP path for layer type {t}')


class KADCNetPlan:
    """HIP forward of a KAD-CNet DetectionModel (layers in ``model.model`` with
    the 'from' indices ``.f`` that parse_model attaches, yolo.py:744-819)."""

    def __init__(self, model):
        self.layers = [(getattr(m, 'f', -1), _layer_op(m)) for m in model.model]
        self.in_ch = None
        first = self.layers[0][1]
        self.in_ch = first.cin if isinstance(first, _ConvOp) else None
        self._elide = {}

    def eligible(self, x):
        return (x.is_cuda and x.dim() == 4 and x.dtype in (torch.float32, torch.float16, torch.bfloat16)
                and x.shape[0] > 0 and (self.in_ch is None or x.shape[1] == self.in_ch)
                and x.shape[2] % 32 == 0 and x.shape[3] % 32 == 0 and min(x.shape[2:]) >= 128)

    def forward(self, x, keep_layers=False):
        """(y, heads); with keep_layers, also every layer's output (NHWC maps; the
        last entry is (y, heads))."""
        N, C, H, W = x.shape
        ys = []
        layers = self.layers
        f0, op0 = layers[0]
        if f0 == -1 and _stem_ok(op0, x):  # the stem reads the NCHW image itself
            cur = _stem(op0, x.contiguous())
            ys.append(cur)
            layers = layers[1:]
        else:
            cs = (C + 7) // 8 * 8
            xin = torch.empty(N, H, W, cs, dtype=x.dtype, device=x.device)
            _ext.to_nhwc(x.contiguous(), xin)
            cur = xin[..., :C]
        key = (tuple(x.shape), x.dtype, x.device)
        el = self._elide.get(key)
        bufs = {}
        for f, op in layers:
            i = len(ys)  # this layer's index in the model
            if f != -1:
                cur = ys[f] if isinstance(f, int) else [cur if j == -1 else ys[j] for j in f]
            if el is not None and i in el[0]:   # writes its slice of a later Concat's buffer
                k, off, c = el[0][i]
                if k not in bufs:
                    bufs[k] = x.new_empty(el[1][k])
                cur = op(cur, out=bufs[k][..., off:off + c])
            elif el is not None and i in el[1]:  # a Concat whose inputs are already in place
                cur = bufs.pop(i)
            else:
                cur = op(cur)
            ys.append(cur)
        if el is None:
            self._elide[key] = self._concat_slots(ys)
        return (cur, ys) if keep_layers else cur

    def _concat_slots(self, ys):
        """From one forward's layer outputs: ({layer i: (Concat layer k, channel offset, channels)},
        {k: buffer shape}) for every Concat whose inputs can all be written straight into its buffer
        (each input layer feeding no other Concat), so that later forwards of the same input shape
        skip the copies.  Other consumers of such an input read its channel slice of the buffer, so
        every slot must start at a multiple of 8 channels (16-byte pieces); a Concat with another
        offset keeps its copies."""
        slots, shapes = {}, {}
        for k, (f, op) in enumerate(self.layers):
            if not isinstance(op, _Concat) or not isinstance(f, (list, tuple)):
                continue
            ins = [k - 1 if j == -1 else j for j in f]
            if (len(set(ins)) != len(ins) or any(j in slots or j == 0 for j in ins)
                    or not all(isinstance(self.layers[j][1], (_ConvOp, _GELAN, _AConv, _SPPELAN, _Upsample))
                               for j in ins)):
                continue
            offs = [0]
            for j in ins:
                offs.append(offs[-1] + ys[j].shape[3])
            if any(o % 8 for o in offs[:-1]):  # consumers of a slice need a 16-byte aligned channel base
                continue
            for j, o in zip(ins, offs):
                slots[j] = (k, o, ys[j].shape[3])
            shapes[k] = tuple(ys[k].shape)
        return slots, shapes


def enable_fast_inference(model, allow_untested_gpu=False):
    """Switch a KAD-CNet DetectionModel to the whole-network HIP forward, in place.
    The model must be in eval mode on a ROCm GPU; inputs the plan does not cover
    (training mode, CPU tensors, sizes not a multiple of 32 or below 128) take
    the plain forward.  Returns the model."""
    if model.training:
        raise ValueError('call model.eval() before enable_fast_inference()')
    params = list(model.parameters())
    if not params or params[0].device.type != 'cuda':
        raise ValueError('move the model to a ROCm GPU first')
    from kadconv.fast import _is_gfx950
    if not _is_gfx950(params[0].device) and not allow_untested_gpu:
        raise ValueError('the HIP kernels are built for gfx950 (MI355X); pass allow_untested_gpu=True')
    _ext.load()
    with torch.no_grad():
        plan = KADCNetPlan(model)
    plain = types.MethodType(type(model).forward, model)

    def forward(x, *args, **kw):
        if model.training or args or kw or not plan.eligible(x):
            return plain(x, *args, **kw)
        with torch.no_grad():
            return plan.forward(x)

    model._kad_plan = plan
    model.forward = forward
    return model


def disable_fast_inference(model):
    if 'forward' in vars(model):
        del model.forward
    if hasattr(model, '_kad_plan'):
        del model._kad_plan
    return model
