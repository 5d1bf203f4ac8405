"""KAD-CNet detection model: DDetect head, model builder and DetectionModel,
following KAD-CNet/models/yolo.py (DDetect :78-136, BaseModel :533-599,
DetectionModel :602-659, parse_model :744-819) and
KAD-CNet/utils/tal/anchor_generator.py:8-32 (make_anchors, dist2bbox).

The builder reads the same model dictionary as the reference's YAML files
(``nc``, ``depth_multiple``, ``width_multiple``, ``backbone`` and ``head`` rows of
[from, number, module, args]); ``DIOR_S_BASE`` / ``DIOR_S_MGL`` are the two
KAD-CNet-S configurations (KAD-CNet/configs/dior_s_{base,mgl}.yaml).  Modules are
looked up by name in a registry (the reference evals the strings).
"""
import copy
import math

import torch
import torch.nn as nn

from .common import AConv, Concat, Conv, DFL, ELAN1, SPPELAN, fuse_conv_and_bn, make_divisible
from .kadc import RepNCSPELAN4_KADC


def make_anchors(feats, strides, grid_cell_offset=0.5):
    """Cell centres (x + 0.5, y + 0.5) of every level, row-major, and their
    strides (anchor_generator.py:8-21)."""
    points, stride_t = [], []
    dtype, device = feats[0].dtype, feats[0].device
    for i, stride in enumerate(strides):
        _, _, h, w = feats[i].shape
        sx = torch.arange(w, device=device, dtype=dtype) + grid_cell_offset
        sy = torch.arange(h, device=device, dtype=dtype) + grid_cell_offset
        sy, sx = torch.meshgrid(sy, sx, indexing='ij')
        points.append(torch.stack((sx, sy), -1).view(-1, 2))
        stride_t.append(torch.full((h * w, 1), float(stride), dtype=dtype, device=device))
    return torch.cat(points), torch.cat(stride_t)


def dist2bbox(distance, anchor_points, xywh=True, dim=-1):
    """(left, top, right, bottom) distances -> xywh or xyxy boxes (anchor_generator.py:24-32)."""
    lt, rb = torch.split(distance, 2, dim)
    x1y1 = anchor_points - lt
    x2y2 = anchor_points + rb
    if xywh:
        return torch.cat(((x1y1 + x2y2) / 2, x2y2 - x1y1), dim)
    return torch.cat((x1y1, x2y2), dim)


class DDetect(nn.Module):
    """Anchor-free detection head (yolo.py:78-136): per level a box branch
    (3x3 Conv, grouped 3x3 Conv, grouped 1x1 -> 4 x reg_max) and a class branch
    (3x3 Conv, 3x3 Conv, 1x1 -> nc); inference decodes DFL distances into xywh
    boxes times the level stride and applies the class sigmoid."""
    dynamic = False
    export = False
    shape = None
    anchors = torch.empty(0)
    strides = torch.empty(0)

    def __init__(self, nc=80, ch=(), inplace=True):
        super().__init__()
        self.nc = nc
        self.nl = len(ch)
        self.reg_max = 16
        self.no = nc + self.reg_max * 4
        self.inplace = inplace
        self.stride = torch.zeros(self.nl)
        c2 = make_divisible(max((ch[0] // 4, self.reg_max * 4, 16)), 4)
        c3 = max((ch[0], min((self.nc * 2, 128))))
        self.cv2 = nn.ModuleList(
            nn.Sequential(Conv(x, c2, 3), Conv(c2, c2, 3, g=4), nn.Conv2d(c2, 4 * self.reg_max, 1, groups=4))
            for x in ch)
        self.cv3 = nn.ModuleList(
            nn.Sequential(Conv(x, c3, 3), Conv(c3, c3, 3), nn.Conv2d(c3, self.nc, 1)) for x in ch)
        self.dfl = DFL(self.reg_max) if self.reg_max > 1 else nn.Identity()

    def forward(self, x):
        shape = x[0].shape
        for i in range(self.nl):
            x[i] = torch.cat((self.cv2[i](x[i]), self.cv3[i](x[i])), 1)
        if self.training:
            return x
        if self.dynamic or self.shape != shape:
            self.anchors, self.strides = (t.transpose(0, 1) for t in make_anchors(x, self.stride, 0.5))
            self.shape = shape
        box, cls = torch.cat([xi.view(shape[0], self.no, -1) for xi in x], 2).split((self.reg_max * 4, self.nc), 1)
        dbox = dist2bbox(self.dfl(box), self.anchors.unsqueeze(0), xywh=True, dim=1) * self.strides
        y = torch.cat((dbox, cls.sigmoid()), 1)
        return y if self.export else (y, x)

    def bias_init(self):
        """Box logits 1.0; class logits log(5 / nc / (640 / s)^2) (yolo.py:129-136)."""
        for a, b, s in zip(self.cv2, self.cv3, self.stride):
            a[-1].bias.data[:] = 1.0
            b[-1].bias.data[:self.nc] = math.log(5 / self.nc / (640 / s) ** 2)


MODULES = {'Conv': Conv, 'AConv': AConv, 'ELAN1': ELAN1, 'SPPELAN': SPPELAN, 'RepNCSPELAN4_KADC': RepNCSPELAN4_KADC,
           'Concat': Concat, 'nn.Upsample': nn.Upsample, 'DDetect': DDetect}
_WIDTH_SCALED = {Conv, AConv, ELAN1, SPPELAN, RepNCSPELAN4_KADC}


def parse_model(d, ch):
    """Build the layer list from a model dictionary (yolo.py:744-819):
    output widths of the listed block types are scaled by width_multiple and
    rounded up to a multiple of 8; repeats by depth_multiple; Concat sums its
    inputs' widths; DDetect receives its inputs' widths.  Returns
    (nn.Sequential of layers with .i / .f / .type attributes, save list)."""
    nc, gd, gw = d['nc'], d['depth_multiple'], d['width_multiple']
    layers, save, c2 = [], [], ch[-1]
    for i, (f, n, m, args) in enumerate(d['backbone'] + d['head']):
        name = m
        m = MODULES[m]
        args = [nc if a == 'nc' else None if a == 'None' else a for a in args]
        n = max(round(n * gd), 1) if n > 1 else n
        if m in _WIDTH_SCALED:
            c1, c2 = ch[f], make_divisible(args[0] * gw, 8)
            args = [c1, c2, *args[1:]]
        elif m is Concat:
            c2 = sum(ch[x] for x in f)
        elif m is DDetect:
            args.append([ch[x] for x in f])
        else:
            c2 = ch[f]
        m_ = nn.Sequential(*(m(*args) for _ in range(n))) if n > 1 else m(*args)
        m_.i, m_.f, m_.type = i, f, name
        save.extend(x % i for x in ([f] if isinstance(f, int) else f) if x != -1)
        layers.append(m_)
        if i == 0:
            ch = []
        ch.append(c2)
    return nn.Sequential(*layers), sorted(save)


def _rows(*rows):
    return [list(r) for r in rows]


_KADC_ELAN = 'RepNCSPELAN4_KADC'
DIOR_S_BASE = {
    'nc': 20, 'depth_multiple': 1.0, 'width_multiple': 1.1, 'anchors': 3,
    'backbone': _rows(
        [-1, 1, 'Conv', [32, 3, 2]],                 # 0  P1/2
        [-1, 1, 'Conv', [64, 3, 2]],                 # 1  P2/4
        [-1, 1, 'ELAN1', [64, 64, 32]],              # 2
        [-1, 1, 'AConv', [128]],                     # 3  P3/8
        [-1, 1, _KADC_ELAN, [128, 128, 64, 3]],      # 4
        [-1, 1, 'AConv', [192]],                     # 5  P4/16
        [-1, 1, _KADC_ELAN, [192, 192, 96, 3]],      # 6
        [-1, 1, 'AConv', [256]],                     # 7  P5/32
        [-1, 1, _KADC_ELAN, [256, 256, 128, 3]],     # 8
    ),
    'head': _rows(
        [-1, 1, 'SPPELAN', [256, 128]],              # 9
        [-1, 1, 'nn.Upsample', ['None', 2, 'nearest']],
        [[-1, 6], 1, 'Concat', [1]],                 # 11
        [-1, 1, _KADC_ELAN, [192, 192, 96, 3]],      # 12
        [-1, 1, 'nn.Upsample', ['None', 2, 'nearest']],
        [[-1, 4], 1, 'Concat', [1]],                 # 14
        [-1, 1, _KADC_ELAN, [128, 128, 64, 3]],      # 15 (P3/8 out)
        [-1, 1, 'AConv', [96]],
        [[-1, 12], 1, 'Concat', [1]],                # 17
        [-1, 1, _KADC_ELAN, [192, 192, 96, 3]],      # 18 (P4/16 out)
        [-1, 1, 'AConv', [128]],
        [[-1, 9], 1, 'Concat', [1]],                 # 20
        [-1, 1, _KADC_ELAN, [256, 256, 128, 3]],     # 21 (P5/32 out)
        [[15, 18, 21], 1, 'DDetect', ['nc']],        # 22
    ),
    'ch': 3,
}


def _mgl(cfg):
    """The MGL variant: KADC4_m (hidden >= 64) in every KAD-Conv block."""
    d = copy.deepcopy(cfg)
    for row in d['backbone'] + d['head']:
        if row[2] == _KADC_ELAN:
            row[3] = row[3] + ['KADC4_m']
    d['mgl_encoder_channels'] = [40, 72, 144, 216, 288]
    return d


DIOR_S_MGL = _mgl(DIOR_S_BASE)


class DetectionModel(nn.Module):
    """KAD-CNet detection model (yolo.py:533-659): layers from parse_model, the
    forward threads earlier outputs to multi-input layers by their 'from'
    indices, strides come from a 256 x 256 probe, BN eps 1e-3 / momentum 0.03
    (utils/torch_utils.py:208-217).  The MGL decoders (training only) are not
    built."""

    def __init__(self, cfg=DIOR_S_BASE, ch=3, nc=None):
        super().__init__()
        self.yaml = copy.deepcopy(cfg)
        ch = self.yaml['ch'] = self.yaml.get('ch', ch)
        if nc and nc != self.yaml['nc']:
            self.yaml['nc'] = nc
        self.model, self.save = parse_model(copy.deepcopy(self.yaml), ch=[ch])
        self.names = [str(i) for i in range(self.yaml['nc'])]
        self.inplace = self.yaml.get('inplace', True)
        m = self.model[-1]
        s = 256
        m.inplace = self.inplace
        m.stride = torch.tensor([s / x.shape[-2] for x in self.forward(torch.zeros(1, ch, s, s))])
        self.stride = m.stride
        m.bias_init()
        for mod in self.modules():
            if type(mod) is nn.BatchNorm2d:
                mod.eps, mod.momentum = 1e-3, 0.03
            elif type(mod) in (nn.ReLU, nn.SiLU):
                mod.inplace = True

    def forward(self, x):
        y = []
        for m in self.model:
            if m.f != -1:
                x = y[m.f] if isinstance(m.f, int) else [x if j == -1 else y[j] for j in m.f]
            x = m(x)
            y.append(x)
        return x

    def fuse(self):
        """Fold every Conv's BatchNorm into its convolution (yolo.py:574-585)."""
        for m in self.model.modules():
            if isinstance(m, Conv) and hasattr(m, 'bn'):
                m.conv = fuse_conv_and_bn(m.conv, m.bn)
                delattr(m, 'bn')
                m.forward = m.forward_fuse
        return self

    def _apply(self, fn):
        self = super()._apply(fn)
        m = self.model[-1]
        m.stride = fn(m.stride)
        m.anchors = fn(m.anchors)
        m.strides = fn(m.strides)
        return self


Model = DetectionModel
