"""KAD-CNet detection model: the DDetect head, the layer builder and DetectionModel.

Kept from the reference (KAD-CNet/models/yolo.py, utils/tal/anchor_generator.py:8-32) because state
dicts, the channel plan and the decoded boxes depend on them: class and attribute names, the
order submodules are created in, DDetect's branch widths, the ``model.{i}`` layer numbering with
its ``from`` indices, and the box formulas.  The code is this package's:

  anchors      cell centres (x + 0.5, y + 0.5) of every level, row-major, levels in order
  dist2bbox    (l, t, r, b) distances around an anchor -> (cx, cy, w, h) or (x1, y1, x2, y2)
  DDetect      per level cat(box branch, class branch); inference: DFL distances -> boxes times
               the level stride, class sigmoid
  parse_model  widths of the width-scaled blocks rounded up to multiples of 8, repeats scaled by
               depth, Concat widths summed, DDetect given its inputs' widths

``DIOR_S_BASE`` / ``DIOR_S_MGL`` restate the rows of KAD-CNet/configs/dior_s_{base,mgl}.yaml.
"""
import copy
import math

import torch
import torch.nn as nn

from .common import AConv, Concat, Conv, DFL, ELAN1, SPPELAN, fuse_conv_and_bn, make_divisible
from .kadc import RepNCSPELAN4_KADC


def make_anchors(feats, strides, grid_cell_offset=0.5):
    """(points [A, 2] as (x, y), stride per point [A, 1]) over the levels' maps, each level's cells
    in row-major order."""
    points, per_point = [], []
    for f, s in zip(feats, strides):
        h, w = f.shape[-2:]
        xs = torch.arange(w, dtype=f.dtype, device=f.device) + grid_cell_offset
        ys = torch.arange(h, dtype=f.dtype, device=f.device) + grid_cell_offset
        points.append(torch.stack((xs.repeat(h), ys.repeat_interleave(w)), dim=1))
        per_point.append(torch.full((h * w, 1), float(s), dtype=f.dtype, device=f.device))
    return torch.cat(points), torch.cat(per_point)


def dist2bbox(distance, anchor_points, xywh=True, dim=-1):
    """Side distances (left, top, right, bottom) along ``dim`` around anchor points -> boxes."""
    near, far = distance.chunk(2, dim)
    lo, hi = anchor_points - near, anchor_points + far
    if xywh:
        return torch.cat(((lo + hi) / 2, hi - lo), dim)
    return torch.cat((lo, hi), dim)


class DDetect(nn.Module):
    """Anchor-free head.  Level i: box branch cv2[i] = (3 x 3 Conv, 3 x 3 Conv in 4 groups, 1 x 1 conv
    in 4 groups -> 4 reg_max bin logits), class branch cv3[i] = (3 x 3 Conv, 3 x 3 Conv, 1 x 1 conv
    -> nc logits).  Training returns the per-level maps; inference returns (y [N, 4 + nc, A], maps)
    with y = (cx, cy, w, h) in input pixels and the class probabilities."""
    dynamic = False   # recompute the anchors on every call
    export = False    # inference returns y alone

    def __init__(self, nc=80, ch=(), inplace=True):
        super().__init__()
        self.nc = nc
        self.nl = len(ch)
        self.reg_max = 16
        self.no = nc + 4 * self.reg_max
        self.inplace = inplace
        self.stride = torch.zeros(self.nl)
        box_w = make_divisible(max(ch[0] // 4, 4 * self.reg_max, 16), 4)
        cls_w = max(ch[0], min(2 * nc, 128))
        self.cv2 = nn.ModuleList([nn.Sequential(Conv(c, box_w, 3), Conv(box_w, box_w, 3, g=4),
                                                nn.Conv2d(box_w, 4 * self.reg_max, 1, groups=4)) for c in ch])
        self.cv3 = nn.ModuleList([nn.Sequential(Conv(c, cls_w, 3), Conv(cls_w, cls_w, 3), nn.Conv2d(cls_w, nc, 1))
                                  for c in ch])
        self.dfl = DFL(self.reg_max) if self.reg_max > 1 else nn.Identity()
        self.shape, self.anchors, self.strides = None, torch.empty(0), torch.empty(0)

    def forward(self, x):
        maps = [torch.cat((box(f), cls(f)), 1) for f, box, cls in zip(x, self.cv2, self.cv3)]
        if self.training:
            return maps
        if self.dynamic or self.shape != maps[0].shape:
            pts, st = make_anchors(maps, self.stride, 0.5)
            self.anchors, self.strides, self.shape = pts.t(), st.t(), maps[0].shape
        flat = torch.cat([m.flatten(2) for m in maps], 2)                      # [N, no, A]
        nb = 4 * self.reg_max
        boxes = dist2bbox(self.dfl(flat[:, :nb]), self.anchors.unsqueeze(0), xywh=True, dim=1) * self.strides
        y = torch.cat((boxes, flat[:, nb:].sigmoid()), 1)
        return y if self.export else (y, maps)

    def bias_init(self):
        """Initial biases: box logits 1; class logits log(5 / nc) - 2 log(640 / stride), a prior of
        about 5 objects per 640 x 640 image spread over the level's cells and the classes."""
        for box, cls, s in zip(self.cv2, self.cv3, self.stride):
            box[-1].bias.data.fill_(1.0)
            cls[-1].bias.data[:self.nc] = math.log(5 / self.nc) - 2 * math.log(640 / float(s))


MODULES = {'Conv': Conv, 'AConv': AConv, 'ELAN1': ELAN1, 'SPPELAN': SPPELAN, 'RepNCSPELAN4_KADC': RepNCSPELAN4_KADC,
           'Concat': Concat, 'nn.Upsample': nn.Upsample, 'DDetect': DDetect}
_WIDTH_SCALED = (Conv, AConv, ELAN1, SPPELAN, RepNCSPELAN4_KADC)


def _arg(a, nc):
    return nc if a == 'nc' else (None if a == 'None' else a)


def parse_model(d, ch):
    """(nn.Sequential of the layers, each tagged with .i / .f / .type, sorted list of the layer
    indices whose outputs later layers read) from a model dictionary; ``ch`` = [input channels]."""
    nc, depth, width = d['nc'], d['depth_multiple'], d['width_multiple']
    widths = []                                     # output width of each layer built so far
    layers, save = [], set()
    for i, (f, n, name, args) in enumerate(d['backbone'] + d['head']):
        cls = MODULES[name]
        args = [_arg(a, nc) for a in args]
        width_of = (lambda j: widths[j]) if widths else (lambda j: ch[j])
        reps = max(round(n * depth), 1) if n > 1 else n
        if cls in _WIDTH_SCALED:
            c_out = make_divisible(args[0] * width, 8)
            args = [width_of(f), c_out] + args[1:]
        elif cls is Concat:
            c_out = sum(width_of(j) for j in f)
        elif cls is DDetect:
            args = args + [[width_of(j) for j in f]]
            c_out = None
        else:
            c_out = width_of(f)
        block = cls(*args) if reps == 1 else nn.Sequential(*[cls(*args) for _ in range(reps)])
        block.i, block.f, block.type = i, f, name
        save.update(j % i for j in ([f] if isinstance(f, int) else f) if j != -1)
        layers.append(block)
        widths.append(c_out)
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
    """The MGL configuration: every KAD-Conv block built with KADC4_m (hidden >= 64)."""
    d = copy.deepcopy(cfg)
    for row in d['backbone'] + d['head']:
        if row[2] == _KADC_ELAN:
            row[3] = list(row[3]) + ['KADC4_m']
    d['mgl_encoder_channels'] = [40, 72, 144, 216, 288]
    return d


DIOR_S_MGL = _mgl(DIOR_S_BASE)


class DetectionModel(nn.Module):
    """The detector: ``model`` (layers from parse_model), ``save``, ``stride`` (from a 256 x 256
    probe forward at construction), the DDetect bias prior, and BatchNorm eps 1e-3 / momentum 0.03
    (KAD-CNet/utils/torch_utils.py:208-217).  The MGL decoders (training only) are not built."""

    def __init__(self, cfg=DIOR_S_BASE, ch=3, nc=None):
        super().__init__()
        self.yaml = copy.deepcopy(cfg)
        in_ch = self.yaml.setdefault('ch', ch)
        if nc and nc != self.yaml['nc']:
            self.yaml['nc'] = nc
        self.model, self.save = parse_model(copy.deepcopy(self.yaml), ch=[in_ch])
        self.names = [str(k) for k in range(self.yaml['nc'])]
        self.inplace = self.yaml.get('inplace', True)
        head = self.model[-1]
        head.inplace = self.inplace
        probe = 256
        maps = self.forward(torch.zeros(1, in_ch, probe, probe))   # training mode: the head returns its maps
        head.stride = torch.tensor([probe / m.shape[-2] for m in maps])
        self.stride = head.stride
        head.bias_init()
        for mod in self.modules():
            if type(mod) is nn.BatchNorm2d:
                mod.eps, mod.momentum = 1e-3, 0.03
            elif type(mod) in (nn.ReLU, nn.SiLU):
                mod.inplace = True

    def forward(self, x):
        outputs = {}
        for layer in self.model:
            f = layer.f
            if f != -1:
                x = outputs[f] if isinstance(f, int) else [x if j == -1 else outputs[j] for j in f]
            x = layer(x)
            outputs[layer.i] = x
        return x

    def fuse(self):
        """Fold every Conv's BatchNorm into a biased convolution (eval-mode statistics)."""
        for mod in self.model.modules():
            if isinstance(mod, Conv) and hasattr(mod, 'bn'):
                mod.conv = fuse_conv_and_bn(mod.conv, mod.bn)
                del mod.bn
        return self

    def _apply(self, fn):
        super()._apply(fn)
        head = self.model[-1]
        for name in ('stride', 'anchors', 'strides'):
            setattr(head, name, fn(getattr(head, name)))
        self.stride = head.stride
        return self


Model = DetectionModel
