"""CPU restatement of the reference's plain-PyTorch KAD-CNet forward.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline) -- never as the thing measured or shipped.

Functional, driven by a state dict with the reference's parameter names
(``model.{i}.…``, KAD-CNet/models/yolo.py:744-819 numbering) and by the model
dictionary (the rows of KAD-CNet/configs/dior_s_base.yaml).  Each block
follows its reference forward:

  Conv            act(bn(conv(x)))             KAD-CNet/models/common.py:43-57
  AConv           avg_pool2d(x, 2, 1) -> Conv s2                 common.py:60-67
  ELAN1           chunk, two chained 3x3 Convs, cat, Conv        common.py:580-598
  SPPELAN         Conv, three chained 5x5 max pools, cat, Conv   common.py:563-577
  RepNCSPELAN4_KADC / RepNCSP_KADC      KAD-CNet/models/module/KADC/module.py:74-111
  KADC4           oracle.kadconv_oracle.kadconv_forward          module.py:14-61
  nn.Upsample(nearest), Concat                                   common.py:535-542
  DDetect         two conv branches per level, DFL expectation,
                  anchors + dist2bbox, class sigmoid            yolo.py:102-127,
                                                                 common.py:232-244,
                                                                 utils/tal/anchor_generator.py:8-32
  NMS             greedy IoU suppression in descending score order, the
                  torchvision.ops.nms contract used by utils/general.py:881-990

BN epsilon: the reference sets every BatchNorm2d to eps 1e-3
(KAD-CNet/utils/torch_utils.py:208-217); the state dict does not carry eps,
so it is a parameter here.  A Conv whose state holds ``conv.bias`` and no
``bn.*`` is a fused one (yolo.py:574-585).
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import kadconv_oracle as K

BN_EPS = 1e-3


def _sub(sd, prefix):
    return {k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)}


def _conv(sd, p, x, s=1, act=True, eps=BN_EPS):
    w = sd[p + 'conv.weight']
    k = w.shape[-1]
    g = x.shape[1] // w.shape[1]
    y = F.conv2d(x, w, sd.get(p + 'conv.bias'), stride=s, padding=k // 2, groups=g)
    if p + 'bn.weight' in sd:
        y = F.batch_norm(y, sd[p + 'bn.running_mean'], sd[p + 'bn.running_var'], sd[p + 'bn.weight'],
                         sd[p + 'bn.bias'], False, 0.0, eps)
    return F.silu(y) if act else y


def _repncsp(sd, p, x):
    a = _conv(sd, p + 'cv1.', x)
    j = 0
    while f'{p}m.{j}.convs.0.0.weight' in sd:
        a = K.kadconv_forward(_sub(sd, f'{p}m.{j}.'), a)
        j += 1
    return _conv(sd, p + 'cv3.', torch.cat((a, _conv(sd, p + 'cv2.', x)), 1))


def _gelan(sd, p, x, kadc):
    y = list(_conv(sd, p + 'cv1.', x).chunk(2, 1))
    for stage in ('cv2.', 'cv3.'):
        if kadc:
            t = _repncsp(sd, p + stage + '0.', y[-1])
            y.append(_conv(sd, p + stage + '1.', t))
        else:
            y.append(_conv(sd, p + stage, y[-1]))
    return _conv(sd, p + 'cv4.', torch.cat(y, 1))


def _aconv(sd, p, x, eps=BN_EPS):
    """2 x 2 average pool, stride 1, no padding (count_include_pad), then the 3x3 stride-2 Conv cv1
    (common.py:60-67)."""
    return _conv(sd, p + 'cv1.', F.avg_pool2d(x, 2, 1, 0, False, True), s=2, eps=eps)


def _sppelan(sd, p, x):
    y = [_conv(sd, p + 'cv1.', x)]
    for _ in range(3):
        y.append(F.max_pool2d(y[-1], 5, 1, 2))
    return _conv(sd, p + 'cv5.', torch.cat(y, 1))


def ddetect_heads(sd, p, xs, nc):
    """The per-level head maps cat(box branch, class branch) [N, 64 + nc, h, w] (yolo.py:104-105)."""
    out = []
    for i, x in enumerate(xs):
        b = _conv(sd, f'{p}cv2.{i}.0.', x)
        b = _conv(sd, f'{p}cv2.{i}.1.', b)
        w = sd[f'{p}cv2.{i}.2.weight']
        b = F.conv2d(b, w, sd[f'{p}cv2.{i}.2.bias'], groups=b.shape[1] // w.shape[1])
        c = _conv(sd, f'{p}cv3.{i}.0.', x)
        c = _conv(sd, f'{p}cv3.{i}.1.', c)
        c = F.conv2d(c, sd[f'{p}cv3.{i}.2.weight'], sd[f'{p}cv3.{i}.2.bias'])
        out.append(torch.cat((b, c), 1))
    return out


def ddetect_decode(heads, strides, nc, reg_max=16):
    """y [N, 4 + nc, A]: per anchor (cell centre (x + 0.5, y + 0.5) of each level,
    levels in order, row-major), the box side distances are the expectation of
    the bin index under a softmax of its reg_max logits; xywh = ((l + r) / 2 ...)
    computed from x1y1 = anchor - (left, top), x2y2 = anchor + (right, bottom),
    times the level stride; then sigmoid of the class logits."""
    ys = []
    bins = torch.arange(reg_max, dtype=heads[0].dtype)
    for h, s in zip(heads, strides):
        N, _, H, W = h.shape
        box = h[:, :4 * reg_max].reshape(N, 4, reg_max, H * W)
        d = (torch.softmax(box, dim=2) * bins.view(1, 1, -1, 1)).sum(2)          # [N, 4, HW]
        gy, gx = torch.meshgrid(torch.arange(H, dtype=h.dtype) + 0.5, torch.arange(W, dtype=h.dtype) + 0.5,
                                indexing='ij')
        ax, ay = gx.reshape(1, -1), gy.reshape(1, -1)
        x1, y1, x2, y2 = ax - d[:, 0], ay - d[:, 1], ax + d[:, 2], ay + d[:, 3]
        xywh = torch.stack(((x1 + x2) / 2, (y1 + y2) / 2, x2 - x1, y2 - y1), 1) * s
        cls = torch.sigmoid(h[:, 4 * reg_max:4 * reg_max + nc].reshape(N, nc, H * W))
        ys.append(torch.cat((xywh, cls), 1))
    return torch.cat(ys, 2)


def kadcnet_forward(sd, cfg, x, eps=BN_EPS, layers=None):
    """(y, heads) of the eval-mode forward of the model described by ``cfg``
    (a model dictionary) with weights ``sd`` on input ``x`` [N, 3, H, W].  With a
    list ``layers``, every layer's output before the head is appended to it."""
    rows = cfg['backbone'] + cfg['head']
    outs = []
    cur = x
    for i, (f, n, m, args) in enumerate(rows):
        if f != -1:
            cur = outs[f] if isinstance(f, int) else [cur if j == -1 else outs[j] for j in f]
        p = f'model.{i}.'
        if m == 'Conv':
            cur = _conv(sd, p, cur, s=args[2] if len(args) > 2 else 1, eps=eps)
        elif m == 'AConv':
            cur = _aconv(sd, p, cur, eps=eps)
        elif m == 'ELAN1':
            cur = _gelan(sd, p, cur, kadc=False)
        elif m == 'RepNCSPELAN4_KADC':
            cur = _gelan(sd, p, cur, kadc=True)
        elif m == 'SPPELAN':
            cur = _sppelan(sd, p, cur)
        elif m == 'nn.Upsample':
            cur = F.interpolate(cur, scale_factor=args[1], mode='nearest')
        elif m == 'Concat':
            cur = torch.cat(cur, 1)
        elif m == 'DDetect':
            heads = ddetect_heads(sd, p, cur, cfg['nc'])
            strides = [x.shape[2] / h.shape[2] for h in heads]
            return ddetect_decode(heads, strides, cfg['nc']), heads
        else:
            raise NotImplementedError(m)
        outs.append(cur)
        if layers is not None:
            layers.append(cur)
    raise ValueError('the model dictionary has no DDetect layer')


# --------------------------------------------------------------------------- #
# NMS (torchvision.ops.nms contract, as used by utils/general.py:881-990)
# --------------------------------------------------------------------------- #
def nms(boxes, scores, iou_thres):
    """Greedy NMS: visit boxes by descending score (stable: ties in index order);
    keep a box unless its IoU with an already kept box exceeds iou_thres.  IoU =
    inter / (area_a + area_b - inter) in the boxes' own precision (float32 boxes:
    float32 arithmetic, as torchvision's kernel computes in the box dtype; else
    float64).  Returns kept indices in visiting order."""
    b = np.asarray(boxes)
    b = b.astype(np.float32 if b.dtype == np.float32 else np.float64)
    thr = b.dtype.type(iou_thres)
    order = np.argsort(-np.asarray(scores, dtype=np.float64), kind='stable')
    area = (b[:, 2] - b[:, 0]) * (b[:, 3] - b[:, 1])
    kept = []
    for i in order:
        if kept:
            k = np.asarray(kept)
            iw = np.maximum(np.minimum(b[k, 2], b[i, 2]) - np.maximum(b[k, 0], b[i, 0]), b.dtype.type(0))
            ih = np.maximum(np.minimum(b[k, 3], b[i, 3]) - np.maximum(b[k, 1], b[i, 1]), b.dtype.type(0))
            inter = iw * ih
            with np.errstate(divide='ignore', invalid='ignore'):
                iou = inter / (area[i] + area[k] - inter)
            if (iou > thr).any():
                continue
        kept.append(int(i))
    return kept


def non_max_suppression(prediction, conf_thres=0.25, iou_thres=0.45, max_det=300, agnostic=False):
    """general.py:881-990 (best class per box, no labels / masks): per image the
    rows (x1, y1, x2, y2, conf, cls) kept, in descending score order."""
    out = []
    max_wh = 7680
    pred = prediction if prediction.dtype in (torch.float32, torch.float64) else prediction.double()
    nc = pred.shape[1] - 4
    for x in pred:
        x = x.T
        x = x[x[:, 4:4 + nc].amax(1) > conf_thres]
        box = torch.stack((x[:, 0] - x[:, 2] / 2, x[:, 1] - x[:, 3] / 2, x[:, 0] + x[:, 2] / 2,
                           x[:, 1] + x[:, 3] / 2), 1)
        conf, j = x[:, 4:4 + nc].max(1, keepdim=True)
        x = torch.cat((box, conf, j.to(x.dtype)), 1)[conf.view(-1) > conf_thres]
        if not x.shape[0]:
            out.append(x)
            continue
        order = np.argsort(-x[:, 4].numpy(), kind='stable')[:30000]
        x = x[torch.from_numpy(order)]
        c = x[:, 5:6] * (0 if agnostic else max_wh)
        keep = nms((x[:, :4] + c).numpy(), x[:, 4].numpy(), iou_thres)[:max_det]
        out.append(x[torch.tensor(keep, dtype=torch.long)])
    return out


def make_divisible(x, divisor):
    """utils/general.py:660-664."""
    return math.ceil(x / divisor) * divisor


def channel_plan(cfg, ch=3):
    """Output channels of every layer of a model dictionary (yolo.py:744-819)."""
    gw = cfg['width_multiple']
    chans = []
    c_in = [ch]
    for i, (f, n, m, args) in enumerate(cfg['backbone'] + cfg['head']):
        src = c_in if i == 0 else chans
        if m in ('Conv', 'AConv', 'ELAN1', 'SPPELAN', 'RepNCSPELAN4_KADC'):
            c2 = make_divisible(args[0] * gw, 8)
        elif m == 'Concat':
            c2 = sum(chans[j] for j in f)
        elif m == 'DDetect':
            c2 = None
        else:
            c2 = src[f]
        chans.append(c2)
    return chans
