"""Detection post-processing on the GPU: candidate selection, class-aware greedy NMS (the HIP
kad_nms kernels stand in for torchvision.ops.nms, which this image does not ship).

``non_max_suppression`` keeps the reference's call signature and result format
(KAD-CNet/utils/general.py:881-990: per image a [k, 6] tensor of x1, y1, x2, y2, score, class in
descending score order).  What it does, per image:

  1. candidates: anchors whose best class probability exceeds conf_thres (every (anchor, class)
     pair above it with multi_label), optionally only the listed classes;
  2. boxes (cx, cy, w, h) -> corners;
  3. order by score, descending, stable (ties keep anchor order), at most 30000;
  4. class-aware NMS: a box is suppressed by a higher-scoring kept box of the same class whose IoU
     with it exceeds iou_thres (classes are kept apart by shifting every box by 7680 px per
     class index, wider than any input, unless agnostic);
  5. at most max_det survivors.

The reference's ``labels`` (autolabelling: prepend known boxes) and ``nm`` (mask coefficients) are
not supported: nothing on the KAD-CNet inference path uses them.
"""
import torch

from kadconv import _ext

_CLASS_SHIFT = 7680   # px per class index: boxes of different classes never overlap
_MAX_CANDIDATES = 30000


def xywh2xyxy(x):
    """(cx, cy, w, h, ...) -> (x1, y1, x2, y2, ...) along the last dimension (other columns kept)."""
    centre, size = x[..., :2], x[..., 2:4]
    return torch.cat((centre - size / 2, centre + size / 2, x[..., 4:]), dim=-1)


def nms(boxes, scores, iou_threshold):
    """Indices (descending score) of the boxes greedy NMS keeps: a box is dropped when its IoU with
    a kept box of higher score exceeds iou_threshold (the torchvision.ops.nms contract).  GPU only."""
    if not boxes.is_cuda:
        raise ValueError('kadcnet.postprocess.nms runs on the GPU (HIP kad_nms)')
    if boxes.shape[0] == 0:
        return torch.empty(0, dtype=torch.int64, device=boxes.device)
    if boxes.shape[0] > _ext.NMS_MAX:
        raise ValueError(f'at most {_ext.NMS_MAX} boxes per call')
    order = torch.sort(scores.float(), descending=True, stable=True).indices
    keep = _ext.nms_keep(boxes.float()[order], iou_threshold)
    return order[keep.bool()]


def _candidates(p, conf_thres, multi_label, classes):
    """[k, 6] (x1, y1, x2, y2, score, class) of one image's prediction p [4 + nc, A]."""
    boxes = xywh2xyxy(p[:4].t())
    probs = p[4:].t()
    if multi_label and probs.shape[1] > 1:
        a, c = (probs > conf_thres).nonzero(as_tuple=True)
        rows = torch.cat((boxes[a], probs[a, c, None], c[:, None].to(p.dtype)), 1)
    else:
        score, c = probs.max(1)
        keep = score > conf_thres
        rows = torch.cat((boxes[keep], score[keep, None], c[keep, None].to(p.dtype)), 1)
    if classes is not None:
        rows = rows[torch.isin(rows[:, 5], torch.as_tensor(classes, dtype=rows.dtype, device=rows.device))]
    return rows


def non_max_suppression(prediction, conf_thres=0.25, iou_thres=0.45, classes=None, agnostic=False,
                        multi_label=False, labels=(), max_det=300, nm=0):
    """Per image of ``prediction`` [N, 4 + nc, A] (or a tuple whose first entry it is): the list of
    [k, 6] detections described in the module docstring."""
    if isinstance(prediction, (list, tuple)):
        prediction = prediction[0]
    if not (0 <= conf_thres <= 1 and 0 <= iou_thres <= 1):
        raise ValueError(f'conf_thres {conf_thres} and iou_thres {iou_thres} must lie in [0, 1]')
    if nm or any(len(lb) for lb in labels):
        raise NotImplementedError('non_max_suppression: labels and mask coefficients (nm) are not supported')
    out = []
    for p in prediction:
        # 16-bit predictions are processed in fp32: the class shift (up to 7680 nc px) exceeds fp16's range
        p = p if p.dtype == torch.float64 else p.float()
        rows = _candidates(p, conf_thres, multi_label, classes)
        if rows.shape[0]:
            rows = rows[torch.sort(rows[:, 4], descending=True, stable=True).indices[:_MAX_CANDIDATES]]
            shift = rows[:, 5:6] * (0 if agnostic else _CLASS_SHIFT)
            rows = rows[nms(rows[:, :4] + shift, rows[:, 4], iou_thres)[:max_det]]
        else:
            rows = torch.zeros((0, 6), dtype=p.dtype, device=p.device)
        out.append(rows)
    return out
