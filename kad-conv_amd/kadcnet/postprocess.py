"""Detection post-processing: non_max_suppression with the reference's
signature and steps (KAD-CNet/utils/general.py:881-990), its IoU suppression on
the GPU through the HIP kad_nms kernels (the reference calls
torchvision.ops.nms, which this image does not ship).

Candidate filtering, the best-class pick and the score sort are tensor
indexing on the prediction's device.  The sort is stable (ties keep anchor
order), so the kept indices are deterministic.
"""
import torch

from kadconv import _ext


def xywh2xyxy(x):
    """(cx, cy, w, h) -> (x1, y1, x2, y2) (utils/general.py xywh2xyxy)."""
    y = x.clone()
    y[..., 0] = x[..., 0] - x[..., 2] / 2
    y[..., 1] = x[..., 1] - x[..., 3] / 2
    y[..., 2] = x[..., 0] + x[..., 2] / 2
    y[..., 3] = x[..., 1] + x[..., 3] / 2
    return y


def nms(boxes, scores, iou_threshold):
    """Indices of the boxes kept by greedy NMS, by descending score (the contract of
    torchvision.ops.nms): a box is dropped when its IoU with a kept box of higher
    score exceeds iou_threshold.  GPU tensors only."""
    if not boxes.is_cuda:
        raise ValueError('kadcnet.postprocess.nms runs on the GPU (HIP kad_nms)')
    if boxes.shape[0] == 0:
        return torch.empty(0, dtype=torch.int64, device=boxes.device)
    if boxes.shape[0] > _ext.NMS_MAX:
        raise ValueError(f'at most {_ext.NMS_MAX} boxes per call')
    order = torch.sort(scores.float(), descending=True, stable=True).indices
    keep = _ext.nms_keep(boxes.float()[order], iou_threshold)
    return order[keep.bool()]


def non_max_suppression(prediction, conf_thres=0.25, iou_thres=0.45, classes=None, agnostic=False,
                        multi_label=False, labels=(), max_det=300, nm=0):
    """Per image: candidates whose best class score exceeds conf_thres, xywh ->
    xyxy, best class (or every class above conf_thres with multi_label), sort by
    score (at most 30000), class-offset boxes (7680 px per class unless
    agnostic), NMS at iou_thres, at most max_det.  Returns a list of [k, 6 + nm]
    tensors (x1, y1, x2, y2, conf, cls).  As general.py:881-990 without its
    wall-clock time limit and merge-NMS (off there)."""
    if isinstance(prediction, (list, tuple)):
        prediction = prediction[0]
    assert 0 <= conf_thres <= 1 and 0 <= iou_thres <= 1
    bs = prediction.shape[0]
    nc = prediction.shape[1] - nm - 4
    mi = 4 + nc
    xc = prediction[:, 4:mi].amax(1) > conf_thres
    max_wh, max_nms = 7680, 30000
    multi_label &= nc > 1
    output = [torch.zeros((0, 6 + nm), device=prediction.device)] * bs
    for xi, x in enumerate(prediction):
        x = x.T[xc[xi]]
        if labels and len(labels[xi]):
            lb = labels[xi]
            v = torch.zeros((len(lb), nc + nm + 5), device=x.device)
            v[:, :4] = lb[:, 1:5]
            v[range(len(lb)), lb[:, 0].long() + 4] = 1.0
            x = torch.cat((x, v), 0)
        if not x.shape[0]:
            continue
        box, cls, mask = x.split((4, nc, nm), 1)
        box = xywh2xyxy(box)
        if multi_label:
            i, j = (cls > conf_thres).nonzero(as_tuple=False).T
            x = torch.cat((box[i], x[i, 4 + j, None], j[:, None].float(), mask[i]), 1)
        else:
            conf, j = cls.max(1, keepdim=True)
            x = torch.cat((box, conf, j.float(), mask), 1)[conf.view(-1) > conf_thres]
        if classes is not None:
            x = x[(x[:, 5:6] == torch.tensor(classes, device=x.device)).any(1)]
        n = x.shape[0]
        if not n:
            continue
        x = x[torch.sort(x[:, 4], descending=True, stable=True).indices[:max_nms]]
        c = x[:, 5:6] * (0 if agnostic else max_wh)
        i = nms(x[:, :4] + c, x[:, 4], iou_thres)
        output[xi] = x[i[:max_det]]
    return output
