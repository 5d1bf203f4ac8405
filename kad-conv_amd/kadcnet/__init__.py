"""kadcnet -- the KAD-CNet-S detector on the gfx950 HIP kernels.

The model classes keep the reference's names and state-dict layout
(KAD-CNet/models/{yolo.py, common.py}, models/module/KADC/module.py), so the
plain forward runs the reference's composition (CPU or GPU) and
``enable_fast_inference`` switches a model to the whole-network HIP forward
(kadcnet.fast).  ``non_max_suppression`` follows KAD-CNet/utils/general.py:881-990
with a HIP NMS.
"""
from .common import AConv, Concat, Conv, DFL, ELAN1, SP, SPPELAN, fuse_conv_and_bn, make_divisible
from .fast import KADCNetPlan, disable_fast_inference, enable_fast_inference
from .kadc import KADC4, KADC4_m, RepNCSP_KADC, RepNCSPELAN4_KADC
from .postprocess import nms, non_max_suppression, xywh2xyxy
from .synthetic import build_kadcnet_s
from .yolo import DIOR_S_BASE, DIOR_S_MGL, DDetect, DetectionModel, Model, dist2bbox, make_anchors, parse_model
