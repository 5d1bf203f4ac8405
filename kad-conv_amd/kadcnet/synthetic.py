"""Seeded random-init KAD-CNet-S for the benchmark and parity tests (no
checkpoint is reachable offline: the released weights are on GitHub Releases,
KAD-CNet/README.md:12).

The model is built under a fixed torch seed, so every layer gets PyTorch's
default initialisation as in the reference (yolo.py:602-659: module init, the
256 x 256 stride probe, DDetect.bias_init, BN eps 1e-3).  One change: the
reference zero-initialises every DSC's conv_offset (KAD-CNet/models/module/ops.py:59-63),
which would make all offsets 0 and leave the deformable sampling untested; here
conv_offset weights are kaiming-uniform, U(+-1/sqrt(9 c)), bias 0, drawn from
the same seed.
"""
import math

import torch

from .yolo import DIOR_S_BASE, DetectionModel


def build_kadcnet_s(seed=0, cfg=DIOR_S_BASE, offsets=True, calibrate=True, offset_std_px=1.0, calib_shape=(2, 256),
                    var_floor=0.1):
    """A KAD-CNet-S DetectionModel (CPU, fp32, eval mode).

    offsets: conv_offset weights U(+-1/sqrt(9 c)), bias 0 (the reference
    zero-initialises them, which makes every offset 0).

    calibrate: PyTorch's default conv init shrinks activations by about 1/sqrt(3)
    per layer, so after the 22 layers of a random-init model the detection logits
    are the head biases alone (-10.2 +- 0.02); BatchNorm statistics set to batch
    statistics go the other way (a deep random network normalised by its own
    batch statistics amplifies every small-variance direction: fp32 and fp64
    runs of it differ by 50% after the neck).  In between, two train-mode
    forwards of a seeded U[0, 1] batch [calib_shape[0], 3, s, s] calibrate it:
    the first measures every DSC's offset standard deviation and rescales its
    conv_offset to offset_std_px pixels; the second sets every BatchNorm's
    running mean to the batch mean and its running variance to
    max(batch variance, var_floor), so no channel gains more than
    1 / sqrt(var_floor + eps).  With var_floor = 0.1 the class logits spread over
    about -18 .. +4 and fp32 / fp64 forwards agree to ~3e-6 at every layer.
    Momentum is then restored to 0.03."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        model = DetectionModel(cfg)
    dscs = [m for m in model.modules() if type(m).__name__ in ('DSC', 'DCN_RCA')]
    if offsets:
        gen = torch.Generator().manual_seed(seed + 1)
        with torch.no_grad():
            for m in dscs:
                bound = 1.0 / math.sqrt(9 * m.in_channels)
                m.conv_offset.weight.copy_((torch.rand(m.conv_offset.weight.shape, generator=gen) * 2 - 1) * bound)
                m.conv_offset.bias.zero_()
    if not calibrate:
        return model.eval()
    n, hw = calib_shape
    x = torch.rand(n, cfg.get('ch', 3), hw, hw, generator=torch.Generator().manual_seed(seed + 2))
    bns = [m for m in model.modules() if isinstance(m, torch.nn.BatchNorm2d)]
    model.train()
    with torch.no_grad():
        if offsets:
            stds = {}
            hooks = [m.conv_offset.register_forward_hook(
                lambda mod, inp, out, key=id(m): stds.__setitem__(key, out.std().item())) for m in dscs]
            model(x)
            for h in hooks:
                h.remove()
            for m in dscs:
                m.conv_offset.weight.mul_(offset_std_px / max(stds[id(m)], 1e-12))
        for bn in bns:
            bn.reset_running_stats()
            bn.momentum = None
        model(x)
        for bn in bns:
            bn.running_var.clamp_(min=var_floor)
            bn.momentum = 0.03
    return model.eval()
