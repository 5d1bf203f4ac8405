"""kadconv -- KAD-Conv with gfx950 (MI355X) HIP kernels behind the reference API.

Public API of the reference (KAD-Conv/kadconv/__init__.py:1-4): ``KADConv``,
``DSC``, ``LCSA``, ``enable_fast_inference``, ``disable_fast_inference``.
Added here: ``deform_conv2d`` (torchvision-compatible DCNv2 on the GPU), the
fused blocks ``Conv1x1SiLU``, ``SqueezeExcitation`` and ``KADDown``, and the
typed custom operators ``torch.ops.kadconv.deform_conv2d`` /
``torch.ops.kadconv.layer_fwd`` (kadconv.library).
"""
from . import library  # registers the kadconv:: custom operators
from .blocks import Conv1x1SiLU, KADDown, SqueezeExcitation
from .fast import disable_fast_inference, enable_fast_inference
from .kad_conv import DSC, LCSA, KADConv
from .ops import deform_conv2d

__all__ = ['KADConv', 'DSC', 'LCSA', 'enable_fast_inference', 'disable_fast_inference', 'deform_conv2d',
           'Conv1x1SiLU', 'SqueezeExcitation', 'KADDown']
