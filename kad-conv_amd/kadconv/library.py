"""The fast forwards as typed PyTorch custom operators (torch.library).

The reference exposes its native kernels as typed pybind11 functions
(KAD-Conv/kadconv/acceleration/kadc_dcn16.cpp:247-330) and calls
torchvision's registered ``torchvision::deform_conv2d``.  Here the ctypes
calls are wrapped as custom ops with fake (meta) implementations, so
``torch.compile`` and FakeTensor tracing see typed operators with known output
shapes instead of breaking the graph at an opaque Python call:

  kadconv::deform_conv2d(input, offset, weight, bias?, stride_h, stride_w,
                         pad_h, pad_w, dil_h, dil_w, mask?) -> Tensor
      the functional operator (kadconv.ops.deform_conv2d, torchvision's
      argument meaning);
  kadconv::layer_fwd(x, handle) -> Tensor
      the fused forward of one enabled layer (a KADConv / KADC4 / DSC plan):
      ``handle`` names the plan in a process-wide registry, because a plan
      (packed weights, folded BN, streams) is not a tensor argument.  The
      output has x's shape for KAD-Conv layers and [N, Cout, H', W'] for DSCs,
      in x's memory format.

The eager implementations run the HIP kernels; nothing here falls back to
another implementation.
"""
import itertools

import torch

_PLANS = {}
_NEXT = itertools.count(1)


def register_plan(plan):
    """Store a plan and return its integer handle for ``kadconv::layer_fwd``."""
    h = next(_NEXT)
    _PLANS[h] = plan
    return h


def release_plan(handle):
    _PLANS.pop(handle, None)


def _memory_format(x):
    if x.dim() == 4 and x.is_contiguous(memory_format=torch.channels_last) and not x.is_contiguous():
        return torch.channels_last
    return torch.contiguous_format


@torch.library.custom_op('kadconv::layer_fwd', mutates_args=())
def layer_fwd(x: torch.Tensor, handle: int) -> torch.Tensor:
    with torch.no_grad():
        return _PLANS[handle].forward(x)


@layer_fwd.register_fake
def _(x, handle):
    plan = _PLANS[handle]
    n, _, h, w = x.shape
    cout, ho, wo = plan.out_shape(h, w)
    return torch.empty((n, cout, ho, wo), dtype=x.dtype, device=x.device, memory_format=_memory_format(x))


@torch.library.custom_op('kadconv::deform_conv2d', mutates_args=())
def deform_conv2d(input: torch.Tensor, offset: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                  stride_h: int, stride_w: int, pad_h: int, pad_w: int, dil_h: int, dil_w: int,
                  mask: torch.Tensor | None) -> torch.Tensor:
    from . import ops
    return ops.deform_conv2d(input, offset, weight, bias, stride=(stride_h, stride_w), padding=(pad_h, pad_w),
                             dilation=(dil_h, dil_w), mask=mask)


@deform_conv2d.register_fake
def _(input, offset, weight, bias, stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, mask):
    n, _, h, w = input.shape
    co, _, kh, kw = weight.shape
    ho = (h + 2 * pad_h - dil_h * (kh - 1) - 1) // stride_h + 1
    wo = (w + 2 * pad_w - dil_w * (kw - 1) - 1) // stride_w + 1
    return input.new_empty((n, co, ho, wo))
