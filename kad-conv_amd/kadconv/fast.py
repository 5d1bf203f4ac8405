"""Switch KAD-Conv layers to the fused gfx950 HIP forward (and back).

Same entry points and discovery rule as the reference
(KAD-Conv/kadconv/fast.py:68-118): layers are found by class name, so the
switch also works on KAD-CNet models without editing them --
{KADConv, KADC4, KADC4_m} for KAD-Conv layers and {DSC, DCN_RCA} for the
deformable convolution.  Differences, by design:

* no env-var profile and no JIT build: the HIP library is prebuilt in-tree
  (``kad-conv_amd/build.py``); ``build_dir`` is accepted and unused;
* the per-call gate accepts any batch size, any H and W, and fp32 / fp16 /
  bf16, NCHW or channels-last, instead of fp32 (1, C, H, H) only
  (fast.py:38-40); training mode and CPU tensors take the plain forward;
* the GPU gate is gfx950 (MI355X) instead of SM80; ``allow_untested_gpu``
  lifts it;
* DSC modules that are not inside a KAD-Conv layer are switched too (the
  reference only accelerates DSCs inside KAD-Conv layers, because its fast DSC
  also applies the next BN and scale; here a standalone DSC gets its own
  fused forward);
* no module-global ``_active`` flag and no data_ptr-keyed side tables: the
  fused KADConv forward does not call its DSC's forward at all.
"""
import types

import torch

from . import _ext, library
from .fused import DSCPlan, KADConvPlan

_LAYER_TYPES = {'KADConv', 'KADC4', 'KADC4_m'}
_DSC_TYPES = {'DSC', 'DCN_RCA'}


def _is_gfx950(device):
    props = torch.cuda.get_device_properties(device)
    return 'gfx950' in getattr(props, 'gcnArchName', '')


def _install(module, plan):
    """Replace the instance's forward: eligible eval-mode calls run the plan through the
    typed custom op kadconv::layer_fwd (so torch.compile traces it as one operator),
    everything else the class's plain forward."""
    plain = types.MethodType(type(module).forward, module)
    handle = library.register_plan(plan)

    def forward(x):
        if module.training or not plan.eligible(x):
            return plain(x)
        with torch.no_grad():
            return torch.ops.kadconv.layer_fwd(x, handle)

    module._kad_plan = plan
    module._kad_handle = handle
    module.forward = forward


def enable_fast_inference(model, build_dir=None, allow_untested_gpu=False):
    """Switch every KAD-Conv (and DSC) layer of ``model`` to the fused HIP
    forward, in place, and return ``model``.

    ``model`` must be in eval mode and on a ROCm GPU.  Raises ``ValueError``
    otherwise, or when the model has no KAD-Conv / DSC layer, and
    ``kadconv._ext.KadExtensionError`` when libkadconv_hip.so is not built.
    """
    del build_dir  # the library is prebuilt; kept for signature compatibility
    if model.training:
        raise ValueError('call model.eval() before enable_fast_inference()')
    params = list(model.parameters())
    if not params or params[0].device.type != 'cuda':
        raise ValueError('move the model to a ROCm GPU first')
    device = params[0].device
    if not _is_gfx950(device) and not allow_untested_gpu:
        raise ValueError('the HIP kernels are built for gfx950 (MI355X); pass allow_untested_gpu=True to try '
                         'another GPU')
    layers = [m for m in model.modules() if type(m).__name__ in _LAYER_TYPES]
    inner = set()
    for layer in layers:
        inner.update(id(m) for m in layer.modules() if type(m).__name__ in _DSC_TYPES)
    dscs = [m for m in model.modules() if type(m).__name__ in _DSC_TYPES and id(m) not in inner]
    if not layers and not dscs:
        raise ValueError('no KAD-Conv layer found in the model')
    _ext.load()  # fail loudly now if the library is missing
    with torch.no_grad():
        for layer in layers:
            _install(layer, KADConvPlan(layer))
        for dsc in dscs:
            plan = DSCPlan(dsc)
            _install(dsc, plan)
    return model


def disable_fast_inference(model):
    """Go back to the plain forward (fast.py:113-118)."""
    for m in model.modules():
        if type(m).__name__ in _LAYER_TYPES | _DSC_TYPES and 'forward' in vars(m):
            del m.forward
            if hasattr(m, '_kad_plan'):
                del m._kad_plan
            if hasattr(m, '_kad_handle'):
                library.release_plan(m._kad_handle)
                del m._kad_handle
    return model
