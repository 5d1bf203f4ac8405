"""ctypes binding of libkadconv_hip.so (declared in include/kadconv_hip.h).

This replaces the reference's JIT-built pybind11 extension
(acceleration/kadc_dcn16_backend.py:55-86, kadc_dcn16.cpp:247-330): the
library is prebuilt in-tree by ``kad-conv_amd/build.py`` and loaded here.
There is no fallback: if the library is missing or fails to load, every
fast-path call raises ``KadExtensionError``.

Every wrapper takes torch tensors, checks device/dtype/contiguity on the host,
passes raw pointers plus ``torch.cuda.current_stream()`` and converts a
negative return code into ``RuntimeError`` carrying ``kad_last_error()``.
"""
import ctypes
import os

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libkadconv_hip.so')

KAD_F32, KAD_F16, KAD_BF16 = 0, 1, 2
KAD_NHWC, KAD_NCHW = 0, 1
ABI_VERSION = 1

_DTYPES = {torch.float32: KAD_F32, torch.float16: KAD_F16, torch.bfloat16: KAD_BF16}


class KadExtensionError(RuntimeError):
    pass


c_int, c_i64, c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p


class DcnArgs(ctypes.Structure):
    _fields_ = [
        ('x', c_vp), ('offset', c_vp), ('mask', c_vp), ('wpack', c_vp), ('bias', c_vp),
        ('post_mul', c_vp), ('post_add', c_vp), ('post_scale', c_vp), ('out', c_vp), ('gap_partial', c_vp),
        ('off_sn', c_i64), ('off_sp', c_i64), ('off_sc', c_i64),
        ('mask_sn', c_i64), ('mask_sp', c_i64), ('mask_sc', c_i64),
        ('n', c_int), ('cin', c_int), ('cout', c_int), ('h', c_int), ('w', c_int), ('stride', c_int), ('pad', c_int),
        ('x_cs', c_int), ('out_layout', c_int), ('out_cs', c_int), ('dtype', c_int), ('relu', c_int),
    ]


# name -> (restype, argtypes); must list every symbol declared in include/kadconv_hip.h
SIGNATURES = {
    'kad_abi_version': (c_int, []),
    'kad_last_error': (ctypes.c_char_p, []),
    'kad_dcn_wpack_elems': (c_i64, [c_int, c_int]),
    'kad_dcn_pack_weights': (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    'kad_dcn_tiles': (c_int, [c_int, c_int]),
    'kad_dcn_fwd': (c_int, [ctypes.POINTER(DcnArgs), c_vp]),
}

_lib = None


def lib_path():
    return _LIB_PATH


def load():
    """Load (once) and return the ctypes library; raise KadExtensionError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise KadExtensionError(
            f'{_LIB_PATH} is not built; run `python kad-conv_amd/build.py` (hipcc, gfx950) first')
    try:
        lib = ctypes.CDLL(_LIB_PATH)
    except OSError as e:  # pragma: no cover - depends on the ROCm runtime install
        raise KadExtensionError(f'cannot load {_LIB_PATH}: {e}') from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.kad_abi_version() != ABI_VERSION:
        raise KadExtensionError(f'ABI mismatch: library {lib.kad_abi_version()} != binding {ABI_VERSION}')
    _lib = lib
    return lib


def _check(rc, what):
    if rc != 0:
        msg = load().kad_last_error().decode(errors='replace')
        raise RuntimeError(f'{what} failed ({rc}): {msg}')


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def kad_dtype(dtype):
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise TypeError(f'unsupported dtype {dtype}; expected float32, float16 or bfloat16') from None


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError('kadconv HIP ops need GPU tensors')


# ---------------------------------------------------------------------------- DCN
def dcn_wpack_elems(cin, cout):
    return load().kad_dcn_wpack_elems(cin, cout)


def dcn_tiles(ho, wo):
    return load().kad_dcn_tiles(ho, wo)


def dcn_pack_weights(weight, dtype):
    """weight [Cout, Cin, 3, 3] (any float dtype, GPU) -> packed buffer of `dtype`."""
    _need_gpu(weight)
    cout, cin = weight.shape[:2]
    if tuple(weight.shape[2:]) != (3, 3):
        raise ValueError('DSC kernels are 3x3')
    w32 = weight.detach().to(torch.float32).contiguous()
    out = torch.empty(dcn_wpack_elems(cin, cout), dtype=dtype, device=weight.device)
    _check(load().kad_dcn_pack_weights(_ptr(w32), _ptr(out), cin, cout, kad_dtype(dtype), _stream()),
           'kad_dcn_pack_weights')
    return out


def dcn_fwd(x_nhwc, cin, offset, offset_strides, mask, mask_strides, wpack, cout, out, *, stride=1, pad=1,
            bias=None, post_mul=None, post_add=None, post_scale=None, relu=False, out_layout=KAD_NHWC,
            gap_partial=None, h=None, w=None):
    """Low-level launcher: x_nhwc is [N, H, W, x_cs] (x_cs % 8 == 0, zero-padded channels)."""
    _need_gpu(x_nhwc, offset, mask, wpack, out)
    N, H, W, cs = x_nhwc.shape
    a = DcnArgs()
    a.x, a.offset, a.mask, a.wpack = _ptr(x_nhwc), _ptr(offset), _ptr(mask), _ptr(wpack)
    a.bias, a.post_mul, a.post_add, a.post_scale = _ptr(bias), _ptr(post_mul), _ptr(post_add), _ptr(post_scale)
    a.out, a.gap_partial = _ptr(out), _ptr(gap_partial)
    a.off_sn, a.off_sp, a.off_sc = offset_strides
    if mask is not None:
        a.mask_sn, a.mask_sp, a.mask_sc = mask_strides
    a.n, a.cin, a.cout, a.h, a.w, a.stride, a.pad = N, cin, cout, H, W, stride, pad
    a.x_cs = cs
    a.out_layout = out_layout
    a.out_cs = out.shape[-1] if out_layout == KAD_NHWC else cout
    a.dtype = kad_dtype(x_nhwc.dtype)
    a.relu = 1 if relu else 0
    for t in (offset, mask, bias, post_mul, post_add, post_scale, gap_partial):
        if t is not None and t.dtype != torch.float32:
            raise TypeError('offset/mask/epilogue/gap tensors must be float32')
    if wpack.dtype != x_nhwc.dtype or out.dtype != x_nhwc.dtype:
        raise TypeError('x, packed weights and out must share a dtype')
    _check(load().kad_dcn_fwd(ctypes.byref(a), _stream()), 'kad_dcn_fwd')
    return out
