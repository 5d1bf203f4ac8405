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
ABI_VERSION = 4

_DTYPES = {torch.float32: KAD_F32, torch.float16: KAD_F16, torch.bfloat16: KAD_BF16}


class KadExtensionError(RuntimeError):
    pass


c_int, c_i64, c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p


class DcnArgs(ctypes.Structure):
    _fields_ = [
        ('x', c_vp), ('offset', c_vp), ('mask', c_vp), ('wpack', c_vp), ('bias', c_vp),
        ('post_mul', c_vp), ('post_add', c_vp), ('post_scale', c_vp), ('out', c_vp), ('gap_partial', c_vp),
        ('off_wpack', c_vp), ('off_bias', c_vp),
        ('off_sn', c_i64), ('off_sp', c_i64), ('off_sc', c_i64),
        ('mask_sn', c_i64), ('mask_sp', c_i64), ('mask_sc', c_i64),
        ('n', c_int), ('cin', c_int), ('cout', c_int), ('h', c_int), ('w', c_int), ('stride', c_int), ('pad', c_int),
        ('x_cs', c_int), ('out_layout', c_int), ('out_cs', c_int), ('dtype', c_int), ('relu', c_int),
        ('se_w1', c_vp), ('se_b1', c_vp), ('se_w2', c_vp), ('se_b2', c_vp), ('se_att', c_vp), ('se_count', c_vp),
        ('se_hid', c_int), ('se_inv_count', ctypes.c_float),
    ]


class LcsaArgs(ctypes.Structure):
    _fields_ = [('rows', c_vp), ('cols', c_vp), ('nrp', c_int), ('ncp', c_int), ('arow', c_vp), ('colm', c_vp),
                ('params', c_vp), ('emat', c_vp), ('ebias', c_vp), ('mask', c_vp),
                ('n', c_int), ('c', c_int), ('h', c_int), ('w', c_int)]


class GemmArgs(ctypes.Structure):
    _fields_ = [
        ('x', c_vp), ('wpack', c_vp), ('bias', c_vp), ('out', c_vp),
        ('n', c_int), ('cin', c_int), ('cout', c_int), ('h', c_int), ('w', c_int), ('pool', c_int),
        ('in_layout', c_int), ('x_cs', c_int), ('out_layout', c_int), ('out_cs', c_int), ('act', c_int),
        ('dtype', c_int),
    ]


MAX_BRANCHES = 4


class PyramidArgs(ctypes.Structure):
    _fields_ = [
        ('x', c_vp), ('n', c_int), ('cin', c_int), ('h', c_int), ('w', c_int), ('in_layout', c_int),
        ('x_cs', c_int), ('dtype', c_int), ('nb', c_int), ('ntx', c_int), ('nty', c_int),
        ('wpack', c_vp * 3), ('bias', c_vp * 3), ('out', c_vp * 3),
        ('cout', c_int * 3), ('out_cs', c_int * 3), ('out_h', c_int * 3), ('out_w', c_int * 3),
        ('rowpart', c_vp * 3), ('colpart', c_vp * 3),
    ]


class MergeArgs(ctypes.Structure):
    _fields_ = [
        ('out', c_vp), ('residual', c_vp), ('gate', c_vp),
        ('n', c_int), ('c', c_int), ('h', c_int), ('w', c_int), ('layout', c_int), ('dtype', c_int),
        ('nbranch', c_int), ('c_begin', c_int), ('c_end', c_int),
        ('br_z', c_vp * MAX_BRANCHES), ('br_att', c_vp * MAX_BRANCHES),
        ('br_c', c_int * MAX_BRANCHES), ('br_c_off', c_int * MAX_BRANCHES),
        ('br_h', c_int * MAX_BRANCHES), ('br_w', c_int * MAX_BRANCHES), ('br_cs', c_int * MAX_BRANCHES),
        ('br_coeff', ctypes.c_float * MAX_BRANCHES),
        ('out_cs', c_int), ('res_cs', c_int),
    ]


class ResampleArgs(ctypes.Structure):
    _fields_ = [('x', c_vp), ('out', c_vp)] + [(f, c_int) for f in (
        'n', 'c', 'h', 'w', 'ho', 'wo', 'x_cs', 'out_cs', 'mode', 'k', 's', 'p', 'dtype')]


MAX_LEVELS = 4


class DecodeArgs(ctypes.Structure):
    _fields_ = [('head', c_vp * MAX_LEVELS), ('lh', c_int * MAX_LEVELS), ('lw', c_int * MAX_LEVELS),
                ('head_cs', c_int * MAX_LEVELS), ('anchor_off', c_int * MAX_LEVELS),
                ('stride', ctypes.c_float * MAX_LEVELS), ('out', c_vp)] + [(f, c_int) for f in (
                    'n', 'nl', 'nc', 'reg_max', 'box_ch', 'dtype')]


# name -> (restype, argtypes); must list every symbol declared in include/kadconv_hip.h
SIGNATURES = {
    'kad_abi_version': (c_int, []),
    'kad_last_error': (ctypes.c_char_p, []),
    'kad_dcn_wpack_elems': (c_i64, [c_int, c_int]),
    'kad_dcn_pack_weights': (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    'kad_dcn_tiles': (c_int, [c_int, c_int]),
    'kad_dcn_fwd': (c_int, [ctypes.POINTER(DcnArgs), c_vp]),
    'kad_conv3x3_fwd': (c_int, [ctypes.POINTER(DcnArgs), c_vp]),
    'kad_dsc_fwd': (c_int, [ctypes.POINTER(DcnArgs), c_vp]),
    'kad_dsc_fwd_noalloc': (c_int, [ctypes.POINTER(DcnArgs), c_vp]),
    'kad_dsc_fwd_group': (c_int, [ctypes.POINTER(DcnArgs), c_int, c_vp]),
    'kad_lcsa_prep_group': (c_int, [ctypes.POINTER(LcsaArgs), c_int, c_vp]),
    'kad_lcsa_mask_group': (c_int, [ctypes.POINTER(LcsaArgs), c_int, c_int, c_vp]),
    'kad_scale_residual': (c_int, [c_vp, c_vp, c_vp] + [c_int] * 8 + [c_vp]),
    'kad_gemm_wpack_elems': (c_i64, [c_int, c_int]),
    'kad_gemm_pack_weights': (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    'kad_gemm1x1_fwd': (c_int, [ctypes.POINTER(GemmArgs), c_vp]),
    'kad_kaddown_prep': (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_pyramid_tiles': (c_int, [c_int, c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int)]),
    'kad_pyramid_proj': (c_int, [ctypes.POINTER(PyramidArgs), c_vp]),
    'kad_lcsa_params_elems': (c_i64, [c_int]),
    'kad_lcsa_emat_elems': (c_i64, [c_int]),
    'kad_axial_sums': (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_axial_sums_nchw': (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_axial_means': (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_axial_means_nchw': (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_lcsa_pack': (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_vp]),
    'kad_lcsa_prep': (c_int, [c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp]),
    'kad_lcsa_mask': (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_lcsa_mask_splits': (c_int, [c_int, c_int, c_int, c_int]),
    'kad_lcsa_mask_work_elems': (c_i64, [c_int, c_int, c_int, c_int]),
    'kad_lcsa_mask_split': (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int,
                                    c_vp, c_vp]),
    'kad_se_pool_tiles': (c_int, [c_int, c_int, c_int]),
    'kad_se_pool': (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_se_mlp': (c_int, [c_vp, c_int, ctypes.c_float, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    'kad_se_mlp_ws': (c_int, [c_vp, c_int, ctypes.c_float, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp,
                              c_vp]),
    'kad_se_hidden': (c_int, [c_vp, c_int, ctypes.c_float, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    'kad_se_scale': (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_channel_scale': (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_to_nhwc': (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_se_nchw_fits': (c_int, [c_int, c_int, c_int, c_int, c_int]),
    'kad_se_nchw': (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int,
                            c_vp]),
    'kad_nhwc_pad': (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_vp]),
    'kad_branch_merge': (c_int, [ctypes.POINTER(MergeArgs), c_vp]),
    'kad_conv_fwd': (c_int, [ctypes.POINTER(DcnArgs), c_vp]),
    'kad_stem_conv_fwd': (c_int, [ctypes.POINTER(DcnArgs), c_vp]),
    'kad_nhwc_resample': (c_int, [ctypes.POINTER(ResampleArgs), c_vp]),
    'kad_ddetect_decode': (c_int, [ctypes.POINTER(DecodeArgs), c_vp]),
    'kad_nms_mask_words': (c_i64, [c_int]),
    'kad_nms': (c_int, [c_vp, c_vp, c_vp, c_int, ctypes.c_float, c_vp]),
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
def _out_cs(out, layout, cout, ho, wo):
    """Channel stride (NHWC) or channel planes per image (NCHW) of `out`, which may be a
    channel slice of a wider tensor; pixel / plane strides must be dense."""
    if layout == KAD_NHWC:
        if out.stride(3) != 1 or out.stride(1) != out.stride(2) * wo or out.stride(0) != out.stride(1) * ho:
            raise ValueError('NHWC output must be dense apart from its channel stride')
        return out.stride(2)
    if out.stride(3) != 1 or out.stride(2) != wo or out.stride(1) != ho * wo or out.stride(0) % (ho * wo):
        raise ValueError('NCHW output must be dense channel planes')
    return out.stride(0) // (ho * wo)


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


def _set_se_weights(a, se, n, cout, ho, wo):
    """MLP fields of the fused squeeze-excitation: se = (w1 [hid, C], b1, w2 [C, hid], b2, att [N, C])."""
    w1, b1, w2, b2, att = se[:5]
    _need_gpu(w1, b1, w2, b2, att)
    for t in (w1, b1, w2, b2, att):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise TypeError('SE weights and att must be contiguous float32')
    hid = w1.shape[0]
    if tuple(w1.shape) != (hid, cout) or tuple(w2.shape) != (cout, hid) or tuple(att.shape) != (n, cout):
        raise ValueError('SE shapes: w1 [hid, C], w2 [C, hid], att [N, C]')
    a.se_w1, a.se_b1, a.se_w2, a.se_b2 = _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2)
    a.se_att, a.se_hid, a.se_inv_count = _ptr(att), hid, 1.0 / (ho * wo)


def _set_se(a, se, gap_partial, n, cout, ho, wo):
    """Fused squeeze-excitation fields of kad_dcn_args: se = (w1 [hid, C], b1, w2 [C, hid], b2, att [N, C],
    count [N] int32, zero before the first call)."""
    if se is None:
        return
    count = se[5]
    if gap_partial is None:
        raise ValueError('the fused squeeze-excitation reads the GAP partials: pass gap_partial')
    _set_se_weights(a, se, n, cout, ho, wo)
    if count.dtype != torch.int32 or count.numel() < n:
        raise ValueError('SE counters: int32 [N]')
    a.se_count = _ptr(count)


def dcn_fwd(x_nhwc, cin, offset, offset_strides, mask, mask_strides, wpack, cout, out, *, stride=1, pad=1,
            bias=None, post_mul=None, post_add=None, post_scale=None, relu=False, out_layout=KAD_NHWC,
            gap_partial=None, h=None, w=None, se=None):
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
    a.out_cs = _out_cs(out, out_layout, cout, (H + 2 * pad - 3) // stride + 1, (W + 2 * pad - 3) // stride + 1)
    a.dtype = kad_dtype(x_nhwc.dtype)
    a.relu = 1 if relu else 0
    for t in (offset, mask, bias, post_mul, post_add, post_scale, gap_partial):
        if t is not None and t.dtype != torch.float32:
            raise TypeError('offset/mask/epilogue/gap tensors must be float32')
    if wpack.dtype != x_nhwc.dtype or out.dtype != x_nhwc.dtype:
        raise TypeError('x, packed weights and out must share a dtype')
    _set_se(a, se, gap_partial, N, cout, (H + 2 * pad - 3) // stride + 1, (W + 2 * pad - 3) // stride + 1)
    _check(load().kad_dcn_fwd(ctypes.byref(a), _stream()), 'kad_dcn_fwd')
    return out


def dsc_args(x_nhwc, cin, off_wpack, off_bias, mask, mask_strides, wpack, cout, out, *, stride=1, pad=1,
             bias=None, post_mul=None, post_add=None, post_scale=None, relu=False, out_layout=KAD_NHWC,
             gap_partial=None, se=None, noalloc=False):
    """kad_dcn_args of one fused DSC problem (checked), for kad_dsc_fwd / _noalloc / _group."""
    _need_gpu(x_nhwc, off_wpack, wpack, out)
    if noalloc and gap_partial is not None:
        raise ValueError('kad_dsc_fwd_noalloc keeps the GAP partials in its own scratch: pass gap_partial=None')
    N, H, W, cs = x_nhwc.shape
    a = DcnArgs()
    a.x, a.mask, a.wpack = _ptr(x_nhwc), _ptr(mask), _ptr(wpack)
    a.off_wpack, a.off_bias = _ptr(off_wpack), _ptr(off_bias)
    a.bias, a.post_mul, a.post_add, a.post_scale = _ptr(bias), _ptr(post_mul), _ptr(post_add), _ptr(post_scale)
    a.out, a.gap_partial = _ptr(out), _ptr(gap_partial)
    if mask is not None:
        a.mask_sn, a.mask_sp, a.mask_sc = mask_strides
    a.n, a.cin, a.cout, a.h, a.w, a.stride, a.pad = N, cin, cout, H, W, stride, pad
    a.x_cs = cs
    a.out_layout = out_layout
    a.out_cs = _out_cs(out, out_layout, cout, (H + 2 * pad - 3) // stride + 1, (W + 2 * pad - 3) // stride + 1)
    a.dtype = kad_dtype(x_nhwc.dtype)
    a.relu = 1 if relu else 0
    for t in (off_bias, mask, bias, post_mul, post_add, post_scale, gap_partial):
        if t is not None and t.dtype != torch.float32:
            raise TypeError('offset bias/mask/epilogue/gap tensors must be float32')
    if wpack.dtype != x_nhwc.dtype or off_wpack.dtype != x_nhwc.dtype or out.dtype != x_nhwc.dtype:
        raise TypeError('x, packed weights and out must share a dtype')
    ho, wo = (H + 2 * pad - 3) // stride + 1, (W + 2 * pad - 3) // stride + 1
    if noalloc:
        if se is not None:
            _set_se_weights(a, se, N, cout, ho, wo)
    else:
        _set_se(a, se, gap_partial, N, cout, ho, wo)
    return a


def dsc_fwd(x_nhwc, cin, off_wpack, off_bias, mask, mask_strides, wpack, cout, out, *, noalloc=False, **kw):
    """conv_offset + deformable conv in one launch (offsets never leave the chip); with `se`,
    also the squeeze-excitation MLP of the output (see _set_se).  noalloc=True calls
    kad_dsc_fwd_noalloc: `se` is then (w1, b1, w2, b2, att) and the GAP partials and arrival
    counters come from the library's own device scratch (gap_partial must be None)."""
    a = dsc_args(x_nhwc, cin, off_wpack, off_bias, mask, mask_strides, wpack, cout, out, noalloc=noalloc, **kw)
    if noalloc:
        _check(load().kad_dsc_fwd_noalloc(ctypes.byref(a), _stream()), 'kad_dsc_fwd_noalloc')
    else:
        _check(load().kad_dsc_fwd(ctypes.byref(a), _stream()), 'kad_dsc_fwd')
    return out


def dsc_fwd_group(args):
    """Several fused DSC problems (kad_dcn_args from dsc_args) in one launch."""
    arr = (DcnArgs * len(args))(*args)
    _check(load().kad_dsc_fwd_group(arr, len(args), _stream()), 'kad_dsc_fwd_group')


def lcsa_args(rows, nrp, cols, ncp, arow, colm, params, emat, ebias, mask, n, c, h, w):
    _need_gpu(rows, cols, arow, colm, params, emat, ebias, mask)
    a = LcsaArgs()
    a.rows, a.cols, a.nrp, a.ncp = _ptr(rows), _ptr(cols), nrp, ncp
    a.arow, a.colm, a.params, a.emat, a.ebias, a.mask = _ptr(arow), _ptr(colm), _ptr(params), _ptr(emat), \
        _ptr(ebias), _ptr(mask)
    a.n, a.c, a.h, a.w = n, c, h, w
    return a


def lcsa_prep_group(args):
    arr = (LcsaArgs * len(args))(*args)
    _check(load().kad_lcsa_prep_group(arr, len(args), _stream()), 'kad_lcsa_prep_group')


def lcsa_mask_group(args, emat_dtype):
    arr = (LcsaArgs * len(args))(*args)
    _check(load().kad_lcsa_mask_group(arr, len(args), kad_dtype(emat_dtype), _stream()), 'kad_lcsa_mask_group')


def conv3x3_fwd(x_nhwc, cin, wpack, cout, out, *, stride=1, pad=1, bias=None, out_layout=KAD_NHWC):
    """Plain 3x3 conv (offset branch) on NHWC input; `out` must be float32."""
    _need_gpu(x_nhwc, wpack, out)
    if out.dtype != torch.float32:
        raise TypeError('conv3x3_fwd writes float32')
    N, H, W, cs = x_nhwc.shape
    a = DcnArgs()
    a.x, a.wpack, a.bias, a.out = _ptr(x_nhwc), _ptr(wpack), _ptr(bias), _ptr(out)
    a.n, a.cin, a.cout, a.h, a.w, a.stride, a.pad = N, cin, cout, H, W, stride, pad
    a.x_cs = cs
    a.out_layout = out_layout
    a.out_cs = _out_cs(out, out_layout, cout, (H + 2 * pad - 3) // stride + 1, (W + 2 * pad - 3) // stride + 1)
    a.dtype = kad_dtype(x_nhwc.dtype)
    _check(load().kad_conv3x3_fwd(ctypes.byref(a), _stream()), 'kad_conv3x3_fwd')
    return out


# ---------------------------------------------------------------------------- 1x1 GEMM
def gemm_pack_weights(weight, dtype):
    """weight [Cout, Cin] or [Cout, Cin, 1, 1] -> packed buffer of `dtype`."""
    _need_gpu(weight)
    cout = weight.shape[0]
    w32 = weight.detach().reshape(cout, -1).to(torch.float32).contiguous()
    cin = w32.shape[1]
    out = torch.empty(load().kad_gemm_wpack_elems(cin, cout), dtype=dtype, device=weight.device)
    _check(load().kad_gemm_pack_weights(_ptr(w32), _ptr(out), cin, cout, kad_dtype(dtype), _stream()),
           'kad_gemm_pack_weights')
    return out


def gemm1x1_fwd(x, in_layout, cin, wpack, cout, out, out_layout, *, bias=None, pool=1, act=0, h=None, w=None):
    """x: NCHW [N,Cin,H,W] or NHWC [N,H,W,x_cs]; out: NCHW [N,Cout,H/s,W/s] or NHWC [N,H/s,W/s,out_cs]."""
    _need_gpu(x, wpack, out, bias)
    a = GemmArgs()
    if in_layout == KAD_NCHW:
        N, C, H, W = x.shape
        cs = C
    else:
        N, H, W, cs = x.shape
    a.x, a.wpack, a.bias, a.out = _ptr(x), _ptr(wpack), _ptr(bias), _ptr(out)
    a.n, a.cin, a.cout, a.h, a.w, a.pool = N, cin, cout, H, W, pool
    a.in_layout, a.x_cs = in_layout, cs
    a.out_layout = out_layout
    a.out_cs = out.shape[-1] if out_layout == KAD_NHWC else cout
    a.act = act
    a.dtype = kad_dtype(x.dtype)
    if wpack.dtype != x.dtype or out.dtype != x.dtype:
        raise TypeError('x, packed weights and out must share a dtype')
    if bias is not None and bias.dtype != torch.float32:
        raise TypeError('bias must be float32')
    _check(load().kad_gemm1x1_fwd(ctypes.byref(a), _stream()), 'kad_gemm1x1_fwd')
    return out


def kaddown_prep(x, u, nb):
    """x NCHW [N,C,H,W] -> u NCHW [N,nb*C,H//2,W//2]: the 2^(b+1)-pooled input of
    branch b resized to (H//2, W//2), stacked along channels."""
    _need_gpu(x, u)
    N, C, H, W = x.shape
    if not x.is_contiguous() or not u.is_contiguous() or tuple(u.shape) != (N, nb * C, H // 2, W // 2):
        raise ValueError('kaddown_prep: x and u must be contiguous NCHW, u [N, nb*C, H//2, W//2]')
    if u.dtype != x.dtype:
        raise TypeError('kaddown_prep: x and u must share a dtype')
    _check(load().kad_kaddown_prep(_ptr(x), _ptr(u), N, C, H, W, nb, kad_dtype(x.dtype), _stream()),
           'kad_kaddown_prep')
    return u


# ---------------------------------------------------------------------------- pyramid
def pyramid_tiles(h, w):
    tx, ty = c_int(), c_int()
    _check(load().kad_pyramid_tiles(h, w, ctypes.byref(tx), ctypes.byref(ty)), 'kad_pyramid_tiles')
    return tx.value, ty.value


def pyramid_proj(x, in_layout, cin, branches):
    """branches: list of dicts {wpack, bias (fp32 or None), cout, out (NHWC [N,h_b,w_b,cs]),
    rowpart (fp32 [N,ntx,h_b,cout] or None), colpart (fp32 [N,nty,w_b,cout] or None)}."""
    _need_gpu(x)
    if in_layout == KAD_NCHW:
        N, C, H, W = x.shape
        cs = C
    else:
        N, H, W, cs = _nhwc_cs(x)   # x may be a channel slice of a wider NHWC buffer
    if not 1 <= len(branches) <= 3:
        raise ValueError('kad_pyramid_proj takes 1..3 branches')
    a = PyramidArgs()
    a.x, a.n, a.cin, a.h, a.w, a.in_layout, a.x_cs = _ptr(x), N, cin, H, W, in_layout, cs
    a.dtype = kad_dtype(x.dtype)
    a.nb = len(branches)
    a.ntx, a.nty = pyramid_tiles(H, W)
    for i, b in enumerate(branches):
        out = b['out']
        _need_gpu(out, b['wpack'], b.get('bias'), b.get('rowpart'), b.get('colpart'))
        if out.dtype != x.dtype or b['wpack'].dtype != x.dtype:
            raise TypeError('x, packed weights and outputs must share a dtype')
        a.wpack[i] = b['wpack'].data_ptr()
        a.bias[i] = b['bias'].data_ptr() if b.get('bias') is not None else None
        a.out[i] = out.data_ptr()
        a.cout[i], a.out_cs[i], a.out_h[i], a.out_w[i] = b['cout'], out.shape[3], out.shape[1], out.shape[2]
        a.rowpart[i] = b['rowpart'].data_ptr() if b.get('rowpart') is not None else None
        a.colpart[i] = b['colpart'].data_ptr() if b.get('colpart') is not None else None
    _check(load().kad_pyramid_proj(ctypes.byref(a), _stream()), 'kad_pyramid_proj')


# ---------------------------------------------------------------------------- LCSA
def lcsa_params_elems(c):
    return load().kad_lcsa_params_elems(c)


def lcsa_pack(params, c, emat_dtype):
    """-> (E [16*11*roundup(c,32)] of emat_dtype (float16 or float32), ebias [16] fp32)."""
    _need_gpu(params)
    emat = torch.empty(load().kad_lcsa_emat_elems(c), dtype=emat_dtype, device=params.device)
    ebias = torch.empty(16, dtype=torch.float32, device=params.device)
    _check(load().kad_lcsa_pack(_ptr(params), _ptr(emat), _ptr(ebias), c, kad_dtype(emat_dtype), _stream()),
           'kad_lcsa_pack')
    return emat, ebias


def axial_sums(x_nhwc, c, rows, cols):
    _need_gpu(x_nhwc, rows, cols)
    N, H, W, cs = x_nhwc.shape
    _check(load().kad_axial_sums(_ptr(x_nhwc), _ptr(rows), _ptr(cols), N, c, H, W, cs, kad_dtype(x_nhwc.dtype),
                                 _stream()), 'kad_axial_sums')


AXIAL_NCHW_MAX_PX = 12288


def axial_sums_nchw(x, rows, cols):
    """Row / column sums of a contiguous NCHW map (planes of at most AXIAL_NCHW_MAX_PX pixels)."""
    _need_gpu(x, rows, cols)
    N, C, H, W = x.shape
    if not x.is_contiguous():
        raise ValueError('axial_sums_nchw: x must be contiguous NCHW')
    _check(load().kad_axial_sums_nchw(_ptr(x), _ptr(rows), _ptr(cols), N, C, H, W, kad_dtype(x.dtype), _stream()),
           'kad_axial_sums_nchw')


def axial_means(x_nhwc, c, arow, colm):
    """Row / column means of an NHWC map straight into LCSA's arow / colm (no partial slices)."""
    _need_gpu(x_nhwc, arow, colm)
    N, H, W, cs = x_nhwc.shape
    _check(load().kad_axial_means(_ptr(x_nhwc), _ptr(arow), _ptr(colm), N, c, H, W, cs, kad_dtype(x_nhwc.dtype),
                                  _stream()), 'kad_axial_means')


def axial_means_nchw(x, arow, colm):
    """Row / column means of a contiguous NCHW map (planes of at most AXIAL_NCHW_MAX_PX pixels)."""
    _need_gpu(x, arow, colm)
    N, C, H, W = x.shape
    if not x.is_contiguous():
        raise ValueError('axial_means_nchw: x must be contiguous NCHW')
    _check(load().kad_axial_means_nchw(_ptr(x), _ptr(arow), _ptr(colm), N, C, H, W, kad_dtype(x.dtype), _stream()),
           'kad_axial_means_nchw')


def lcsa_prep(rows, nrp, cols, ncp, arow, colm, n, c, h, w):
    _need_gpu(rows, cols, arow, colm)
    _check(load().kad_lcsa_prep(_ptr(rows), nrp, _ptr(cols), ncp, _ptr(arow), _ptr(colm), n, c, h, w, _stream()),
           'kad_lcsa_prep')


def lcsa_mask_splits(n, c, h, w):
    return load().kad_lcsa_mask_splits(n, c, h, w)


def lcsa_mask_work_elems(n, h, w, ksplit):
    return load().kad_lcsa_mask_work_elems(n, h, w, ksplit)


def lcsa_mask(arow, colm, params, emat, ebias, mask, n, c, h, w, ksplit=1, work=None):
    """ksplit > 1: the channel contraction split over blocks, partial logits in `work`
    (fp32, lcsa_mask_work_elems(n, h, w, ksplit) elements)."""
    _need_gpu(arow, colm, params, emat, ebias, mask, work)
    if ksplit == 1:
        _check(load().kad_lcsa_mask(_ptr(arow), _ptr(colm), _ptr(params), _ptr(emat), _ptr(ebias), _ptr(mask), n,
                                    c, h, w, kad_dtype(emat.dtype), _stream()), 'kad_lcsa_mask')
        return
    if work is None or work.dtype != torch.float32 or work.numel() < lcsa_mask_work_elems(n, h, w, ksplit):
        raise ValueError('lcsa_mask: ksplit > 1 needs a float32 work buffer of lcsa_mask_work_elems elements')
    _check(load().kad_lcsa_mask_split(_ptr(arow), _ptr(colm), _ptr(params), _ptr(emat), _ptr(ebias), _ptr(mask), n,
                                      c, h, w, kad_dtype(emat.dtype), ksplit, _ptr(work), _stream()),
           'kad_lcsa_mask_split')


# ---------------------------------------------------------------------------- SE
def se_pool_tiles(h, w, layout):
    return load().kad_se_pool_tiles(h, w, layout)


def se_pool(x, c, layout, partial):
    _need_gpu(x, partial)
    if layout == KAD_NCHW:
        N, _, H, W = x.shape
        cs = c
    else:
        N, H, W, cs = x.shape
    _check(load().kad_se_pool(_ptr(x), _ptr(partial), N, c, H, W, layout, cs, kad_dtype(x.dtype), _stream()),
           'kad_se_pool')


def se_mlp(partial, tiles, inv_count, w1, b1, w2, b2, att, n, c, hid):
    _need_gpu(partial, w1, b1, w2, b2, att)
    _check(load().kad_se_mlp(_ptr(partial), tiles, inv_count, _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(att),
                             n, c, hid, _stream()), 'kad_se_mlp')


def se_mlp_ws(partial, tiles, inv_count, w1, b1, w2, b2, att, n, c, hid, hidden):
    """kad_se_mlp_ws: the MLP spread over the batch, hidden [n][hid] fp32 as workspace."""
    _need_gpu(partial, w1, b1, w2, b2, att, hidden)
    assert hidden.dtype == torch.float32 and hidden.is_contiguous() and hidden.numel() >= n * hid
    _check(load().kad_se_mlp_ws(_ptr(partial), tiles, inv_count, _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(att),
                                n, c, hid, _ptr(hidden), _stream()), 'kad_se_mlp_ws')


def se_hidden(partial, tiles, inv_count, w1, b1, hidden, n, c, hid):
    """kad_se_hidden: hidden [n][hid] = relu(W1 g + b1) from the GAP partials."""
    _need_gpu(partial, w1, b1, hidden)
    assert hidden.dtype == torch.float32 and hidden.is_contiguous() and hidden.numel() >= n * hid
    _check(load().kad_se_hidden(_ptr(partial), tiles, inv_count, _ptr(w1), _ptr(b1), _ptr(hidden), n, c, hid,
                                _stream()), 'kad_se_hidden')


def se_nchw_fits(n, c, h, w, hid):
    return bool(load().kad_se_nchw_fits(n, c, h, w, hid))


def se_nchw(x, w1, b1, w2, b2, att, out):
    """kad_se_nchw: the SE block on a dense NCHW x in two launches; att [N, C] fp32 written too."""
    _need_gpu(x, w1, w2, att, out)
    N, C, H, W = x.shape
    hid = w1.shape[0]
    if not (x.is_contiguous() and out.is_contiguous() and out.dtype == x.dtype and out.shape == x.shape):
        raise ValueError('se_nchw wants dense NCHW x and out of one shape and dtype')
    for t in (w1, w2, att) + ((b1,) if b1 is not None else ()) + ((b2,) if b2 is not None else ()):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise TypeError('se_nchw: weights, biases and att are dense float32')
    hpart = torch.empty(N * (C // 32) * 64, dtype=torch.float32, device=x.device)
    _check(load().kad_se_nchw(_ptr(x), _ptr(out), _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(att), _ptr(hpart), N, C,
                              H, W, hid, kad_dtype(x.dtype), _stream()), 'kad_se_nchw')
    return out


def se_scale(x, hidden, w2, b2, att, out, hid):
    """kad_se_scale: NCHW out = x * sigmoid(W2 hidden + b2) (att written too)."""
    _need_gpu(x, hidden, w2, b2, att, out)
    N, C, H, W = x.shape
    assert x.is_contiguous() and out.is_contiguous() and out.dtype == x.dtype
    assert att.dtype == torch.float32 and att.is_contiguous() and att.numel() >= N * C
    _check(load().kad_se_scale(_ptr(x), _ptr(hidden), _ptr(w2), _ptr(b2), _ptr(att), _ptr(out), N, C, H, W, hid,
                               kad_dtype(x.dtype), _stream()), 'kad_se_scale')


def channel_scale(x, att, out, c, layout):
    _need_gpu(x, att, out)
    if layout == KAD_NCHW:
        N, _, H, W = x.shape
        cs = c
    else:
        N, H, W, cs = x.shape
    _check(load().kad_channel_scale(_ptr(x), _ptr(att), _ptr(out), N, c, H, W, layout, cs, kad_dtype(x.dtype),
                                    _stream()), 'kad_channel_scale')


# ---------------------------------------------------------------------------- layout / merge
def to_nhwc(x, out):
    """x NCHW contiguous -> out NHWC [N,H,W,cs] (pad channels zeroed)."""
    _need_gpu(x, out)
    N, C, H, W = x.shape
    _check(load().kad_to_nhwc(_ptr(x), _ptr(out), N, C, H, W, out.shape[-1], kad_dtype(x.dtype), _stream()),
           'kad_to_nhwc')
    return out


def nhwc_pad(x, out):
    """x: an NHWC view [N,H,W,C] with channel stride 1 and pixel stride >= C ->
    out NHWC [N,H,W,cs] dense, cs % 8 == 0, channels >= C zeroed; one launch."""
    _need_gpu(x, out)
    N, H, W, C = x.shape
    xs = x.stride()
    if xs[3] != 1 or xs[2] < C or xs[1] != xs[2] * W or xs[0] != xs[1] * H:
        raise ValueError('nhwc_pad wants channels-last pixels of one stride')
    if not out.is_contiguous() or tuple(out.shape[:3]) != (N, H, W) or out.dtype != x.dtype:
        raise ValueError('nhwc_pad: out must be dense [N, H, W, cs] of x\'s dtype')
    _check(load().kad_nhwc_pad(_ptr(x), xs[2], _ptr(out), out.shape[3], N, C, H, W, kad_dtype(x.dtype), _stream()),
           'kad_nhwc_pad')
    return out


def scale_residual(out, att, residual, c_off, c, layout):
    """In place on channels [c_off, c_off + c) of `out` (full tensor, NCHW or NHWC):
    out = att[n, j] * out + residual."""
    _need_gpu(out, att, residual)
    if layout == KAD_NCHW:
        N, C, H, W = out.shape
    else:
        N, H, W, C = out.shape
    if not out.is_contiguous() or (residual is not None and (residual.shape != out.shape or not residual.is_contiguous())):
        raise ValueError('scale_residual wants dense out / residual of one shape')
    if att.dtype != torch.float32 or tuple(att.shape) != (N, c):
        raise TypeError('att must be float32 [N, c]')
    _check(load().kad_scale_residual(_ptr(out), _ptr(att), _ptr(residual), N, c, H, W, C, c_off, layout,
                                     kad_dtype(out.dtype), _stream()), 'kad_scale_residual')
    return out


def branch_merge(out, layout, branches, residual=None, gate=None, channels=None):
    """branches: list of dicts {z (NHWC [N,h,w,cs]), c, c_off, att (fp32 [N,c] or None), coeff};
    channels = (begin, end): the output channels written (default: all)."""
    _need_gpu(out, residual, gate)
    if len(branches) > MAX_BRANCHES:
        raise ValueError(f'at most {MAX_BRANCHES} branches')
    a = MergeArgs()
    if layout == KAD_NCHW:
        N, C, H, W = out.shape
    else:
        N, H, W, C = out.shape
        # out / residual may be channel slices of wider NHWC buffers (pixel strides >= C)
        a.out_cs = _nhwc_cs(out)[3]
        if residual is not None:
            a.res_cs = _nhwc_cs(residual)[3]
    a.out, a.residual, a.gate = _ptr(out), _ptr(residual), _ptr(gate)
    a.n, a.c, a.h, a.w, a.layout, a.dtype, a.nbranch = N, C, H, W, layout, kad_dtype(out.dtype), len(branches)
    if channels is not None:
        a.c_begin, a.c_end = channels
    for i, b in enumerate(branches):
        z = b['z']
        _need_gpu(z, b.get('att'))
        if z.dtype != out.dtype:
            raise TypeError('branch maps and output must share a dtype')
        a.br_z[i] = z.data_ptr()
        att = b.get('att')
        a.br_att[i] = att.data_ptr() if att is not None else None
        a.br_c[i], a.br_c_off[i] = b['c'], b['c_off']
        _, zh, zw, zcs = _nhwc_cs(z)   # z may be a channel slice (e.g. the output's own window)
        a.br_h[i], a.br_w[i], a.br_cs[i] = zh, zw, zcs
        a.br_coeff[i] = float(b.get('coeff', 1.0))
    _check(load().kad_branch_merge(ctypes.byref(a), _stream()), 'kad_branch_merge')
    return out


# ---------------------------------------------------------------------------- network ops (KAD-CNet-S)
KAD_ACT_NONE, KAD_ACT_RELU, KAD_ACT_SILU = 0, 1, 2
KAD_RS_AVG, KAD_RS_MAX, KAD_RS_NEAREST, KAD_RS_MAX3 = 0, 1, 2, 3


def _nhwc_cs(t):
    """(N, H, W, channel stride) of an NHWC view whose pixels are dense apart from the channel stride."""
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError('NHWC view with unit channel step expected')
    N, H, W, _ = t.shape
    cs = t.stride(2)
    if t.stride(1) != W * cs or t.stride(0) != H * W * cs:
        raise ValueError('NHWC view must be dense apart from its channel stride')
    return N, H, W, cs


def conv_fwd(x_nhwc, cin, wpack, cout, out_nhwc, *, stride=1, pad=1, bias=None, act=KAD_ACT_SILU):
    """act(conv3x3(x) + bias) in x's dtype; x and out are NHWC views (channel slices allowed)."""
    _need_gpu(x_nhwc, wpack, out_nhwc, bias)
    N, H, W, cs = _nhwc_cs(x_nhwc)
    No, Ho, Wo, ocs = _nhwc_cs(out_nhwc)
    if (No, Ho, Wo) != (N, (H + 2 * pad - 3) // stride + 1, (W + 2 * pad - 3) // stride + 1) or \
            out_nhwc.shape[3] < cout or x_nhwc.shape[3] < cin:
        raise ValueError('conv_fwd: output shape does not match the convolution')
    if wpack.dtype != x_nhwc.dtype or out_nhwc.dtype != x_nhwc.dtype:
        raise TypeError('x, packed weights and out must share a dtype')
    if bias is not None and bias.dtype != torch.float32:
        raise TypeError('bias must be float32')
    a = DcnArgs()
    a.x, a.wpack, a.bias, a.out = _ptr(x_nhwc), _ptr(wpack), _ptr(bias), _ptr(out_nhwc)
    a.n, a.cin, a.cout, a.h, a.w, a.stride, a.pad = N, cin, cout, H, W, stride, pad
    a.x_cs, a.out_layout, a.out_cs = cs, KAD_NHWC, ocs
    a.dtype = kad_dtype(x_nhwc.dtype)
    a.relu = act
    _check(load().kad_conv_fwd(ctypes.byref(a), _stream()), 'kad_conv_fwd')
    return out_nhwc


def stem_conv_fwd(x_nchw, wpack, cout, out_nhwc, *, stride=2, bias=None, act=KAD_ACT_SILU):
    """act(conv3x3(x) + bias), pad 1, of a contiguous 16-bit NCHW image with 1-3 channels,
    written into the NHWC view out (channel slices allowed)."""
    _need_gpu(x_nchw, wpack, out_nhwc, bias)
    if x_nchw.dim() != 4 or not x_nchw.is_contiguous():
        raise ValueError('stem_conv_fwd: x must be a contiguous NCHW tensor')
    N, C, H, W = x_nchw.shape
    No, Ho, Wo, ocs = _nhwc_cs(out_nhwc)
    if (No, Ho, Wo) != (N, (H - 1) // stride + 1, (W - 1) // stride + 1) or out_nhwc.shape[3] < cout:
        raise ValueError('stem_conv_fwd: output shape does not match the convolution')
    if wpack.dtype != x_nchw.dtype or out_nhwc.dtype != x_nchw.dtype:
        raise TypeError('x, packed weights and out must share a dtype')
    if bias is not None and bias.dtype != torch.float32:
        raise TypeError('bias must be float32')
    a = DcnArgs()
    a.x, a.wpack, a.bias, a.out = _ptr(x_nchw), _ptr(wpack), _ptr(bias), _ptr(out_nhwc)
    a.n, a.cin, a.cout, a.h, a.w, a.stride, a.pad = N, C, cout, H, W, stride, 1
    a.x_cs, a.out_layout, a.out_cs = 0, KAD_NHWC, ocs
    a.dtype = kad_dtype(x_nchw.dtype)
    a.relu = act
    _check(load().kad_stem_conv_fwd(ctypes.byref(a), _stream()), 'kad_stem_conv_fwd')
    return out_nhwc


def nhwc_resample(x_nhwc, out_nhwc, c, mode, k=1, s=1, p=0):
    """Pool (KAD_RS_AVG / KAD_RS_MAX, kernel k, stride s, padding p), nearest upsample
    (KAD_RS_NEAREST, factor s) or copy (AVG with k = s = 1) of channels [0, c); KAD_RS_MAX3:
    three chained max pools (s = 1, p = k // 2) into channels [0, c), [c, 2c), [2c, 3c) of out."""
    _need_gpu(x_nhwc, out_nhwc)
    N, H, W, cs = _nhwc_cs(x_nhwc)
    No, Ho, Wo, ocs = _nhwc_cs(out_nhwc)
    if No != N or out_nhwc.dtype != x_nhwc.dtype:
        raise ValueError('nhwc_resample: batch or dtype mismatch')
    a = ResampleArgs()
    a.x, a.out = _ptr(x_nhwc), _ptr(out_nhwc)
    a.n, a.c, a.h, a.w, a.ho, a.wo, a.x_cs, a.out_cs = N, c, H, W, Ho, Wo, cs, ocs
    a.mode, a.k, a.s, a.p, a.dtype = mode, k, s, p, kad_dtype(x_nhwc.dtype)
    _check(load().kad_nhwc_resample(ctypes.byref(a), _stream()), 'kad_nhwc_resample')
    return out_nhwc


def ddetect_decode(heads, strides, out, nc, reg_max=16, box_ch=None):
    """heads: per level NHWC views [N, h, w, >= box_ch + nc]; out [N, 4 + nc, A] (heads' dtype)."""
    _need_gpu(out, *heads)
    if len(heads) > MAX_LEVELS:
        raise ValueError(f'at most {MAX_LEVELS} levels')
    a = DecodeArgs()
    off = 0
    for l, h in enumerate(heads):
        N, H, W, cs = _nhwc_cs(h)
        if h.dtype != out.dtype:
            raise TypeError('heads and out must share a dtype')
        a.head[l], a.lh[l], a.lw[l], a.head_cs[l] = h.data_ptr(), H, W, cs
        a.anchor_off[l], a.stride[l] = off, float(strides[l])
        off += H * W
    if tuple(out.shape) != (heads[0].shape[0], 4 + nc, off) or not out.is_contiguous():
        raise ValueError(f'out must be contiguous [N, {4 + nc}, {off}]')
    a.out = _ptr(out)
    a.n, a.nl, a.nc, a.reg_max = heads[0].shape[0], len(heads), nc, reg_max
    a.box_ch = 4 * reg_max if box_ch is None else box_ch
    a.dtype = kad_dtype(out.dtype)
    _check(load().kad_ddetect_decode(ctypes.byref(a), _stream()), 'kad_ddetect_decode')
    return out


NMS_MAX = 32768


def nms_keep(boxes_sorted, iou_thr):
    """keep flags (uint8 [n]) of greedy NMS over fp32 xyxy boxes sorted by descending score."""
    _need_gpu(boxes_sorted)
    n = boxes_sorted.shape[0]
    keep = torch.empty(n, dtype=torch.uint8, device=boxes_sorted.device)
    if n == 0:
        return keep
    b = boxes_sorted.to(torch.float32).contiguous()
    mask = torch.empty(load().kad_nms_mask_words(n), dtype=torch.int64, device=b.device)
    _check(load().kad_nms(_ptr(b), _ptr(mask), _ptr(keep), n, float(iou_thr), _stream()), 'kad_nms')
    return keep


def gemm1x1_nhwc(x_nhwc, cin, wpack, cout, out_nhwc, *, bias=None, act=KAD_ACT_NONE):
    """act(W x + b) for NHWC views (channel slices allowed on both sides), act
    KAD_ACT_NONE or KAD_ACT_SILU: the output's channels [cout, roundup(cout, 8))
    inside its stride are zeroed."""
    if act not in (KAD_ACT_NONE, KAD_ACT_SILU):
        raise NotImplementedError('the 1x1 GEMM epilogue has no activation but SiLU')
    _need_gpu(x_nhwc, wpack, out_nhwc, bias)
    N, H, W, cs = _nhwc_cs(x_nhwc)
    No, Ho, Wo, ocs = _nhwc_cs(out_nhwc)
    if (No, Ho, Wo) != (N, H, W) or x_nhwc.shape[3] < cin or out_nhwc.shape[3] < cout:
        raise ValueError('gemm1x1_nhwc: shape mismatch')
    if wpack.dtype != x_nhwc.dtype or out_nhwc.dtype != x_nhwc.dtype:
        raise TypeError('x, packed weights and out must share a dtype')
    a = GemmArgs()
    a.x, a.wpack, a.bias, a.out = _ptr(x_nhwc), _ptr(wpack), _ptr(bias), _ptr(out_nhwc)
    a.n, a.cin, a.cout, a.h, a.w, a.pool = N, cin, cout, H, W, 1
    a.in_layout, a.x_cs, a.out_layout, a.out_cs = KAD_NHWC, cs, KAD_NHWC, ocs
    a.act, a.dtype = (1 if act == KAD_ACT_SILU else 0), kad_dtype(x_nhwc.dtype)   # kad_gemm_args.act: 1 = SiLU
    _check(load().kad_gemm1x1_fwd(ctypes.byref(a), _stream()), 'kad_gemm1x1_fwd')
    return out_nhwc
