"""ctypes loader for oracle/dcn_brute.c (float64 brute-force DCNv2).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py)."""
import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, '_build', 'liboracle_dcn.so')
_lib = None


def build():
    subprocess.run(['make', '-s', '-C', _HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        _lib = ctypes.CDLL(_LIB)
        _lib.oracle_dcn_brute_f64.restype = ctypes.c_int
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def dcn_brute(x, offset, weight, bias=None, mask=None, stride=1, padding=1, dilation=1):
    """float64 brute force; accepts torch tensors, returns a float64 torch tensor."""
    lib = _load()
    xs = np.ascontiguousarray(x.detach().double().numpy())
    off = np.ascontiguousarray(offset.detach().double().numpy())
    w = np.ascontiguousarray(weight.detach().double().numpy())
    b = None if bias is None else np.ascontiguousarray(bias.detach().double().numpy())
    m = None if mask is None else np.ascontiguousarray(mask.detach().double().numpy())
    N, Ci, H, W = xs.shape
    Co, _, KH, KW = w.shape
    Ho = (H + 2 * padding - dilation * (KH - 1) - 1) // stride + 1
    Wo = (W + 2 * padding - dilation * (KW - 1) - 1) // stride + 1
    out = np.zeros((N, Co, Ho, Wo), dtype=np.float64)
    rc = lib.oracle_dcn_brute_f64(_ptr(xs), _ptr(off), _ptr(m), _ptr(w), _ptr(b), _ptr(out),
                                  N, Ci, H, W, Co, KH, KW, stride, padding, dilation)
    if rc != 0:
        raise ValueError('dcn_brute: empty output')
    return torch.from_numpy(out)
