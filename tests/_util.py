"""Shared helpers for the parity tests (tolerances stated in BASELINE.json north_star)."""
import torch

FP32_REL = 1e-4      # fp32: max|d| <= 1e-4 * max|ref|
HALF_ABS = 1e-2      # fp16/bf16: max|d| <= 1e-2 against the fp32 oracle fed the same quantised inputs


def bf16_half_ulp(v):
    """Half a bf16 unit in the last place at |v| (8 significant bits): the rounding
    error of storing v as bf16.  Above |v| = 2 it exceeds 1e-2 by itself
    (|v| in [4, 8): 2^-6 = 1.56e-2), so an absolute 1e-2 bound on a bf16 output
    is only reachable on top of this floor."""
    a = v.abs().clamp_min(2.0 ** -126)
    return torch.ldexp(torch.ones_like(a), torch.floor(torch.log2(a)).to(torch.int32) - 8)


def check_close(got, ref, dtype, what=''):
    """fp32: max|d| <= 1e-4 max|ref|.  fp16: max|d| <= 1e-2.  bf16: |d| <= 1e-2 plus the
    bf16 output-rounding floor at that element (half an ulp of |ref| + 1e-2), which
    the report gives separately as `floor`."""
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert torch.isfinite(got).all(), f'{what}: non-finite output'
    d = (got - ref).abs()
    err = d.max().item()
    scale = ref.abs().max().item()
    if dtype == torch.float32:
        assert err <= FP32_REL * max(scale, 1e-30), f'{what}: max|d|={err:.3e} > 1e-4*{scale:.3e}'
    elif dtype == torch.bfloat16:
        floor = bf16_half_ulp(ref.abs() + HALF_ABS)
        excess = (d - floor).max().item()
        assert excess <= HALF_ABS, (f'{what}: max(|d| - bf16 rounding floor)={excess:.3e} > 1e-2 '
                                    f'(max|d|={err:.3e}, max floor={floor.max().item():.3e}, max|ref|={scale:.3e})')
    else:
        assert err <= HALF_ABS, f'{what}: max|d|={err:.3e} > 1e-2 (max|ref|={scale:.3e})'
    return err, scale


def quant(t, dtype):
    """Round through `dtype` and come back as float64 (the oracle's inputs)."""
    return t.to(dtype).double()


def nhwc_padded(x, mult=8):
    """[N, C, H, W] -> contiguous [N, H, W, roundup(C, mult)] with zero padding."""
    N, C, H, W = x.shape
    cs = (C + mult - 1) // mult * mult
    out = torch.zeros(N, H, W, cs, dtype=x.dtype, device=x.device)
    out[..., :C] = x.permute(0, 2, 3, 1)
    return out
