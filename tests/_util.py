"""Shared helpers for the parity tests (tolerances stated in BASELINE.json north_star)."""
import torch

FP32_REL = 1e-4      # fp32: max|d| <= 1e-4 * max|ref|
HALF_ABS = 1e-2      # fp16/bf16: max|d| <= 1e-2 against the fp32 oracle fed the same quantised inputs


def check_close(got, ref, dtype, what=''):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert torch.isfinite(got).all(), f'{what}: non-finite output'
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    if dtype == torch.float32:
        assert err <= FP32_REL * max(scale, 1e-30), f'{what}: max|d|={err:.3e} > 1e-4*{scale:.3e}'
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
