"""The LCSA mask kernels (kad_axial_sums / kad_lcsa_prep / kad_lcsa_mask and the
split variant) compared directly with sigmoid(oracle.lcsa_forward), i.e. the
modulation mask of DSC.forward (KAD-Conv/kadconv/kad_conv.py:38-39,65), not
through a DSC output where the DCN weights would damp a mask error.

Shapes: BASELINE config 2's three DSC scales and the metric KADConv's three
branch maps.  LCSA BatchNorm statistics are drawn far from identity (running
mean in [-1, 1], variance in [0.3, 3], gamma in [0.5, 1.5], beta in [-0.5, 0.5])
so that the folded BN is exercised.  The input is the dtype-rounded map; the
oracle runs in float64 on it.

Tolerance on the mask (values in (0, 1)): fp32 1e-5; fp16/bf16 2e-3.  The
16-bit runs contract in fp16 (the E = w4 w3 matrix and the strip activation u
are fp16 MFMA operands, accumulated in fp32), so their error is a few fp16
ulps of the logits times sigmoid's slope <= 1/4."""
import pytest
import torch

from kadconv import synthetic as S
from oracle import kadconv_oracle as O

pytestmark = pytest.mark.gpu

DT = {'f32': torch.float32, 'f16': torch.float16, 'bf16': torch.bfloat16}
TOL = {'f32': 1e-5, 'f16': 2e-3, 'bf16': 1e-5}  # bf16 runs form the mask GEMM in fp32 (fused._emat_dtype)


def _wide_bn(sd, c, seed):
    g = torch.Generator().manual_seed(seed)
    r = 'RCA_mask.excite.1.'
    sd[r + 'running_mean'] = torch.rand(c, generator=g) * 2 - 1
    sd[r + 'running_var'] = torch.rand(c, generator=g) * 2.7 + 0.3
    sd[r + 'weight'] = torch.rand(c, generator=g) + 0.5
    sd[r + 'bias'] = torch.rand(c, generator=g) - 0.5
    return sd


@pytest.mark.parametrize('dt', ['f32', 'f16', 'bf16'])
@pytest.mark.parametrize('n,c,h,w,split', [
    (8, 128, 100, 100, True), (8, 256, 50, 50, True), (8, 512, 25, 25, True),   # config 2 (standalone DSC plan)
    (8, 86, 100, 100, False), (8, 85, 50, 50, False), (8, 85, 25, 25, False),   # metric KADConv branches
])
def test_lcsa_mask_matches_oracle(dt, n, c, h, w, split):
    import kadconv
    from kadconv import _ext
    from kadconv.fused import DSCPlan
    dtype, dev = DT[dt], 'cuda'
    print(f'lcsa mask {dt} n={n} c={c} {h}x{w} split={split}', flush=True)
    d = kadconv.DSC(c, c)
    d.load_state_dict(_wide_bn(S.make_dsc_state(c, c, seed=c + h), c, seed=c), strict=False)
    d = d.to(dev, dtype).eval()
    plan = DSCPlan(d)
    _, _, emat, ebias = plan.packed(dtype)
    x = torch.randn(n, c, h, w, generator=torch.Generator().manual_seed(h * 7 + c)).to(dtype)
    cs = (c + 7) // 8 * 8
    y = torch.zeros(n, h, w, cs, dtype=dtype)
    y[..., :c] = x.permute(0, 2, 3, 1)
    y = y.to(dev)
    rows = torch.empty(n, h, c, device=dev)
    cols = torch.empty(n, w, c, device=dev)
    arow = torch.empty(n, h, c, device=dev)
    colm = torch.empty(n, w, c, device=dev)
    mask = torch.full((n, h, w, 9), float('nan'), device=dev)
    ks = _ext.lcsa_mask_splits(n, c, h, w) if split else 1
    work = torch.empty(_ext.lcsa_mask_work_elems(n, h, w, ks), device=dev) if ks > 1 else None
    _ext.axial_sums(y, c, rows, cols)
    _ext.lcsa_prep(rows, 1, cols, 1, arow, colm, n, c, h, w)
    _ext.lcsa_mask(arow, colm, plan.lcsa, emat, ebias, mask, n, c, h, w, ks, work)
    torch.cuda.synchronize()
    sd = {k: v.detach().double().cpu() for k, v in d.state_dict().items()}
    ref = torch.sigmoid(O.lcsa_forward(sd, 'RCA_mask.', x.double())).permute(0, 2, 3, 1)
    got = mask.cpu().double()
    assert torch.isfinite(got).all()
    err = (got - ref).abs().max().item()
    print(f'  max|d| = {err:.3e} (ksplit={ks})', flush=True)
    assert err <= TOL[dt], f'mask max|d| = {err:.3e} > {TOL[dt]}'


def test_lcsa_mask_bf16_beyond_fp16_range():
    """A bf16 map whose axial means exceed fp16's 65504: the mask GEMM of a bf16 run is fp32, so
    the mask stays finite (an fp16 strip activation would be inf and the mask NaN) and matches
    the oracle.  Tolerance 2e-3: most logits are saturated, and the fp32 sums of terms of
    ~1e5 leave ~1e-3 on the few logits near 0 (sigmoid slope <= 1/4)."""
    import kadconv
    from kadconv import _ext
    from kadconv.fused import DSCPlan
    dtype, dev = torch.bfloat16, 'cuda'
    n, c, h, w = 2, 86, 30, 30
    d = kadconv.DSC(c, c)
    d.load_state_dict(_wide_bn(S.make_dsc_state(c, c, seed=5), c, seed=6), strict=False)
    d = d.to(dev, dtype).eval()
    plan = DSCPlan(d)
    _, _, emat, ebias = plan.packed(dtype)
    assert emat.dtype == torch.float32
    x = (torch.randn(n, c, h, w, generator=torch.Generator().manual_seed(7)) * 1e5).to(dtype)
    y = torch.zeros(n, h, w, 88, dtype=dtype)
    y[..., :c] = x.permute(0, 2, 3, 1)
    y = y.to(dev)
    arow = torch.empty(n, h, c, device=dev)
    colm = torch.empty(n, w, c, device=dev)
    mask = torch.full((n, h, w, 9), float('nan'), device=dev)
    _ext.axial_means(y, c, arow, colm)
    _ext.lcsa_mask(arow, colm, plan.lcsa, emat, ebias, mask, n, c, h, w, 1, None)
    torch.cuda.synchronize()
    sd = {k: v.detach().double().cpu() for k, v in d.state_dict().items()}
    ref = torch.sigmoid(O.lcsa_forward(sd, 'RCA_mask.', x.double())).permute(0, 2, 3, 1)
    got = mask.cpu().double()
    assert x.double().mean(3).abs().max().item() > 65504
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max().item() <= 2e-3
