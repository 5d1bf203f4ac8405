"""Parity of the HIP deformable-convolution core (kad_dcn_fwd) against the
oracle's restatement of torchvision.ops.deform_conv2d (kad_conv.py:66-67)."""
import pytest
import torch

from oracle import kadconv_oracle as O
from tests._util import check_close, nhwc_padded, quant

pytestmark = pytest.mark.gpu

DT = {'f32': torch.float32, 'f16': torch.float16, 'bf16': torch.bfloat16}


def _inputs(N, C, Co, H, W, seed, off_std=2.0, stride=1):
    g = torch.Generator().manual_seed(seed)
    Ho = (H + 2 - 3) // stride + 1
    Wo = (W + 2 - 3) // stride + 1
    x = torch.randn(N, C, H, W, generator=g)
    off = torch.randn(N, 18, Ho, Wo, generator=g) * off_std
    mask = torch.sigmoid(torch.randn(N, 9, Ho, Wo, generator=g))
    bound = 1 / (9 * C) ** 0.5
    w = (torch.rand(Co, C, 3, 3, generator=g) * 2 - 1) * bound
    b = (torch.rand(Co, generator=g) * 2 - 1) * bound
    return x, off, mask, w, b


def _run(x, off, mask, w, b, dtype, stride=1, pixel_major=True, out_layout='nchw', epi=None):
    from kadconv import _ext
    dev = 'cuda'
    N, C, H, W = x.shape
    Co = w.shape[0]
    Ho, Wo = off.shape[2:]
    xq = nhwc_padded(x.to(dtype).to(dev))
    if pixel_major:
        offd = off.permute(0, 2, 3, 1).contiguous().to(dev)
        md = mask.permute(0, 2, 3, 1).contiguous().to(dev)
        os_, ms = (Ho * Wo * 18, 18, 1), (Ho * Wo * 9, 9, 1)
    else:
        offd = off.contiguous().to(dev)
        md = mask.contiguous().to(dev)
        os_, ms = (18 * Ho * Wo, 1, Ho * Wo), (9 * Ho * Wo, 1, Ho * Wo)
    wp = _ext.dcn_pack_weights(w.to(dtype).to(dev), dtype)
    kw = {}
    if epi is not None:
        kw = {k: v.to(dev) for k, v in epi.items() if k != 'relu'}
        kw['relu'] = epi.get('relu', False)
    if out_layout == 'nchw':
        out = torch.empty(N, Co, Ho, Wo, dtype=dtype, device=dev)
        _ext.dcn_fwd(xq, C, offd, os_, md, ms, wp, Co, out, stride=stride, bias=b.to(dev),
                     out_layout=_ext.KAD_NCHW, **kw)
        return out
    out = torch.empty(N, Ho, Wo, Co, dtype=dtype, device=dev)
    _ext.dcn_fwd(xq, C, offd, os_, md, ms, wp, Co, out, stride=stride, bias=b.to(dev),
                 out_layout=_ext.KAD_NHWC, **kw)
    return out.permute(0, 3, 1, 2)


def _ref(x, off, mask, w, b, dtype, stride=1):
    return O.deform_conv2d(quant(x, dtype), off.double(), quant(w, dtype), b.double(), stride=stride,
                           padding=1, mask=mask.double())


@pytest.mark.parametrize('dt', ['f32', 'f16', 'bf16'])
@pytest.mark.parametrize('shape', [(2, 8, 8, 9, 11), (1, 22, 22, 20, 20), (2, 86, 86, 17, 23), (1, 40, 72, 13, 7)])
def test_dcn_small(dt, shape):
    N, C, Co, H, W = shape
    dtype = DT[dt]
    x, off, mask, w, b = _inputs(N, C, Co, H, W, seed=hash(shape) % 1000)
    print(f'dcn_small dt={dt} shape={shape}', flush=True)
    got = _run(x, off, mask, w, b, dtype)
    torch.cuda.synchronize()
    check_close(got, _ref(x, off, mask, w, b, dtype), dtype, f'{dt} {shape}')


@pytest.mark.parametrize('dt', ['f16', 'bf16'])
@pytest.mark.parametrize('shape,pixel_major', [((8, 12, 16, 100, 100), True), ((12, 20, 44, 64, 64), False)])
def test_dcn_two_blocks_per_cu(dt, shape, pixel_major):
    """16-bit, stride 1, Cout <= 64 and >= 384 tile blocks: the launch runs on the
    two-blocks-per-CU kernel (16-channel half-chunks, records in registers)."""
    from kadconv import _ext
    N, C, Co, H, W = shape
    assert N * _ext.dcn_tiles(H, W) >= 384
    dtype = DT[dt]
    x, off, mask, w, b = _inputs(N, C, Co, H, W, seed=C + Co)
    print(f'dcn_two_per_cu dt={dt} shape={shape}', flush=True)
    got = _run(x, off, mask, w, b, dtype, pixel_major=pixel_major, out_layout='nhwc' if pixel_major else 'nchw')
    torch.cuda.synchronize()
    check_close(got, _ref(x, off, mask, w, b, dtype), dtype, f'{dt} {shape}')


@pytest.mark.parametrize('dt', ['f16', 'f32', 'bf16'])
@pytest.mark.parametrize('C,H', [(128, 100), (256, 50), (512, 25)])
def test_dcn_config2_shapes(dt, C, H):
    """BASELINE config 2 scales, batch 8, offsets ~N(0, 2) px (with out-of-bounds samples)."""
    dtype = DT[dt]
    x, off, mask, w, b = _inputs(8, C, C, H, H, seed=C)
    print(f'dcn_config2 dt={dt} C={C} H={H}', flush=True)
    got = _run(x, off, mask, w, b, dtype, out_layout='nhwc')
    torch.cuda.synchronize()
    check_close(got, _ref(x, off, mask, w, b, dtype), dtype, f'{dt} C={C} H={H}')


@pytest.mark.parametrize('dt', ['f32', 'f16'])
def test_dcn_plane_major_offsets_stride2_epilogue(dt):
    dtype = DT[dt]
    x, off, mask, w, b = _inputs(2, 24, 40, 15, 12, seed=11, stride=2)
    g = torch.Generator().manual_seed(5)
    epi = {'post_mul': torch.rand(40, generator=g) + 0.5, 'post_add': torch.randn(40, generator=g) * 0.1,
           'post_scale': torch.randn(40, generator=g), 'relu': True}
    print(f'dcn_stride2 dt={dt}', flush=True)
    got = _run(x, off, mask, w, b, dtype, stride=2, pixel_major=False, epi=epi)
    torch.cuda.synchronize()
    ref = _ref(x, off, mask, w, b, dtype, stride=2)
    ref = torch.relu(ref * epi['post_mul'].double().view(1, -1, 1, 1) + epi['post_add'].double().view(1, -1, 1, 1))
    ref = ref * epi['post_scale'].double().view(1, -1, 1, 1)
    check_close(got, ref, dtype, f'stride2 {dt}')


def test_dcn_gap_partials_sum_to_mean():
    from kadconv import _ext
    dtype = torch.float32
    x, off, mask, w, b = _inputs(2, 16, 20, 30, 30, seed=3)
    dev = 'cuda'
    xq = nhwc_padded(x.to(dev))
    offd = off.permute(0, 2, 3, 1).contiguous().to(dev)
    md = mask.permute(0, 2, 3, 1).contiguous().to(dev)
    wp = _ext.dcn_pack_weights(w.to(dev), dtype)
    tiles = _ext.dcn_tiles(30, 30)
    gap = torch.full((2, tiles, 20), float('nan'), device=dev)
    out = torch.empty(2, 30, 30, 20, device=dev)
    _ext.dcn_fwd(xq, 16, offd, (900 * 18, 18, 1), md, (900 * 9, 9, 1), wp, 20, out, bias=b.to(dev),
                 gap_partial=gap)
    torch.cuda.synchronize()
    got = gap.sum(1).cpu().double() / 900
    ref = out.double().mean(dim=(1, 2)).cpu()
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5)


def test_dcn_offsets_far_out_give_bias():
    dtype = torch.float16
    x, off, mask, w, b = _inputs(1, 16, 16, 9, 9, seed=4)
    off = torch.full_like(off, 50.0)
    got = _run(x, off, mask, w, b, dtype)
    torch.cuda.synchronize()
    exp = b.to(dtype).double().view(1, -1, 1, 1).expand(1, 16, 9, 9)
    assert torch.allclose(got.double().cpu(), exp, atol=1e-3)
