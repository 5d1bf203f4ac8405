"""Parity of the one-launch DSC core (kad_dsc_fwd: conv_offset computed inside the
tile and consumed by the deformable convolution, kad_conv.py:63-67 minus the
mask branch) and of the plain 3x3 convolution entry (kad_conv3x3_fwd,
kad_conv.py:55-56) against the CPU oracle.

The oracle side computes the offsets with F.conv2d in float64 on the same
quantised input and weights, then O.deform_conv2d (pinned by tests/test_oracle_dcn.py).
Tolerances: fp32 max|d| <= 1e-4 max|ref|; fp16/bf16 max|d| <= 1e-2."""
import pytest
import torch
import torch.nn.functional as F

from oracle import kadconv_oracle as O
from tests._util import check_close, nhwc_padded, quant

pytestmark = pytest.mark.gpu

DT = {'f32': torch.float32, 'f16': torch.float16, 'bf16': torch.bfloat16}


def _inputs(N, C, Co, H, W, seed, off_std=2.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, C, H, W, generator=g)
    # offsets ~N(0, off_std) px on unit-variance input
    ow = torch.randn(18, C, 3, 3, generator=g) * (off_std / (9 * C) ** 0.5)
    ob = torch.randn(18, generator=g) * 0.3
    bound = 1 / (9 * C) ** 0.5
    w = (torch.rand(Co, C, 3, 3, generator=g) * 2 - 1) * bound
    b = (torch.rand(Co, generator=g) * 2 - 1) * bound
    return x, ow, ob, w, b


def _mask(N, Ho, Wo, seed):
    g = torch.Generator().manual_seed(seed + 1000)
    return torch.sigmoid(torch.randn(N, 9, Ho, Wo, generator=g))


def _ref(x, ow, ob, w, b, mask, dtype, stride=1):
    xq = quant(x, dtype)
    off = F.conv2d(xq, quant(ow, dtype), ob.double(), stride=stride, padding=1)
    return O.deform_conv2d(xq, off, quant(w, dtype), b.double(), stride=stride, padding=1,
                           mask=None if mask is None else mask.double())


def _run_dsc(x, ow, ob, w, b, mask, dtype, stride=1, out_layout='nchw', epi=None, gap=None):
    from kadconv import _ext
    dev = 'cuda'
    N, C, H, W = x.shape
    Co = w.shape[0]
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    xq = nhwc_padded(x.to(dtype).to(dev))
    md = None if mask is None else mask.permute(0, 2, 3, 1).contiguous().to(dev)
    wp = _ext.dcn_pack_weights(w.to(dtype).to(dev), dtype)
    owp = _ext.dcn_pack_weights(ow.to(dtype).to(dev), dtype)
    kw = {}
    if epi is not None:
        kw = {k: v.to(dev) for k, v in epi.items() if k != 'relu'}
        kw['relu'] = epi.get('relu', False)
    if out_layout == 'nchw':
        out = torch.empty(N, Co, Ho, Wo, dtype=dtype, device=dev)
        _ext.dsc_fwd(xq, C, owp, ob.to(dev), md, (Ho * Wo * 9, 9, 1), wp, Co, out, stride=stride, bias=b.to(dev),
                     out_layout=_ext.KAD_NCHW, gap_partial=gap, **kw)
        return out
    cs = (Co + 7) // 8 * 8
    out = torch.full((N, Ho, Wo, cs), 7.0, dtype=dtype, device=dev)
    _ext.dsc_fwd(xq, C, owp, ob.to(dev), md, (Ho * Wo * 9, 9, 1), wp, Co, out, stride=stride, bias=b.to(dev),
                 out_layout=_ext.KAD_NHWC, gap_partial=gap, **kw)
    if cs > Co:  # channels past Cout belong to the caller: untouched
        assert (out[..., Co:] == 7.0).all()
    return out[..., :Co].permute(0, 3, 1, 2)


@pytest.mark.parametrize('dt', ['f32', 'f16', 'bf16'])
@pytest.mark.parametrize('shape', [(2, 8, 8, 9, 11), (1, 22, 22, 20, 20), (2, 86, 86, 17, 23), (1, 40, 72, 13, 7),
                                   (1, 33, 130, 12, 70), (2, 3, 16, 11, 9), (1, 16, 24, 3, 190), (1, 96, 96, 5, 6)])
def test_dsc_small(dt, shape):
    N, C, Co, H, W = shape
    dtype = DT[dt]
    x, ow, ob, w, b = _inputs(N, C, Co, H, W, seed=sum(shape))
    mask = _mask(N, H, W, seed=sum(shape))
    print(f'dsc_small dt={dt} shape={shape}', flush=True)
    got = _run_dsc(x, ow, ob, w, b, mask, dtype)
    torch.cuda.synchronize()
    check_close(got, _ref(x, ow, ob, w, b, mask, dtype), dtype, f'{dt} {shape}')


@pytest.mark.parametrize('dt', ['f16', 'bf16', 'f32'])
@pytest.mark.parametrize('off_std', [0.6, 4.0])
def test_dsc_branch0_shape(dt, off_std):
    """KADConv(256) branch 0 at the metric's spatial size (c = 86, 100 x 100),
    NHWC out with a padded channel stride; off_std 4 px forces capped regions
    and the global-memory sample pass."""
    dtype = DT[dt]
    x, ow, ob, w, b = _inputs(2, 86, 86, 100, 100, seed=86, off_std=off_std)
    mask = _mask(2, 100, 100, seed=86)
    print(f'dsc_branch0 dt={dt} off_std={off_std}', flush=True)
    got = _run_dsc(x, ow, ob, w, b, mask, dtype, out_layout='nhwc')
    torch.cuda.synchronize()
    check_close(got, _ref(x, ow, ob, w, b, mask, dtype), dtype, f'{dt} off_std={off_std}')


@pytest.mark.parametrize('dt', ['f16', 'bf16'])
@pytest.mark.parametrize('shape,off_std,layout', [((8, 10, 12, 100, 100), 2.0, 'nhwc'), ((12, 16, 16, 64, 64), 4.0, 'nchw'),
                                                  ((8, 22, 44, 80, 80), 2.0, 'nchw'), ((12, 3, 64, 60, 70), 1.0, 'nhwc'),
                                                  ((6, 40, 33, 90, 90), 12.0, 'nhwc')])
def test_dsc_two_blocks_per_cu(dt, shape, off_std, layout):
    """16-bit, stride 1, Cout <= 64 and >= 384 tile blocks: the launch runs on the
    two-blocks-per-CU kernel.  Cin 3 / 10 / 22 / 40 (one half-chunk partly
    padded, two, three), Cout not a multiple of 16, NCHW and NHWC outputs,
    offsets up to 12 px (capped regions: samples from global memory)."""
    from kadconv import _ext
    N, C, Co, H, W = shape
    assert N * _ext.dcn_tiles(H, W) >= 384
    dtype = DT[dt]
    x, ow, ob, w, b = _inputs(N, C, Co, H, W, seed=C * 3 + Co, off_std=off_std)
    mask = _mask(N, H, W, seed=C)
    print(f'dsc_two_per_cu dt={dt} shape={shape} off_std={off_std}', flush=True)
    got = _run_dsc(x, ow, ob, w, b, mask, dtype, out_layout=layout)
    torch.cuda.synchronize()
    check_close(got, _ref(x, ow, ob, w, b, mask, dtype), dtype, f'{dt} {shape} off_std={off_std}')


# KAD-CNet-S at 800 x 800: the DSC(c, c) shapes of its 42 KADC4 layers,
# c in {12, 10, 10} at {100, 50, 25}^2, {16, 16, 16} at {50, 25, 12}^2, {22, 21, 21} at {25, 12, 6}^2
KADCNET_DSC = [(12, 100), (10, 50), (10, 25), (16, 50), (16, 25), (16, 12), (22, 25), (21, 12), (21, 6)]


@pytest.mark.parametrize('dt', ['f16', 'f32'])
@pytest.mark.parametrize('C,H', KADCNET_DSC)
def test_dsc_kadcnet_shapes(dt, C, H):
    """Every small-channel DSC shape of KAD-CNet-S, batch 16, channels-last output (the
    network's layout), offsets ~N(0, 2) px: the fp16 launches with >= 384 tile blocks run on
    the two-blocks-per-CU kernel, the others on the general one."""
    dtype = DT[dt]
    x, ow, ob, w, b = _inputs(16, C, C, H, H, seed=C * 7 + H)
    mask = _mask(16, H, H, seed=C + H)
    print(f'dsc_kadcnet dt={dt} C={C} H={H}', flush=True)
    got = _run_dsc(x, ow, ob, w, b, mask, dtype, out_layout='nhwc')
    torch.cuda.synchronize()
    check_close(got, _ref(x, ow, ob, w, b, mask, dtype), dtype, f'{dt} C={C} H={H}')


@pytest.mark.parametrize('dt', ['f16', 'bf16'])
def test_dsc_two_blocks_per_cu_gap(dt):
    """GAP partials of the two-blocks-per-CU kernel: fp32 sums of the rounded outputs."""
    from kadconv import _ext
    N, C, Co, H, W = 8, 16, 20, 100, 100
    assert N * _ext.dcn_tiles(H, W) >= 384
    x, ow, ob, w, b = _inputs(N, C, Co, H, W, seed=5)
    mask = _mask(N, H, W, seed=5)
    gap = torch.full((N, _ext.dcn_tiles(H, W), Co), float('nan'), device='cuda')
    out = _run_dsc(x, ow, ob, w, b, mask, DT[dt], out_layout='nhwc', gap=gap)
    torch.cuda.synchronize()
    got = gap.sum(1).cpu().double() / (H * W)
    ref = out.double().mean(dim=(2, 3)).cpu()
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize('dt', ['f32', 'f16'])
def test_dsc_stride2_epilogue_nomask(dt):
    dtype = DT[dt]
    x, ow, ob, w, b = _inputs(2, 24, 40, 15, 12, seed=11)
    g = torch.Generator().manual_seed(5)
    epi = {'post_mul': torch.rand(40, generator=g) + 0.5, 'post_add': torch.randn(40, generator=g) * 0.1,
           'post_scale': torch.randn(40, generator=g), 'relu': True}
    print(f'dsc_stride2 dt={dt}', flush=True)
    got = _run_dsc(x, ow, ob, w, b, None, dtype, stride=2, epi=epi)
    torch.cuda.synchronize()
    ref = _ref(x, ow, ob, w, b, None, dtype, stride=2)
    ref = torch.relu(ref * epi['post_mul'].double().view(1, -1, 1, 1) + epi['post_add'].double().view(1, -1, 1, 1))
    ref = ref * epi['post_scale'].double().view(1, -1, 1, 1)
    check_close(got, ref, dtype, f'stride2 {dt}')


@pytest.mark.parametrize('dt', ['f32', 'f16'])
def test_dsc_gap_partials_sum_to_mean(dt):
    """The per-tile GAP partials are fp32 sums of the rounded outputs."""
    from kadconv import _ext
    x, ow, ob, w, b = _inputs(2, 16, 20, 30, 30, seed=3)
    mask = _mask(2, 30, 30, seed=3)
    gap = torch.full((2, _ext.dcn_tiles(30, 30), 20), float('nan'), device='cuda')
    out = _run_dsc(x, ow, ob, w, b, mask, DT[dt], out_layout='nhwc', gap=gap)
    torch.cuda.synchronize()
    got = gap.sum(1).cpu().double() / 900
    ref = out.double().mean(dim=(2, 3)).cpu()
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize('dt', ['f16', 'bf16'])
def test_dsc_far_offsets(dt):
    """Offsets of ~20 px: most samples fall outside any region that fits the
    LDS budget (capped or 1 x 1 regions), so the pass from global memory
    carries them; many are dead (outside the image)."""
    dtype = DT[dt]
    x, ow, ob, w, b = _inputs(2, 40, 48, 37, 41, seed=20, off_std=20.0)
    mask = _mask(2, 37, 41, seed=20)
    print(f'dsc_far_offsets dt={dt}', flush=True)
    got = _run_dsc(x, ow, ob, w, b, mask, dtype, out_layout='nhwc')
    torch.cuda.synchronize()
    check_close(got, _ref(x, ow, ob, w, b, mask, dtype), dtype, f'far offsets {dt}')


@pytest.mark.parametrize('dt', ['f32', 'f16', 'bf16'])
@pytest.mark.parametrize('shape,stride', [((2, 86, 18, 100, 100), 1), ((1, 40, 130, 13, 7), 1),
                                          ((2, 24, 18, 15, 12), 2), ((1, 8, 3, 5, 64), 2),
                                          ((1, 130, 18, 9, 200), 1), ((3, 8, 18, 25, 25), 1),
                                          ((1, 3, 18, 6, 6), 1), ((2, 256, 18, 50, 50), 1)])
def test_conv3x3(dt, shape, stride):
    """kad_conv3x3_fwd (fp32 output, NHWC and NCHW) against F.conv2d in float64."""
    from kadconv import _ext
    dtype = DT[dt]
    N, C, Co, H, W = shape
    g = torch.Generator().manual_seed(C + Co)
    x = torch.randn(N, C, H, W, generator=g)
    w = torch.randn(Co, C, 3, 3, generator=g) / (9 * C) ** 0.5
    b = torch.randn(Co, generator=g)
    ref = F.conv2d(quant(x, dtype), quant(w, dtype), b.double(), stride=stride, padding=1)
    Ho, Wo = ref.shape[2:]
    dev = 'cuda'
    xq = nhwc_padded(x.to(dtype).to(dev))
    wp = _ext.dcn_pack_weights(w.to(dtype).to(dev), dtype)
    print(f'conv3x3 dt={dt} shape={shape} stride={stride}', flush=True)
    out = torch.empty(N, Ho, Wo, Co, dtype=torch.float32, device=dev)
    _ext.conv3x3_fwd(xq, C, wp, Co, out, stride=stride, bias=b.to(dev))
    out2 = torch.empty(N, Co, Ho, Wo, dtype=torch.float32, device=dev)
    _ext.conv3x3_fwd(xq, C, wp, Co, out2, stride=stride, bias=b.to(dev), out_layout=_ext.KAD_NCHW)
    torch.cuda.synchronize()
    # fp32 accumulation of fp16/bf16 products: fp32 bar for every dtype
    check_close(out.permute(0, 3, 1, 2), ref, torch.float32, f'conv3x3 nhwc {dt} {shape}')
    check_close(out2, ref, torch.float32, f'conv3x3 nchw {dt} {shape}')


def test_dsc_rejects_stride3():
    from kadconv import _ext
    x = torch.zeros(1, 64, 64, 8, dtype=torch.float16, device='cuda')
    wp = torch.zeros(_ext.dcn_wpack_elems(8, 8), dtype=torch.float16, device='cuda')
    owp = torch.zeros(_ext.dcn_wpack_elems(8, 18), dtype=torch.float16, device='cuda')
    out = torch.empty(1, 22, 22, 8, dtype=torch.float16, device='cuda')
    with pytest.raises(RuntimeError, match='stride 3'):
        _ext.dsc_fwd(x, 8, owp, None, None, (0, 0, 0), wp, 8, out, stride=3)


@pytest.mark.parametrize('dt', ['f32', 'f16', 'bf16'])
@pytest.mark.parametrize('C,Co,hid,H,W', [(86, 86, 86, 23, 31), (24, 130, 16, 17, 40), (40, 40, 32, 9, 9),
                                           (16, 16, 16, 128, 128)])
def test_dsc_fused_squeeze_excitation(dt, C, Co, hid, H, W):
    """kad_dsc_fwd with the SE fields set: the last block of each image turns the
    GAP partials into att = sigmoid(W2 relu(W1 mean(out) + b1) + b2)
    (KADConv.forward, kad_conv.py:125).  Reference: that MLP in float64 over the
    kernel's own output (so only the reduction and the MLP are under test).
    Several calls in a row with changing batch sizes share one counter buffer,
    which every completed call must leave at zero; Co = 130 spans two column
    blocks, whose partials the last block must both see; at 16 channels and
    128 x 128 the 16-bit calls with N >= 3 run on the two-blocks-per-CU kernel
    and the others on the 8-wave one, on the same counters.  att tolerance: 2e-5
    absolute (fp32 sums of at most H*W values, sigmoid slope <= 1/4)."""
    from kadconv import _ext
    dtype, dev = DT[dt], 'cuda'
    g = torch.Generator().manual_seed(C * 7 + Co)
    w1 = (torch.randn(hid, Co, generator=g) / Co ** 0.5).to(dev)
    b1 = (torch.randn(hid, generator=g) * 0.1).to(dev)
    w2 = (torch.randn(Co, hid, generator=g) / hid ** 0.5).to(dev)
    b2 = (torch.randn(Co, generator=g) * 0.1).to(dev)
    count = torch.zeros(4, dtype=torch.int32, device=dev)
    for call, N in enumerate([3, 1, 4, 2]):
        x, ow, ob, w, b = _inputs(N, C, Co, H, W, seed=call + 11)
        mask = _mask(N, H, W, seed=call)
        xq = nhwc_padded(x.to(dtype).to(dev))
        md = mask.permute(0, 2, 3, 1).contiguous().to(dev)
        wp = _ext.dcn_pack_weights(w.to(dtype).to(dev), dtype)
        owp = _ext.dcn_pack_weights(ow.to(dtype).to(dev), dtype)
        out = torch.empty(N, Co, H, W, dtype=dtype, device=dev)
        gap = torch.full((N, _ext.dcn_tiles(H, W), Co), float('nan'), device=dev)
        att = torch.full((N, Co), float('nan'), device=dev)
        print(f'fused SE {dt} C={C} Co={Co} hid={hid} {H}x{W} call {call} N={N}', flush=True)
        _ext.dsc_fwd(xq, C, owp, ob.to(dev), md, (H * W * 9, 9, 1), wp, Co, out, bias=b.to(dev),
                     out_layout=_ext.KAD_NCHW, gap_partial=gap, se=(w1, b1, w2, b2, att, count))
        torch.cuda.synchronize()
        assert int(count.abs().sum().item()) == 0, 'arrival counters not reset'
        m = out.double().mean(dim=(2, 3))
        h = torch.relu(m @ w1.double().t() + b1.double())
        ref = torch.sigmoid(h @ w2.double().t() + b2.double())
        err = (att.double() - ref).abs().max().item()
        assert err <= 2e-5, f'call {call}: att max|d| = {err:.3e}'
        check_close(out, _ref(x, ow, ob, w, b, mask, dtype), dtype, 'output')
