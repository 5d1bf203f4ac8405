"""The product modules' plain forward on CPU (no GPU, no torchvision):
kadconv.ops.deform_conv2d's CPU restatement and the KADConv / DSC modules built
on it, against the oracle.  KAD-Conv alone on the CPU
plain-PyTorch path, x [1, 64, 80, 80] fp32 ~N(0, 1), every weight
kaiming-uniform from seed 0 (conv_offset and LCSA included, so the offsets are
not all zero).  Tolerance fp32: max|d| <= 1e-4 max|ref| (float64 oracle on the
same inputs); float64 runs agree to 1e-10."""
import pytest
import torch

from kadconv import synthetic as S
from oracle import kadconv_oracle as O
from tests._util import check_close


@pytest.mark.parametrize('stride,pad,dil,k,use_mask', [(1, 1, 1, 3, True), (2, 1, 1, 3, True), (1, 0, 1, 3, False),
                                                       (1, 2, 2, 3, True), (1, 1, 1, 1, True)])
def test_cpu_deform_conv2d_matches_oracle(stride, pad, dil, k, use_mask):
    from kadconv import ops
    g = torch.Generator().manual_seed(stride * 10 + pad + k)
    N, C, H, W, Co = 2, 5, 11, 13, 7
    x = torch.randn(N, C, H, W, generator=g, dtype=torch.float64)
    Ho = (H + 2 * pad - dil * (k - 1) - 1) // stride + 1
    Wo = (W + 2 * pad - dil * (k - 1) - 1) // stride + 1
    off = torch.randn(N, 2 * k * k, Ho, Wo, generator=g, dtype=torch.float64) * 3   # many samples fall outside
    mask = torch.rand(N, k * k, Ho, Wo, generator=g, dtype=torch.float64) if use_mask else None
    w = torch.randn(Co, C, k, k, generator=g, dtype=torch.float64)
    b = torch.randn(Co, generator=g, dtype=torch.float64)
    got = ops.deform_conv2d(x, off, w, b, stride=stride, padding=pad, dilation=dil, mask=mask)
    ref = O.deform_conv2d(x, off, w, b, stride=stride, padding=pad, dilation=dil, mask=mask)
    assert got.shape == ref.shape
    assert torch.allclose(got, ref, atol=1e-10, rtol=0), (got - ref).abs().max()


def test_cpu_deform_conv2d_edges():
    """Samples exactly on the live/dead borders (p = -1, p = H - 1, p just above -1)."""
    from kadconv import ops
    x = torch.randn(1, 2, 4, 5, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    w = torch.randn(3, 2, 3, 3, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    for v in (-1.0, -0.999, 0.0, 2.0, 2.5, 3.0, 3.999, 4.0, -4.0):
        off = torch.full((1, 18, 4, 5), v, dtype=torch.float64)
        got = ops.deform_conv2d(x, off, w, None, padding=1)
        ref = O.deform_conv2d(x, off, w, None, padding=1)
        assert torch.allclose(got, ref, atol=1e-12, rtol=0), v


def test_config1_dsc_cpu_plain():
    import kadconv
    d = kadconv.DSC(64, 64)
    d.load_state_dict(S.make_dsc_state(64, 64, seed=0), strict=False)
    d.eval()
    x = torch.randn(1, 64, 80, 80, generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        got = d(x)
    sd = {k: v.double() for k, v in d.state_dict().items()}
    check_close(got, O.dsc_forward(sd, '', x.double()), torch.float32, 'config 1 DSC')


def test_config1_kadconv_cpu_plain():
    import kadconv
    m = kadconv.KADConv(64)
    m.load_state_dict(S.make_kadconv_state(64, seed=0), strict=False)
    m.eval()
    x = torch.randn(1, 64, 80, 80, generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        got = m(x)
    sd = {k: v.double() for k, v in m.state_dict().items()}
    y0 = torch.nn.functional.conv2d(x.double(), sd['convs.0.0.weight'], sd['convs.0.0.bias'])
    off = torch.nn.functional.conv2d(y0, sd['convs.0.1.conv_offset.weight'], sd['convs.0.1.conv_offset.bias'], padding=1)
    assert off.abs().max() > 0.5   # the offsets are live (kaiming-uniform conv_offset)
    check_close(got, O.kadconv_forward(sd, x.double()), torch.float32, 'config 1 KADConv')
