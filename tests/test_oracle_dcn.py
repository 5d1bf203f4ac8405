"""Pins the oracle's deformable convolution (oracle/kadconv_oracle.py:deform_conv2d)
against independent formulations and closed-form special cases.

The reference holds no golden vector for this path (no test suite ships with
MLMIP/KAD-Conv); torchvision, which owns the arithmetic, is absent here.  So
the pins are: a float64 brute-force C loop (oracle/dcn_brute.c), an
F.grid_sample formulation, and the conv2d special cases the sampling rule
implies (kadc_dcn_direct.py:57-107)."""
import torch
import torch.nn.functional as F

from oracle import kadconv_oracle as O
from oracle.brute import dcn_brute


def _case(N=2, Ci=3, Co=4, H=6, W=7, scale=2.5, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, Ci, H, W, generator=g, dtype=torch.float64)
    off = torch.randn(N, 18, H, W, generator=g, dtype=torch.float64) * scale
    mask = torch.rand(N, 9, H, W, generator=g, dtype=torch.float64)
    w = torch.randn(Co, Ci, 3, 3, generator=g, dtype=torch.float64)
    b = torch.randn(Co, generator=g, dtype=torch.float64)
    return x, off, mask, w, b


def test_vectorised_matches_bruteforce_c():
    for seed, (H, W) in enumerate([(6, 7), (5, 5), (9, 4), (1, 8)]):
        x, off, mask, w, b = _case(H=H, W=W, seed=seed)
        ref = dcn_brute(x, off, w, b, mask)
        got = O.deform_conv2d(x, off, w, b, mask=mask)
        assert torch.allclose(got, ref, atol=1e-12, rtol=0), (H, W)


def test_bruteforce_stride2_and_no_mask():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 2, 9, 8, generator=g, dtype=torch.float64)
    off = torch.randn(1, 18, 5, 4, generator=g, dtype=torch.float64) * 3
    w = torch.randn(3, 2, 3, 3, generator=g, dtype=torch.float64)
    ref = dcn_brute(x, off, w, None, None, stride=2, padding=1)
    got = O.deform_conv2d(x, off, w, None, stride=2, padding=1)
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)


def test_matches_grid_sample_formulation():
    x, off, mask, w, b = _case(N=2, Ci=5, Co=3, H=11, W=9, scale=4.0, seed=7)
    a = O.deform_conv2d(x, off, w, b, mask=mask)
    c = O.deform_conv2d_gridsample(x, off, w, b, mask=mask)
    assert torch.allclose(a, c, atol=1e-10, rtol=0)


def test_zero_offset_unit_mask_is_conv2d():
    x, off, mask, w, b = _case(Ci=4, Co=5, H=8, W=10)
    got = O.deform_conv2d(x, torch.zeros_like(off), w, b, mask=torch.ones_like(mask))
    ref = F.conv2d(x, w, b, padding=1)
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)


def test_integer_offset_is_shifted_conv2d():
    x, off, mask, w, b = _case(Ci=3, Co=2, H=8, W=9)
    dy, dx = 2, -1
    off = torch.zeros_like(off)
    off[:, 0::2] = dy
    off[:, 1::2] = dx
    got = O.deform_conv2d(x, off, w, b, mask=torch.ones_like(mask))
    H, W = x.shape[2:]
    # padded frame: framed[a + 1, c + 1] = x[a + dy, c + dx] for a in [-1, H], c in [-1, W]
    framed = torch.zeros(x.shape[0], x.shape[1], H + 2, W + 2, dtype=x.dtype)
    for a in range(-1, H + 1):
        for c in range(-1, W + 1):
            if 0 <= a + dy < H and 0 <= c + dx < W:
                framed[:, :, a + 1, c + 1] = x[:, :, a + dy, c + dx]
    ref = F.conv2d(framed, w, b, padding=0)
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)


def test_mask_zero_and_far_out_of_bounds_give_bias():
    x, off, mask, w, b = _case()
    got = O.deform_conv2d(x, off, w, b, mask=torch.zeros_like(mask))
    assert torch.allclose(got, b.view(1, -1, 1, 1).expand_as(got), atol=0, rtol=0)
    far = torch.full_like(off, 1000.0)
    got = O.deform_conv2d(x, far, w, b, mask=mask)
    assert torch.allclose(got, b.view(1, -1, 1, 1).expand_as(got), atol=0, rtol=0)
    # exactly -1 on both axes: every corner is outside or has zero weight
    edge = torch.zeros_like(off)
    edge[:, 0::2] = -1.0 - torch.arange(3, dtype=off.dtype).repeat_interleave(3).view(1, 9, 1, 1)
    got = O.deform_conv2d(x[:, :, :1, :], edge[:, :, :1, :], w, b, mask=mask[:, :, :1, :])
    assert torch.allclose(got, b.view(1, -1, 1, 1).expand_as(got), atol=1e-15, rtol=0)


def test_linear_in_mask_and_input():
    x, off, mask, w, b = _case(seed=5)
    m2 = torch.rand_like(mask)
    lhs = O.deform_conv2d(x, off, w, None, mask=2 * mask - 0.5 * m2)
    rhs = 2 * O.deform_conv2d(x, off, w, None, mask=mask) - 0.5 * O.deform_conv2d(x, off, w, None, mask=m2)
    assert torch.allclose(lhs, rhs, atol=1e-12, rtol=0)
    x2 = torch.randn_like(x)
    lhs = O.deform_conv2d(x + 3 * x2, off, w, None, mask=mask)
    rhs = O.deform_conv2d(x, off, w, None, mask=mask) + 3 * O.deform_conv2d(x2, off, w, None, mask=mask)
    assert torch.allclose(lhs, rhs, atol=1e-12, rtol=0)


def test_offset_layout_dy_before_dx():
    # a pure +0.5 px shift along x on tap 4 (centre) alone, with other taps masked out,
    # must average horizontal neighbours: distinguishes (dy, dx) from (dx, dy)
    x = torch.arange(20, dtype=torch.float64).view(1, 1, 4, 5)
    off = torch.zeros(1, 18, 4, 5, dtype=torch.float64)
    off[:, 2 * 4 + 1] = 0.5
    mask = torch.zeros(1, 9, 4, 5, dtype=torch.float64)
    mask[:, 4] = 1
    w = torch.zeros(1, 1, 3, 3, dtype=torch.float64)
    w[0, 0, 1, 1] = 1
    got = O.deform_conv2d(x, off, w, None, mask=mask)[0, 0]
    exp = x[0, 0].clone()
    exp[:, :4] = 0.5 * (x[0, 0, :, :4] + x[0, 0, :, 1:])
    exp[:, 4] = 0.5 * x[0, 0, :, 4]
    assert torch.allclose(got, exp, atol=1e-12, rtol=0)
