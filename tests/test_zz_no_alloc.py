"""kad_dsc_fwd_noalloc (the fused DSC + squeeze-excitation forward whose GAP
partials and arrival counters live in the library's own device scratch)
against kad_dsc_fwd with caller-owned partials and counters, through the
C-ABI: two calls in a row on the same inputs' shapes, the second with a
smaller batch and image, each compared bit for bit (same kernel, same fixed
reduction order), plus the size-limit error."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(n, c, h, w, dtype, seed):
    import kadconv
    from kadconv import _ext
    from kadconv.fused import DSCPlan
    from kadconv import synthetic as S
    dev = 'cuda'
    g = torch.Generator().manual_seed(seed)
    d = kadconv.DSC(c, c)
    d.load_state_dict(S.make_dsc_state(c, c, seed=seed, offset_std_px=2.0), strict=False)
    d = d.to(dev).eval()
    plan = DSCPlan(d)
    wp, owp, _, _ = plan.packed(dtype)
    cs = (c + 7) // 8 * 8
    y = torch.zeros(n, h, w, cs)
    y[..., :c] = torch.randn(n, h, w, c, generator=g)
    y = y.to(dev, dtype)
    mask = torch.rand(n, h, w, 9, generator=g).to(dev)
    hid = max(32, c)
    se_w = [(torch.randn(hid, c, generator=g) * 0.2).to(dev), (torch.randn(hid, generator=g) * 0.1).to(dev),
            (torch.randn(c, hid, generator=g) * 0.2).to(dev), (torch.randn(c, generator=g) * 0.1).to(dev)]
    post = [(torch.rand(c, generator=g) + 0.5).to(dev), (torch.randn(c, generator=g) * 0.1).to(dev),
            (torch.rand(c, generator=g) + 0.5).to(dev)]
    P = h * w
    args = dict(bias=plan.bias, post_mul=post[0], post_add=post[1], post_scale=post[2], relu=True)

    # kad_dsc_fwd with caller-owned GAP partials and counters
    out_ref = torch.full((n, h, w, cs), float('nan'), dtype=dtype, device=dev)
    att_ref = torch.full((n, c), float('nan'), device=dev)
    gap = torch.empty(n, _ext.dcn_tiles(h, w), c, device=dev)
    count = torch.zeros(n, dtype=torch.int32, device=dev)
    _ext.dsc_fwd(y, c, owp, plan.off_b, mask, (P * 9, 9, 1), wp, c, out_ref[..., :c], gap_partial=gap,
                 se=(*se_w, att_ref, count), **args)
    # the no-allocation entry point: inputs and outputs only
    out = torch.full((n, h, w, cs), float('nan'), dtype=dtype, device=dev)
    att = torch.full((n, c), float('nan'), device=dev)
    _ext.dsc_fwd(y, c, owp, plan.off_b, mask, (P * 9, 9, 1), wp, c, out[..., :c], se=(*se_w, att), noalloc=True,
                 **args)
    torch.cuda.synchronize()
    assert torch.isfinite(att_ref).all() and int(count.abs().sum()) == 0
    assert torch.equal(out[..., :c], out_ref[..., :c]), 'output differs from kad_dsc_fwd'
    assert torch.equal(att, att_ref), 'SE attention differs from kad_dsc_fwd'


@pytest.mark.parametrize('dt', ['f16', 'f32'])
def test_dsc_noalloc_matches_dsc_fwd(dt):
    dtype = {'f16': torch.float16, 'f32': torch.float32}[dt]
    for n, c, h, w in [(4, 86, 40, 44), (2, 40, 24, 20)]:   # second call: smaller batch and image
        print(f'dsc noalloc {dt} n={n} c={c} {h}x{w}', flush=True)
        _case(n, c, h, w, dtype, seed=n * 100 + c)


@pytest.mark.parametrize('dt', ['f16', 'bf16'])
def test_dsc_noalloc_narrow_path(dt):
    """16-bit, Cout <= 64 and at least 384 tile blocks: kad_dsc_fwd_noalloc takes the narrow
    two-blocks-per-CU kernel, whose fused SE keeps its partials and counters in the same library
    scratch; two calls in a row, the second smaller."""
    from kadconv import _ext
    dtype = {'f16': torch.float16, 'bf16': torch.bfloat16}[dt]
    for n, c, h, w in [(16, 16, 64, 64), (12, 24, 72, 60)]:
        assert n * _ext.dcn_tiles(h, w) >= 384
        print(f'dsc noalloc narrow {dt} n={n} c={c} {h}x{w}', flush=True)
        _case(n, c, h, w, dtype, seed=n * 10 + c)


def test_dsc_noalloc_rejects_oversize():
    """Beyond the scratch limit (N x tiles x Cout > 2^20 partials) the entry point
    returns KAD_EINVAL before any launch."""
    from kadconv import _ext
    a = _ext.DcnArgs()
    a.x = a.wpack = a.out = a.off_wpack = a.se_w1 = a.se_w2 = a.se_att = 256  # never dereferenced: rejected first
    a.n, a.cin, a.cout, a.h, a.w, a.stride, a.pad = 64, 128, 128, 200, 200, 1, 1
    a.x_cs, a.out_cs, a.se_hid = 128, 128, 128
    rc = _ext.load().kad_dsc_fwd_noalloc(a, None)
    assert rc == -1 and b'scratch limits' in _ext.load().kad_last_error()
