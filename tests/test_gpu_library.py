"""torch.compile over the fast path: the HIP calls are typed custom operators
(kadconv::layer_fwd, kadconv::deform_conv2d), so a fast-enabled layer compiles
with fullgraph=True (no graph break) and gives the eager output bit for bit.
Backend aot_eager: dynamo + AOT tracing with the fake implementations, no code
generation."""
import pytest
import torch

from kadconv import synthetic as S

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('kind', ['kadconv', 'dsc'])
def test_compile_fast_layer_fullgraph(kind):
    import kadconv
    if kind == 'kadconv':
        m = kadconv.KADConv(64)
        m.load_state_dict(S.make_kadconv_state(64, seed=4), strict=False)
        x = torch.randn(2, 64, 40, 36, generator=torch.Generator().manual_seed(1))
    else:
        m = kadconv.DSC(48, 40)
        m.load_state_dict(S.make_dsc_state(48, 40, seed=4, offset_std_px=2.0), strict=False)
        x = torch.randn(2, 48, 30, 22, generator=torch.Generator().manual_seed(1))
    m = m.to('cuda', torch.float16).eval()
    kadconv.enable_fast_inference(m)
    x = x.to('cuda', torch.float16)
    torch._dynamo.reset()
    cm = torch.compile(m, backend='aot_eager', fullgraph=True)
    print(f'compile {kind}', flush=True)
    with torch.no_grad():
        eager = m(x)
        got = cm(x)
        got2 = cm(x)
    torch.cuda.synchronize()
    assert torch.equal(got, eager) and torch.equal(got2, eager)


def test_compile_deform_conv2d_op():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 12, 15, 17, generator=g).cuda()
    off = (torch.randn(2, 18, 15, 17, generator=g) * 2).cuda()
    w = (torch.randn(20, 12, 3, 3, generator=g) * 0.1).cuda()
    b = torch.randn(20, generator=g).cuda()
    mask = torch.rand(2, 9, 15, 17, generator=g).cuda()

    def f(x, off, w, b, mask):
        return torch.ops.kadconv.deform_conv2d(x, off, w, b, 1, 1, 1, 1, 1, 1, mask) * 2.0

    torch._dynamo.reset()
    cf = torch.compile(f, backend='aot_eager', fullgraph=True)
    eager = f(x, off, w, b, mask)
    got = cf(x, off, w, b, mask)
    torch.cuda.synchronize()
    assert torch.equal(got, eager)
