"""kad_pyramid_proj on its own: the per-branch pooled 1x1 projections
(avg_pool2d(x, 2^b) then conv1x1, kad_conv.py:101,115) against F.conv2d in
float64, and the row / column partial sums it hands to the LCSA prep.

The partial-sum buffers are filled with NaN first: every slice the consumer
reads (all ntx row slices of a pooled row, all nty column slices of a pooled
column, including tiles that hold no row of a coarse branch) must be written,
and the slices must add up to the branch output's row and column sums.
Shapes cover ragged tiles: (21, 70) has a last tile row band with no pooled row of
branch 1 (its column partials must be zeros); (13, 66) has a last tile column with no
column of branch 2 (its row partial must be written, as zero).
The 16-bit band shapes (H and W multiples of 4, W <= 100 with 4 W mod 128 <= 16) run the
one-block-per-4-row-band kernel: W = 100 has three full 128-pixel groups and a 16-pixel tail, 96
three groups, 36 one group and a tail, 64 and 32 whole groups; C = 40, 96 and 160 give K loops of
2, 3 and 5 steps (padded to multiples of three), C = 256 the KADConv(256) metric's eight.
Tolerances: fp32 1e-4 relative; fp16/bf16 1e-2 (outputs) and 2e-2 relative
(sums of up to W values)."""
import pytest
import torch
import torch.nn.functional as F

from tests._util import check_close, quant

pytestmark = pytest.mark.gpu

DT = {'f32': torch.float32, 'f16': torch.float16, 'bf16': torch.bfloat16}


@pytest.mark.parametrize('dt', ['f32', 'f16', 'bf16'])
@pytest.mark.parametrize('shape', [(2, 48, 37, 29), (1, 40, 21, 70), (2, 24, 8, 8), (1, 24, 13, 66),
                                   (2, 256, 8, 100), (1, 96, 12, 96), (2, 40, 4, 36), (1, 160, 8, 64),
                                   (1, 48, 8, 32)])
def test_pyramid_proj_and_partial_sums(dt, shape):
    from kadconv import _ext
    dtype = DT[dt]
    N, C, H, W = shape
    g = torch.Generator().manual_seed(H * W)
    x = torch.randn(N, C, H, W, generator=g)
    couts = [C // 3 + 1, C // 3, C // 3 - 1]
    ws = [torch.randn(c, C, generator=g) * (0.3 / C ** 0.5) for c in couts]  # |y| < 2: bf16 rounding < 1e-2
    bs = [torch.randn(c, generator=g) * 0.1 for c in couts]
    ntx, nty = _ext.pyramid_tiles(H, W)
    dev = 'cuda'
    xd = x.to(dtype).to(dev)
    br = []
    for b, c in enumerate(couts):
        h, w = H >> b, W >> b
        cs = (c + 7) // 8 * 8
        br.append({'wpack': _ext.gemm_pack_weights(ws[b].to(dev), dtype), 'bias': bs[b].to(dev), 'cout': c,
                   'out': torch.full((N, h, w, cs), float('nan'), dtype=dtype, device=dev),
                   'rowpart': torch.full((N, ntx, h, c), float('nan'), device=dev),
                   'colpart': torch.full((N, nty, w, c), float('nan'), device=dev)})
    print(f'pyramid {dt} {shape} ntx={ntx} nty={nty}', flush=True)
    _ext.pyramid_proj(xd, _ext.KAD_NCHW, C, br)
    torch.cuda.synchronize()
    xq = quant(x, dtype)
    for b, c in enumerate(couts):
        p = F.avg_pool2d(xq, 2 ** b) if b else xq
        ref = F.conv2d(p, quant(ws[b], dtype).view(c, C, 1, 1), bs[b].double())  # [N, c, h, w]
        y = br[b]['out'][..., :c].permute(0, 3, 1, 2)
        check_close(y, ref, dtype, f'branch {b} output')
        rp, cp = br[b]['rowpart'].cpu().double(), br[b]['colpart'].cpu().double()
        assert torch.isfinite(rp).all(), f'branch {b}: unwritten row partial slices'
        assert torch.isfinite(cp).all(), f'branch {b}: unwritten column partial slices'
        rows_ref = ref.sum(dim=3).permute(0, 2, 1)   # [N, h, c]
        cols_ref = ref.sum(dim=2).permute(0, 2, 1)   # [N, w, c]
        tol = 1e-4 if dtype == torch.float32 else 2e-2
        for got, want, what in [(rp.sum(1), rows_ref, 'row'), (cp.sum(1), cols_ref, 'column')]:
            err = (got - want).abs().max().item()
            assert err <= tol * max(want.abs().max().item(), 1.0), f'branch {b} {what} sums: {err:.3e}'
