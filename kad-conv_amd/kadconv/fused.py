"""Fused HIP forwards for KADConv and DSC (the fast inference path).

``KADConvPlan`` snapshots one KADConv-like layer (KADConv, or KAD-CNet's
KADC4 / KADC4_m -- same attribute names, KAD-CNet/models/module/KADC/module.py:14-68)
into the form the kernels want: packed MFMA weights per dtype, eval-mode
BatchNorm folded into the DCN epilogue, LCSA parameters in one block.  Its
``forward`` runs, per branch i (kad_conv.py:112-121):

  kad_pyramid_proj  (once, all branches) avg_pool 2^i + 1x1 projection
                    x (NCHW/NHWC) -> y_i (NHWC), plus LCSA row/column partial sums
  kad_lcsa_prep     row means, strip-conv coefficients alpha/beta
  kad_lcsa_mask     sigmoid(LCSA) mask (MFMA GEMM)        -> [N, H_i, W_i, 9] fp32
  kad_dsc_fwd       conv_offset (kept on chip) + DCN + bias, BN, ReLU, branch
                    scale, GAP partials                   -> z_i (NHWC)
  kad_se_mlp        channel attention from the GAP partials -> att_i

and ``kad_branch_merge`` of the branch's own output channels: bilinear upsample,
x att, + x (the concat is the channel window each merge writes).  The three
chains run on side streams (fork after the pyramid, join at the end).

The reference does the same stage split on A100 at batch 1 with Triton, cuDNN
and one CUDA kernel (acceleration/kadc_fused_parallel.py:74-103,268-286;
kadc_fused_sm75.py:1400-1488,1544-1557).  Weights are captured when the plan
is built (as the reference folds BN at patch time, kadc_fused_parallel.py:647-655):
rebuild it (call enable_fast_inference again) after loading new weights.
"""
import torch

from . import _ext


DCN_BLOCK_COLS = 128  # output channels per block of the DCN kernels (8 MFMA column fragments)
SPLIT_MIN_TILES = 128  # tiles per launch from which a separate offset conv pays (half the CUs)
GROUPED = True         # KADConvPlan: branch stages as grouped launches on one stream for small layers
GROUP_MAX_WORK = 2048  # ... whose full-resolution DSC has less work: N x tiles x column fragments


def _f32(t):
    return None if t is None else t.detach().to(torch.float32).contiguous()


def _emat_dtype(dtype):
    """Precision of the LCSA mask GEMM (E matrix and strip activation u) for a run in `dtype`:
    fp16 for fp16 runs (packed-fp16 u, fp16 MFMA); fp32 for fp32 and bf16 runs, whose
    activations may exceed fp16's range (65504), where an fp16 u would turn the mask to NaN.
    The mask reads fp32 means whatever the input dtype, so bf16 loses nothing by this."""
    return torch.float16 if dtype == torch.float16 else torch.float32


def _fold_bn(bn):
    a = bn.weight.detach().double() / torch.sqrt(bn.running_var.detach().double() + bn.eps)
    b = bn.bias.detach().double() - bn.running_mean.detach().double() * a
    return a.float().contiguous(), b.float().contiguous()


def _lcsa_block(lcsa):
    """LCSA parameters as the fp32 block kad_lcsa_mask reads:
    w1[C][11] | b1[C] | bn_a[C] | bn_b[C] | w3[C][11] | b3[C] | w4[9][C] | b4[9]."""
    ex = lcsa.excite
    c = ex[0].weight.shape[0]
    if tuple(ex[0].weight.shape[1:]) != (1, 1, 11) or tuple(ex[3].weight.shape[1:]) != (1, 11, 1):
        raise NotImplementedError('LCSA kernels are written for band_kernel_size=11')
    bna, bnb = _fold_bn(ex[1])
    parts = [ex[0].weight.reshape(c, 11), ex[0].bias, bna, bnb, ex[3].weight.reshape(c, 11), ex[3].bias,
             ex[4].weight.reshape(9, c), ex[4].bias]
    blk = torch.cat([p.detach().to(torch.float32).reshape(-1) for p in parts]).contiguous()
    assert blk.numel() == _ext.lcsa_params_elems(c)
    return blk


class DSCPlan:
    """Snapshot of one DSC / DCN_RCA (kad_conv.py:42-67; KAD-CNet ops.py:40-72)."""

    def __init__(self, dsc):
        self.cin, self.cout = dsc.in_channels, dsc.out_channels
        ks = dsc.kernel_size if isinstance(dsc.kernel_size, int) else dsc.kernel_size[0]
        if ks != 3:
            raise NotImplementedError('DSC kernels are 3x3')
        st = dsc.stride if isinstance(dsc.stride, int) else dsc.stride[0]
        pad = dsc.padding if isinstance(dsc.padding, int) else dsc.padding[0]
        self.stride, self.pad = st, pad
        self.weight = _f32(dsc.weight)
        self.bias = _f32(dsc.bias)
        self.off_w = _f32(dsc.conv_offset.weight)
        self.off_b = _f32(dsc.conv_offset.bias)
        self.use_mask = bool(getattr(dsc, 'mask', True)) and hasattr(dsc, 'RCA_mask')
        self.lcsa = _lcsa_block(dsc.RCA_mask) if self.use_mask else None
        self._packed = {}

    def packed(self, dtype):
        """(DCN weights, offset-conv weights, LCSA E matrix, LCSA bias) for `dtype`;
        the LCSA matrix is fp16 for fp16 runs and fp32 otherwise (see _emat_dtype)."""
        if dtype not in self._packed:
            emat = ebias = None
            if self.use_mask:
                emat, ebias = _ext.lcsa_pack(self.lcsa, self.cin, _emat_dtype(dtype))
            self._packed[dtype] = (_ext.dcn_pack_weights(self.weight, dtype),
                                   _ext.dcn_pack_weights(self.off_w, dtype), emat, ebias)
        return self._packed[dtype]

    def eligible(self, x):
        return (x.is_cuda and x.dim() == 4 and x.dtype in (torch.float32, torch.float16, torch.bfloat16)
                and x.shape[1] == self.cin and self.stride == 1 and self.pad == 1 and x.numel() > 0)

    def out_shape(self, h, w):
        """(Cout, Ho, Wo) of the forward on an h x w input."""
        return self.cout, (h + 2 * self.pad - 3) // self.stride + 1, (w + 2 * self.pad - 3) // self.stride + 1

    def stages(self, y, n, h, w, out, out_layout, bias=None, post_mul=None, post_add=None, post_scale=None,
               relu=False, gap=None, tag='', sums=None, se=None, mask_split=True, x_nchw=None):
        """DSC on an NHWC map y [N, h, w, cs] (cin channels) as a list of
        (name, launch) pairs with every buffer allocated up front.  `sums` =
        (rows, nrp, cols, ncp) axial partial sums of y if already computed."""
        dev = y.device
        wp, owp, emat, ebias = self.packed(y.dtype)
        P = h * w
        st = []
        mask = None
        if self.use_mask:
            arow = torch.empty(n, h, self.cin, dtype=torch.float32, device=dev)
            colm = torch.empty(n, w, self.cin, dtype=torch.float32, device=dev)
            if sums is None:
                # no partial slices to reduce: the axial means in one launch (sums + prep)
                if x_nchw is not None and h * w <= _ext.AXIAL_NCHW_MAX_PX and x_nchw.data_ptr() % 16 == 0:
                    # the NCHW input itself: contiguous planes, one block each
                    st.append(('axial_means' + tag, lambda: _ext.axial_means_nchw(x_nchw, arow, colm)))
                else:
                    st.append(('axial_means' + tag, lambda: _ext.axial_means(y, self.cin, arow, colm)))
            else:
                rows, nrp, cols, ncp = sums
            mask = torch.empty(n, h, w, 9, dtype=torch.float32, device=dev)
            # split the mask's channel contraction over blocks when the image has few tiles (standalone
            # DSC); KADConv's coarse branches run beside the full-resolution chain and stay unsplit
            ks = _ext.lcsa_mask_splits(n, self.cin, h, w) if mask_split else 1
            work = torch.empty(_ext.lcsa_mask_work_elems(n, h, w, ks), dtype=torch.float32, device=dev) \
                if ks > 1 else None
            if sums is not None:
                st.append(('lcsa_prep' + tag, lambda: _ext.lcsa_prep(rows, nrp, cols, ncp, arow, colm, n, self.cin,
                                                                     h, w)))
            st.append(('lcsa_mask' + tag, lambda: _ext.lcsa_mask(arow, colm, self.lcsa, emat, ebias, mask, n,
                                                                 self.cin, h, w, ks, work)))
        b = self.bias if bias is None else bias
        if self.cout > DCN_BLOCK_COLS and se is None and n * _ext.dcn_tiles(h, w) >= SPLIT_MIN_TILES:
            # several 128-channel column blocks per tile: conv_offset once per tile (a plain 3x3 conv
            # into an fp32 [N, h, w, 18] map), then the deformable conv reading those offsets, instead
            # of every column block of the fused kernel recomputing the same offsets.  With few tiles
            # the separate offset launch occupies few CUs and costs more than it saves (measured:
            # [8,256,50,50] 166 -> 158 us split; [8,512,25,25], 40 tiles, 153 -> 156 us).
            off = torch.empty(n, h, w, 18, dtype=torch.float32, device=dev)
            st.append(('conv_offset' + tag, lambda: _ext.conv3x3_fwd(y, self.cin, owp, 18, off, bias=self.off_b)))
            st.append(('dsc' + tag, lambda: _ext.dcn_fwd(
                y, self.cin, off, (P * 18, 18, 1), mask, (P * 9, 9, 1), wp, self.cout, out, bias=b,
                post_mul=post_mul, post_add=post_add, post_scale=post_scale, relu=relu, out_layout=out_layout,
                gap_partial=gap)))
            return st
        # conv_offset + deformable conv in one kernel: the offsets stay on chip
        st.append(('dsc' + tag, lambda: _ext.dsc_fwd(
            y, self.cin, owp, self.off_b, mask, (P * 9, 9, 1), wp, self.cout, out, bias=b, post_mul=post_mul,
            post_add=post_add, post_scale=post_scale, relu=relu, out_layout=out_layout, gap_partial=gap, se=se)))
        return st

    def run(self, *args, **kw):
        for _, fn in self.stages(*args, **kw):
            fn()
        return args[4]

    def forward(self, x):
        """Standalone DSC forward: NCHW (or channels-last) in, same format out."""
        from .ops import _nhwc_view
        n, _, h, w = x.shape
        y, _ = _nhwc_view(x)
        if x.is_contiguous(memory_format=torch.channels_last) and not x.is_contiguous():
            out = torch.empty(n, self.cout, h, w, dtype=x.dtype, device=x.device, memory_format=torch.channels_last)
            self.run(y, n, h, w, out.permute(0, 2, 3, 1), _ext.KAD_NHWC)
            return out
        out = torch.empty(n, self.cout, h, w, dtype=x.dtype, device=x.device)
        return self.run(y, n, h, w, out, _ext.KAD_NCHW, x_nchw=x if x.is_contiguous() else None)


def _channels_last_view(x):
    """x is channels-last memory (NCHW-shaped view), dense or a channel slice of a wider buffer
    (pixel stride >= C); a dense NCHW tensor is not."""
    if x.dim() != 4 or x.is_contiguous():
        return False
    N, C, H, W = x.shape
    return (x.stride(1) == 1 and x.stride(3) >= C and x.stride(2) == x.stride(3) * W
            and (N == 1 or x.stride(0) == x.stride(2) * H))


class _Branch:
    def __init__(self, conv, fc, scale, c_off):
        proj, dsc, bn = conv[0], conv[1], conv[2]
        self.c = proj.weight.shape[0]
        self.cs = (self.c + 7) // 8 * 8
        self.c_off = c_off
        self.proj_w = _f32(proj.weight.reshape(self.c, -1))
        self.proj_b = _f32(proj.bias)
        self.dsc = DSCPlan(dsc)
        self.bn_a, self.bn_b = _fold_bn(bn)
        self.scale = _f32(scale.weight.reshape(-1))
        self.w1, self.b1 = _f32(fc[0].weight.reshape(fc[0].weight.shape[0], -1)), _f32(fc[0].bias)
        self.w2, self.b2 = _f32(fc[2].weight.reshape(fc[2].weight.shape[0], -1)), _f32(fc[2].bias)
        self.hid = self.w1.shape[0]
        self._packed = {}

    def proj_packed(self, dtype):
        if dtype not in self._packed:
            self._packed[dtype] = _ext.gemm_pack_weights(self.proj_w, dtype)
        return self._packed[dtype]


class KADConvPlan:
    def __init__(self, layer):
        self.n = layer.n
        self.dim = layer.convs[0][0].weight.shape[1]
        self.branches = []
        c_off = 0
        for i in range(self.n):
            scale = layer.weight[i][0]
            br = _Branch(layer.convs[i], layer.fc[i], scale, c_off)
            c_off += br.c
            self.branches.append(br)
        if c_off != self.dim:
            raise ValueError('branch widths do not add up to the layer width')
        if self.n > 3:
            raise NotImplementedError('the fused forward covers n <= 3 branches (the paper uses 3)')
        # grouped: the branches' LCSA and DSC stages run as one launch each (all branches), on the
        # caller's stream; else each branch chain runs on a side stream of its own (see _grouped)
        self.groupable = GROUPED and all(br.dsc.use_mask for br in self.branches)

    def _grouped(self, x):
        """Grouped launches unless the full-resolution DSC is heavy: N x tiles x 16-channel
        column fragments >= GROUP_MAX_WORK.  Small layers are bound by launch and queue
        latency, and under HIP-graph replay the three side-stream chains of a small layer
        were measured to run one after another (KAD-CNet-S: 9.62 -> 9.14 ms per batch with
        every KADC4 grouped).  A heavy layer keeps the side streams: the coarse branches'
        DSCs and merges then fill the last, partly empty round of the full-resolution DSC
        (KADConv(256) at [8, 256, 100, 100], 640 tiles x 6 fragments: 210 us with streams,
        227 us grouped)."""
        frags = min((self.branches[0].c + 15) // 16, 8)
        work = x.shape[0] * _ext.dcn_tiles(x.shape[2], x.shape[3]) * frags
        return self.groupable and work < GROUP_MAX_WORK

    def eligible(self, x):
        if not (x.is_cuda and x.dim() == 4 and x.dtype in (torch.float32, torch.float16, torch.bfloat16)):
            return False
        if x.shape[1] != self.dim or x.shape[0] == 0:  # an empty batch takes the module's own forward
            return False
        s = 2 ** (self.n - 1)
        return x.shape[2] >= s and x.shape[3] >= s

    def out_shape(self, h, w):
        """(C, H, W): shape-preserving."""
        return self.dim, h, w

    def stages(self, x):
        """The fused forward as (name, launch) pairs in stream order; returns (stages, out)."""
        if self._grouped(x):
            return self.schedule_grouped(x)
        pre, branches, post, out = self.schedule(x)
        return pre + [s for b in branches for s in b] + post, out

    def _io(self, x, out=None):
        """(x view for the kernels, its layout, out, out view, out layout).  out: for a channels-last
        x, an NCHW-shaped view of channels-last memory whose pixel stride may exceed C (a channel
        slice of a wider buffer, e.g. a concat), written in place."""
        nhwc = _channels_last_view(x)
        if nhwc:
            if out is None:
                out = torch.empty_like(x, memory_format=torch.channels_last)
            elif (out.shape != x.shape or out.dtype != x.dtype or out.device != x.device or out.stride(1) != 1
                  or out.stride(3) < x.shape[1] or out.stride(2) != out.stride(3) * x.shape[3]):
                raise ValueError('out must be a channels-last view shaped like x (channel stride 1)')
            return x.permute(0, 2, 3, 1), _ext.KAD_NHWC, out, out.permute(0, 2, 3, 1), _ext.KAD_NHWC
        if out is not None:
            raise ValueError('out= needs a channels-last input')
        x = x.contiguous()
        out = torch.empty_like(x)
        return x, _ext.KAD_NCHW, out, out, _ext.KAD_NCHW

    def schedule_grouped(self, x, out=None):
        """The forward as one chain of launches on one stream: the pyramid, then the LCSA
        means, the LCSA masks and the fused DSCs (+ SE) of all branches as one launch each
        (kad_lcsa_prep_group, kad_lcsa_mask_group, kad_dsc_fwd_group), then the merges.
        Returns (stages, out)."""
        N, C, H, W = x.shape
        dev, dtype = x.device, x.dtype
        xin, in_layout, out, out_v, out_layout = self._io(x, out)
        ntx, nty = _ext.pyramid_tiles(H, W)
        pyr, lcsa, dcn, keep, merges = [], [], {}, [], []
        edt = _emat_dtype(dtype)
        st = []
        for i, br in enumerate(self.branches):
            h, w = H >> i, W >> i
            P = h * w
            full = (h, w) == (H, W)
            y = torch.empty(N, h, w, br.cs, dtype=dtype, device=dev)
            rows = torch.empty(N, ntx, h, br.c, dtype=torch.float32, device=dev)
            cols = torch.empty(N, nty, w, br.c, dtype=torch.float32, device=dev)
            pyr.append({'wpack': br.proj_packed(dtype), 'bias': br.proj_b, 'cout': br.c, 'out': y,
                        'rowpart': rows, 'colpart': cols})
            wp, owp, emat, ebias = br.dsc.packed(dtype)
            arow = torch.empty(N, h, br.c, dtype=torch.float32, device=dev)
            colm = torch.empty(N, w, br.c, dtype=torch.float32, device=dev)
            mask = torch.empty(N, h, w, 9, dtype=torch.float32, device=dev)
            lcsa.append(_ext.lcsa_args(rows, ntx, cols, nty, arow, colm, br.dsc.lcsa, emat, ebias, mask, N, br.c, h,
                                       w))
            gap = torch.empty(N, _ext.dcn_tiles(h, w), br.c, dtype=torch.float32, device=dev)
            if full:  # written straight into its channel slice of the output
                z = out_v[:, br.c_off:br.c_off + br.c] if out_layout == _ext.KAD_NCHW \
                    else out_v[..., br.c_off:br.c_off + br.c]
                z_layout = out_layout
            else:
                z = torch.empty(N, h, w, br.cs, dtype=dtype, device=dev)
                z_layout = _ext.KAD_NHWC
            att = torch.empty(N, br.c, dtype=torch.float32, device=dev)
            se = (br.w1, br.b1, br.w2, br.b2, att, self._se_counters(dev, i, N))
            a = _ext.dsc_args(y, br.c, owp, br.dsc.off_b, mask, (P * 9, 9, 1), wp, br.c, z, bias=br.dsc.bias,
                              post_mul=br.bn_a, post_add=br.bn_b, post_scale=br.scale, relu=True,
                              out_layout=z_layout, gap_partial=gap, se=se)
            dcn.setdefault(min((br.c + 15) // 16, 8), []).append(a)   # one launch per instantiation
            keep += [y, rows, cols, arow, colm, mask, gap, z, att]
            merges.append((full, {'z': z, 'c': br.c, 'c_off': br.c_off, 'att': att}))
        st.append(('pyramid', lambda: _ext.pyramid_proj(xin, in_layout, C, pyr)))
        st.append(('lcsa_prep', lambda keep=keep: _ext.lcsa_prep_group(lcsa)))
        st.append(('lcsa_mask', lambda keep=keep: _ext.lcsa_mask_group(lcsa, edt)))
        for k, args in dcn.items():
            st.append(('dsc' if len(dcn) == 1 else f'dsc_nb{k}', lambda args=args, keep=keep: _ext.dsc_fwd_group(args)))
        if out_layout == _ext.KAD_NHWC:
            mb = [m for _, m in merges]
            st.append(('merge', lambda: _ext.branch_merge(out_v, out_layout, mb, residual=xin)))
        else:
            for full, m in merges:
                if full:
                    st.append(('merge0', lambda m=m: _ext.scale_residual(out_v, m['att'], xin, m['c_off'], m['c'],
                                                                        out_layout)))
            up = [m for full, m in merges if not full]
            if up:  # the upsampled branches' windows are contiguous: one band merge
                lo, hi = up[0]['c_off'], up[-1]['c_off'] + up[-1]['c']
                st.append(('merge', lambda: _ext.branch_merge(out_v, out_layout, up, residual=xin, channels=(lo, hi))))
        return st, out

    def schedule(self, x, out=None):
        """(pre, [per-branch stages], post, out): the branch chains (LCSA, DSC,
        SE, and the merge of the branch's own output channels) only depend on
        `pre` (the pyramid), so forward() runs them on side streams concurrently."""
        N, C, H, W = x.shape
        dev, dtype = x.device, x.dtype
        xin, in_layout, out, out_v, out_layout = self._io(x, out)
        x = xin if in_layout == _ext.KAD_NCHW else x
        st = []
        ys, sums = [], []
        pyr = []
        ntx, nty = _ext.pyramid_tiles(H, W)
        for i, br in enumerate(self.branches):
            h, w = H >> i, W >> i
            y = torch.empty(N, h, w, br.cs, dtype=dtype, device=dev)
            rows = torch.empty(N, ntx, h, br.c, dtype=torch.float32, device=dev)
            cols = torch.empty(N, nty, w, br.c, dtype=torch.float32, device=dev)
            ys.append(y)
            sums.append((rows, ntx, cols, nty))
            pyr.append({'wpack': br.proj_packed(dtype), 'bias': br.proj_b, 'cout': br.c, 'out': y,
                        'rowpart': rows, 'colpart': cols})
        st.append(('pyramid', lambda: _ext.pyramid_proj(xin, in_layout, C, pyr)))
        chains, merges = [], []
        for i, br in enumerate(self.branches):
            h, w = H >> i, W >> i
            P = h * w
            full = (h, w) == (H, W)
            tiles = _ext.dcn_tiles(h, w)
            gap = torch.empty(N, tiles, br.c, dtype=torch.float32, device=dev)
            if full:
                # full resolution: the DSC writes its channel slice of the output directly
                # (no upsampling needed); attention and residual are applied in place below
                z = out_v[:, br.c_off:br.c_off + br.c] if out_layout == _ext.KAD_NCHW \
                    else out_v[..., br.c_off:br.c_off + br.c]
                z_layout = out_layout
            else:
                z = torch.empty(N, h, w, br.cs, dtype=dtype, device=dev)
                z_layout = _ext.KAD_NHWC
            # the SE MLP runs in the DSC kernel's last block per image (att from the GAP partials)
            att = torch.empty(N, br.c, dtype=torch.float32, device=dev)
            se = (br.w1, br.b1, br.w2, br.b2, att, self._se_counters(dev, i, N))
            ch = br.dsc.stages(ys[i], N, h, w, z, z_layout, post_mul=br.bn_a, post_add=br.bn_b,
                               post_scale=br.scale, relu=True, gap=gap, tag=str(i), sums=sums[i], se=se,
                               mask_split=False)
            if out_layout == _ext.KAD_NHWC:
                # channels-last: one merge of every branch after the join (below)
                merges.append({'z': z, 'c': br.c, 'c_off': br.c_off, 'att': att})
            elif full:
                ch.append((f'merge{i}', lambda br=br, att=att: _ext.scale_residual(
                    out_v, att, xin, br.c_off, br.c, out_layout)))
            else:
                # this branch's channels of the output, as soon as the branch is done
                mb = [{'z': z, 'c': br.c, 'c_off': br.c_off, 'att': att}]
                ch.append((f'merge{i}', lambda mb=mb, br=br: _ext.branch_merge(
                    out_v, out_layout, mb, residual=xin, channels=(br.c_off, br.c_off + br.c))))
            chains.append(ch)
        post = []
        if merges:
            # NHWC: all branches in one launch, a thread per pixel and 8-channel piece (the full-
            # resolution branch is read from its own window of the output, in place)
            post.append(('merge', lambda: _ext.branch_merge(out_v, out_layout, merges, residual=xin)))
        return st, chains, post, out

    def _se_counters(self, dev, i, n):
        """Per-image arrival counters of branch i's fused SE (zero between calls), kept per device.
        A larger batch gets a new buffer, but the old one stays alive with the plan: a HIP graph
        captured earlier holds its address and its replays keep using it.  Forwards of one layer
        that overlap on the GPU (several streams) share these counters and must not run concurrently."""
        key = (torch.device(dev).index, i)
        counters = getattr(self, '_se_count', {})
        c = counters.get(key)
        if c is None or c.numel() < n:
            if c is not None:
                self.__dict__.setdefault('_se_retired', []).append(c)
            c = torch.zeros(max(n, 1), dtype=torch.int32, device=dev)
            counters[key] = c
            self._se_count = counters
        return c

    def _side_streams(self, dev):
        """One side stream per branch chain (default priority), created once per device."""
        key = torch.device(dev).index
        streams = getattr(self, '_side', {})
        if key not in streams:
            streams[key] = [torch.cuda.Stream(device=dev) for _ in self.branches]
            self._side = streams
        return streams[key]

    def forward(self, x, out=None):
        """Grouped: every stage on the caller's stream.  Else the pyramid on the caller's
        stream, the branch chains forked onto side streams (concurrent on the GPU;
        HIP-graph capture records the fork/join as graph edges), merge after the join.
        out: see _io (channels-last input only)."""
        if self._grouped(x):
            st, out = self.schedule_grouped(x, out)
            for _, fn in st:
                fn()
            return out
        pre, chains, post, out = self.schedule(x, out)
        for _, fn in pre:
            fn()
        main = torch.cuda.current_stream(x.device)
        side = self._side_streams(x.device)
        fork = torch.cuda.Event()
        fork.record(main)
        joins = []
        for s, chain in zip(side, chains):
            s.wait_event(fork)
            with torch.cuda.stream(s):
                for _, fn in chain:
                    fn()
            ev = torch.cuda.Event()
            ev.record(s)
            joins.append(ev)
        for ev in joins:
            main.wait_event(ev)
        for _, fn in post:
            fn()
        return out
