/*
 * kadconv_hip.h -- C ABI of libkadconv_hip.so, the gfx950 HIP kernels behind
 * the kadconv package's fast KAD-Conv inference forward.
 *
 * Reference interface replaced: the pybind11 extension `kadc_dcn16_*`
 * (KAD-Conv/kadconv/acceleration/kadc_dcn16.cpp:247-330, JIT-loaded by
 * kadc_dcn16_backend.py:55-86) and the Triton launchers the fast forward calls
 * (acceleration/kadc_fused_sm75.py, acceleration/kadc_dcn_direct.py).  Each
 * declaration below cites the reference entry point it stands in for.
 *
 * Rules for every entry point:
 *  - plain pointers and sizes only; all pointers are device pointers unless
 *    stated otherwise; the caller owns every buffer (the library never
 *    allocates or synchronises);
 *  - work is enqueued on `stream` (a hipStream_t; NULL = the null stream), so
 *    calls are capturable into a HIP graph;
 *  - return 0 on success or a negative KAD_E* code; the message for the last
 *    failure on the calling thread is returned by kad_last_error();
 *  - no mutable global state, with one exception: kad_dsc_fwd_noalloc keeps its
 *    scratch in a file-scope device array and a per-device address table (see
 *    its declaration).  Every other call, from any host thread on any stream,
 *    touches only the buffers the caller passes, so such calls do not interfere.
 */
#ifndef KADCONV_HIP_H_
#define KADCONV_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KAD_ABI_VERSION 4

/* element types */
#define KAD_F32 0
#define KAD_F16 1
#define KAD_BF16 2

/* activations (kad_dcn_args.relu) */
#define KAD_ACT_NONE 0
#define KAD_ACT_RELU 1
#define KAD_ACT_SILU 2

/* feature-map layouts */
#define KAD_NHWC 0
#define KAD_NCHW 1

/* error codes */
#define KAD_OK 0
#define KAD_EINVAL (-1)   /* bad argument (shape, dtype, alignment, null pointer) */
#define KAD_ELAUNCH (-2)  /* the HIP runtime rejected a launch */
#define KAD_EUNSUPPORTED (-3)

/* Version of this ABI (KAD_ABI_VERSION).  No reference counterpart. */
int kad_abi_version(void);

/* Message of the last failed call on this thread ("" if none).
 * Replaces TORCH_CHECK's RuntimeError text (acceleration/kadc_dcn16.cpp:148-202). */
const char *kad_last_error(void);

/* ------------------------------------------------------------------------ */
/* Deformable convolution core (DCNv2, 3x3, one offset group).               */
/* ------------------------------------------------------------------------ */

/* Number of elements of the packed weight buffer for kad_dcn_fwd.
 * Layout: [Cout_pad][Cin_pad/32][9][32], Cin_pad = roundup(Cin, 32),
 * Cout_pad = roundup(Cout, 16); element type = the op's dtype.  */
int64_t kad_dcn_wpack_elems(int cin, int cout);

/* Pack fp32 weights [Cout][Cin][3][3] (device) into the layout above.
 * Stands in for the weight repacking the reference does at install time
 * (acceleration/kadc_dcn16_backend.py:218-264). */
int kad_dcn_pack_weights(const float *w, void *wpack, int cin, int cout, int dtype, void *stream);

/* Number of output tiles per image (the row count of the per-tile GAP
 * partials kad_dcn_fwd writes when gap_partial != NULL). */
int kad_dcn_tiles(int ho, int wo);

typedef struct kad_dcn_args {
  const void *x;          /* input, NHWC [N][H][W][x_cs], dtype; channels >= Cin are 0 */
  const float *offset;    /* offset(n, p, j): offset[n*off_sn + p*off_sp + j*off_sc], j in [0,18): 2k=dy, 2k+1=dx */
  const float *mask;      /* mask(n, p, k) likewise with mask_s*; NULL = all ones */
  const void *wpack;      /* weights packed by kad_dcn_pack_weights, dtype */
  const float *bias;      /* [Cout] or NULL */
  const float *post_mul;  /* [Cout] or NULL: v = (acc + bias) * post_mul + post_add */
  const float *post_add;  /* [Cout] or NULL */
  const float *post_scale;/* [Cout] or NULL: applied after the optional ReLU */
  void *out;              /* NHWC [N][Ho][Wo][out_cs] or NCHW [N][Cout][Ho][Wo], dtype */
  float *gap_partial;     /* [N][kad_dcn_tiles(Ho,Wo)][Cout] per-tile sums of out, or NULL */
  const void *off_wpack;  /* kad_dsc_fwd only: conv_offset weights packed by kad_dcn_pack_weights (Cout = 18) */
  const float *off_bias;  /* kad_dsc_fwd only: conv_offset bias [18] or NULL */
  int64_t off_sn, off_sp, off_sc;
  int64_t mask_sn, mask_sp, mask_sc;
  int n, cin, cout, h, w, stride, pad;
  int x_cs;               /* channel stride of x (multiple of 8; >= Cin) */
  int out_layout;         /* KAD_NHWC or KAD_NCHW */
  int out_cs;             /* NHWC: channel stride of out; NCHW: channel planes per image of out
                             (both >= Cout: a channel slice of a wider tensor can be written) */
  int dtype;              /* KAD_F32 / KAD_F16 / KAD_BF16 (x, wpack, out) */
  int relu;               /* activation between post_add and post_scale: KAD_ACT_NONE (0), KAD_ACT_SILU (2),
                             else ReLU (KAD_ACT_RELU = 1) */
  /* Squeeze-excitation of the output, fused (needs gap_partial).  When se_att is
   * not NULL, the last block of each image to finish sums that image's GAP
   * partials in a fixed order and writes
   *   se_att[n][c] = sigmoid(W2 relu(W1 g + b1) + b2)[c],  g = se_inv_count * sum of partials,
   * i.e. kad_se_mlp over the partials, without a launch of its own.
   * se_count: [N] counters, zero before the first call; every call that
   * completes leaves them zero again.  Calls that overlap on one se_count race. */
  const float *se_w1;     /* [se_hid][Cout] */
  const float *se_b1;     /* [se_hid] or NULL */
  const float *se_w2;     /* [Cout][se_hid] */
  const float *se_b2;     /* [Cout] or NULL */
  float *se_att;          /* [N][Cout], or NULL: no SE */
  unsigned *se_count;     /* [N] */
  int se_hid;
  float se_inv_count;     /* 1 / (Ho * Wo) */
} kad_dcn_args;

/* out = post_scale * act((deform_conv3x3(x, offset, mask, W) + bias) * post_mul + post_add).
 * Stands in for kadc_dcn16.cpp:247-289 `forward*`/`forward_*_unsafe`
 * (kernel kadc_dcn16_kernel.cu:92-314) and for torchvision.ops.deform_conv2d
 * as called at KAD-Conv/kadconv/kad_conv.py:66-67. */
int kad_dcn_fwd(const kad_dcn_args *a, void *stream);

/* Plain 3x3 convolution on the same NHWC machinery (offset/mask ignored, may
 * be NULL): DSC's offset branch `conv_offset` (KAD-Conv/kadconv/kad_conv.py:55-56,64),
 * run by cuDNN in the reference fast path (acceleration/kadc_fused_sm75.py:1414-1421).
 * `out` is always fp32 here (offsets feed the sampling coordinates); weights
 * are packed with kad_dcn_pack_weights; post_* and relu apply as in kad_dcn_fwd. */
int kad_conv3x3_fwd(const kad_dcn_args *a, void *stream);

/* Whole DSC forward given the LCSA mask: offset = conv_offset(x) (weights
 * a->off_wpack, bias a->off_bias) is computed inside each output tile and
 * consumed by the deformable convolution in the same kernel, so the offsets
 * never go to memory (a->offset is ignored).  Otherwise as kad_dcn_fwd.
 * Stands in for DSC.forward (KAD-Conv/kadconv/kad_conv.py:63-67) minus the
 * mask branch, i.e. the reference fast path's cuDNN conv_offset
 * (acceleration/kadc_fused_sm75.py:1414-1421) followed by its DCN kernel
 * (kadc_dcn16.cpp:247-289).  stride <= 2 (also for kad_conv3x3_fwd). */
int kad_dsc_fwd(const kad_dcn_args *a, void *stream);

/* Up to KAD_DCN_GROUP_MAX independent kad_dsc_fwd problems in one launch (the
 * three branches of a KAD-Conv layer): a[0..count) as for kad_dsc_fwd, all with
 * the same dtype and the same ceil(Cout / 16) (capped at 8).  Each problem's
 * results are those of kad_dsc_fwd on it; problems must not share outputs or SE
 * counters.  No reference counterpart (scheduling: one launch instead of three
 * concurrent streams, whose overlap a HIP graph does not guarantee). */
#define KAD_DCN_GROUP_MAX 4
int kad_dsc_fwd_group(const kad_dcn_args *a, int count, void *stream);

/* kad_dsc_fwd that allocates nothing and needs no caller-owned scratch.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture that must not call hipMalloc, tight
 * serving loops, harnesses that forbid allocation).  The fused
 * squeeze-excitation's GAP partials and per-image arrival counters live in a
 * library-owned device array (one per GPU, held until the process ends):
 * a->gap_partial and a->se_count must be NULL; with a->se_att set, at most
 * 4096 images and N x kad_dcn_tiles(Ho, Wo) x Cout <= 1048576 partials
 * (4 MiB), else KAD_EINVAL.  Inputs and outputs are the caller's, as in
 * kad_dsc_fwd, and the results are identical to it.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams or
 * host threads) race.  The device is the calling thread's current device. */
int kad_dsc_fwd_noalloc(const kad_dcn_args *a, void *stream);

/* ------------------------------------------------------------------------ */
/* 1x1 convolution GEMM with fused input average pool and bias/SiLU epilogue */
/* ------------------------------------------------------------------------ */

/* Elements of the packed weight buffer (dtype): the rows
 * [roundup(roundup(Cout,8),128)][roundup(Cin,32)], then the same values in the
 * MFMA fragment order of the NCHW fast path (twice the row layout in all). */
int64_t kad_gemm_wpack_elems(int cin, int cout);

/* Pack fp32 weights [Cout][Cin] (device) for kad_gemm1x1_fwd. */
int kad_gemm_pack_weights(const float *w, void *wpack, int cin, int cout, int dtype, void *stream);

typedef struct kad_gemm_args {
  const void *x;          /* NCHW [N][Cin][H][W] or NHWC [N][H][W][x_cs], dtype */
  const void *wpack;      /* kad_gemm_pack_weights output */
  const float *bias;      /* [Cout] or NULL */
  void *out;              /* NCHW [N][Cout][H/pool][W/pool] or NHWC [...][out_cs]: channels [0, Cout) written,
                             [Cout, min(out_cs, roundup(Cout, 8))) zeroed, the rest of the stride untouched (so
                             out may be a channel slice of a concat buffer) */
  int n, cin, cout, h, w;
  int pool;               /* s >= 1: avg_pool2d(kernel=s, stride=s, floor) applied to x first */
  int in_layout, x_cs;
  int out_layout, out_cs;
  int act;                /* 0 = none, 1 = SiLU */
  int dtype;
} kad_gemm_args;

/* out = act(W * avgpool_s(x) + b).  Stands in for the per-branch
 * `avg_pool2d` + `nn.Conv2d(dim, c, 1)` of KADConv (kad_conv.py:101,115;
 * reference fast path kadc_fused_parallel.py:74-103 with cuDNN) and for the
 * fused 1x1 conv + bias + SiLU (KAD-CNet/inference/acceleration/kadc_gemm_silu.cpp:1-33
 * -> kadc_gemm_silu.cu:125-176; acceleration/kadc_fused_sm75.py:504-532,616-629). */
int kad_gemm1x1_fwd(const kad_gemm_args *a, void *stream);

/* KADDown input pass (the op is builder-defined: no reference counterpart;
 * definition oracle/kadconv_oracle.py:kaddown_forward).  x NCHW [N][C][H][W]
 * -> u NCHW [N][nb*C][H/2][W/2], same dtype, with
 *   u[:, b*C + c] = bilinear_resize(avgpool(x, 2^(b+1))[:, c], (H/2, W/2))
 * (align_corners=False; b = 0 needs no resize), b < nb <= 3, H, W >= 2^nb.
 * KADDown is then one kad_gemm1x1_fwd over u with the branch projections
 * stacked along Cin, softmax(alpha)_b and sigmoid(gate) folded into them. */
int kad_kaddown_prep(const void *x, void *u, int n, int c, int h, int w, int nb, int dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* One-pass branch pyramid: avg-pool 2^b + 1x1 projection for b = 0..nb-1    */
/* ------------------------------------------------------------------------ */

/* Tile grid of kad_pyramid_proj (4 x 32 input pixels per tile): the number of
 * row / column partial-sum slices it writes. */
int kad_pyramid_tiles(int h, int w, int *ntx, int *nty);

typedef struct kad_pyramid_args {
  const void *x;            /* NCHW [N][Cin][H][W] or NHWC [N][H][W][x_cs], dtype */
  int n, cin, h, w, in_layout, x_cs, dtype;
  int nb;                   /* branches, 1..3; branch b pools by 2^b */
  int ntx, nty;             /* from kad_pyramid_tiles */
  const void *wpack[3];     /* kad_gemm_pack_weights(W_b [cout_b][Cin]) */
  const float *bias[3];     /* [cout_b] or NULL */
  void *out[3];             /* y_b NHWC [N][H>>b][W>>b][out_cs_b], pad channels written 0 */
  int cout[3], out_cs[3], out_h[3], out_w[3];
  float *rowpart[3];        /* [N][ntx][H>>b][cout_b]: sums over each tile's columns (fp32), or NULL */
  float *colpart[3];        /* [N][nty][W>>b][cout_b]: sums over each tile's rows, or NULL */
} kad_pyramid_args;

/* y_b = conv1x1_b(avg_pool2d(x, 2^b)) + bias_b for every branch from one read
 * of x, plus the LCSA axial partial sums of each y_b.  Stands in for
 * KADConv's per-branch `F.avg_pool2d` + `nn.Conv2d(dim, c, 1)`
 * (kad_conv.py:101,115; reference kadc_fused_parallel.py:74-103 with
 * k_avg_pool_pow2, kadc_fused_sm75.py:707-726) and LCSA's pool_h/pool_w
 * (kad_conv.py:26-27; k_reduce_hconv_bn_relu, kadc_fused_sm75.py:830-888). */
int kad_pyramid_proj(const kad_pyramid_args *a, void *stream);

/* ------------------------------------------------------------------------ */
/* LCSA mask                                                                 */
/* ------------------------------------------------------------------------ */

/* Elements of the fp32 LCSA parameter block for C channels:
 * w1[C][11] | b1[C] | bn_a[C] | bn_b[C] | w3[C][11] | b3[C] | w4[9][C] | b4[9]
 * (bn_a = gamma / sqrt(var + eps), bn_b = beta - mean * bn_a: eval-mode BN). */
int64_t kad_lcsa_params_elems(int c);

/* Elements of the packed projection matrix E[16][11][roundup(C, 32)]. */
int64_t kad_lcsa_emat_elems(int c);

/* Row sums rows[N][H][C] (over w) and column sums cols[N][W][C] (over h) of an
 * NHWC map, one partial slice each: LCSA's pool_h / pool_w numerators
 * (kad_conv.py:26-27,39); reference Triton k_reduce_hw / k_reduce_hconv_bn_relu
 * (acceleration/kadc_fused_sm75.py:800-888).  kad_pyramid_proj produces the
 * same sums as partial slices for KADConv branches. */
int kad_axial_sums(const void *x, float *rows, float *cols, int n, int c, int h, int w, int x_cs, int dtype,
                   void *stream);

/* The same sums of a contiguous NCHW map [N][C][H][W] (x aligned to 4
 * elements), one block per channel plane of at most 12288 pixels: the
 * standalone DSC reads its NCHW input here instead of the NHWC copy. */
int kad_axial_sums_nchw(const void *x, float *rows, float *cols, int n, int c, int h, int w, int dtype, void *stream);

/* kad_axial_sums / kad_axial_sums_nchw followed by kad_lcsa_prep of that one slice, in one
 * launch: arow[N][H][C] = row means and colm[N][W][C] = column means (each sum times 1 / W or
 * 1 / H, the same product kad_lcsa_prep forms; bit-identical).  LCSA's pool_h / pool_w
 * (kad_conv.py:26-27) for a standalone DSC, whose input has no pyramid partial sums. */
int kad_axial_means(const void *x, float *arow, float *colm, int n, int c, int h, int w, int x_cs, int dtype,
                    void *stream);
int kad_axial_means_nchw(const void *x, float *arow, float *colm, int n, int c, int h, int w, int dtype,
                         void *stream);

/* E[j][k][c] = w4[j][c] * w3[c][k] (j < 9, else 0) and ebias[16] = b4 + w4 . b3:
 * the 11x1 depthwise conv and the 1x1 projection of LCSA (kad_conv.py:33-35)
 * fused into one matrix.  emat_dtype KAD_F16 (fp16/bf16 runs) or KAD_F32. */
int kad_lcsa_pack(const float *params, void *emat, float *ebias, int c, int emat_dtype, void *stream);

/* Axial means from sums given as partial slices rows[N][nrp][H][C],
 * cols[N][ncp][W][C]: arow[N][H][C] = sum / W, colm[N][W][C] = sum / H
 * (LCSA's pool_h / pool_w, kad_conv.py:26-27). */
int kad_lcsa_prep(const float *rows, int nrp, const float *cols, int ncp, float *arow, float *colm, int n, int c,
                  int h, int w, void *stream);

/* mask[N][H][W][9] = sigmoid(E * u + ebias) with the strip activation
 * u = relu(bn(a[h] * S(w) + B(w) + b1)) formed from the means and the fp32
 * parameter block (the separable 1x11 conv, BN and ReLU of kad_conv.py:29-32;
 * identity of kadc_fused_sm75.py:861-878), then LCSA's 11x1 conv + 1x1
 * projection + DSC's sigmoid (kad_conv.py:33-35,65) as an MFMA GEMM.  Reference
 * k_vconv_pointwise9* (acceleration/kadc_fused_sm75.py:905-1080) and the RCA tail
 * inside the CUDA DCN kernel (kadc_dcn16_kernel.cu:132-157,219-229). */
int kad_lcsa_mask(const float *arow, const float *colm, const float *params, const void *emat, const float *ebias,
                  float *mask, int n, int c, int h, int w, int emat_dtype, void *stream);

/* kad_lcsa_mask with the channel contraction split over ksplit blocks per
 * 16x16 tile (for small images, whose few tiles would leave most CUs idle):
 * each split writes its raw logits to work[ksplit][N][H][W][9] (fp32,
 * kad_lcsa_mask_work_elems elements; NULL for ksplit = 1), a second launch adds
 * the splits in order, then ebias and the sigmoid (deterministic).
 * kad_lcsa_mask_splits gives the split count used by the fused forwards (1 for
 * shapes with enough tiles).  No reference counterpart (scheduling only). */
int kad_lcsa_mask_splits(int n, int c, int h, int w);
int64_t kad_lcsa_mask_work_elems(int n, int h, int w, int ksplit);
int kad_lcsa_mask_split(const float *arow, const float *colm, const float *params, const void *emat,
                        const float *ebias, float *mask, int n, int c, int h, int w, int emat_dtype, int ksplit,
                        float *work, void *stream);

/* The LCSA stages of several problems (the branches of a KAD-Conv layer) as
 * one launch each: kad_lcsa_prep_group computes every problem's means from its
 * partial sums (kad_lcsa_prep), kad_lcsa_mask_group every problem's mask
 * (kad_lcsa_mask, unsplit), all with one emat dtype.  No reference counterpart
 * (scheduling: one launch instead of three concurrent streams). */
#define KAD_LCSA_GROUP_MAX 4
typedef struct kad_lcsa_args {
  const float *rows;    /* [N][nrp][H][C] partial row sums */
  const float *cols;    /* [N][ncp][W][C] partial column sums */
  int nrp, ncp;
  float *arow;          /* [N][H][C] row means (prep output, mask input) */
  float *colm;          /* [N][W][C] column means */
  const float *params;  /* kad_lcsa_params_elems(C) fp32 block */
  const void *emat;     /* kad_lcsa_pack output */
  const float *ebias;   /* [16] */
  float *mask;          /* [N][H][W][9] */
  int n, c, h, w;
} kad_lcsa_args;
int kad_lcsa_prep_group(const kad_lcsa_args *a, int count, void *stream);
int kad_lcsa_mask_group(const kad_lcsa_args *a, int count, int emat_dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* Squeeze-excitation                                                        */
/* ------------------------------------------------------------------------ */

/* Rows of the partial-sum buffer kad_se_pool writes per image (1 for NCHW). */
int kad_se_pool_tiles(int h, int w, int layout);

/* partial[N][tiles][C] = per-tile channel sums of x (NCHW or NHWC).
 * Reference: GAP inside the DCN kernel / k_gap_only (kadc_dcn16_kernel.cu:270-300;
 * acceleration/kadc_fused_sm75.py:1195-1201). */
int kad_se_pool(const void *x, float *partial, int n, int c, int h, int w, int layout, int x_cs, int dtype,
                void *stream);

/* att[N][C] = sigmoid(W2 relu(W1 (inv_count * sum_t partial[n][t]) + b1) + b2);
 * W1 [hid][C], W2 [C][hid] fp32.  KADConv's `fc` (kad_conv.py:105-109,117);
 * reference k_se_mlp (acceleration/kadc_fused_sm75.py:1518-1542) and
 * gap_se_kernel (kadc_dcn16_kernel.cu:439-497). */
int kad_se_mlp(const float *partial, int tiles, float inv_count, const float *w1, const float *b1, const float *w2,
               const float *b2, float *att, int n, int c, int hid, void *stream);

/* kad_se_mlp with a caller-owned workspace hidden [n][hid] fp32 (its contents on return are
 * the hidden activations relu(W1 g + b1)): each layer runs as one launch spread over the
 * batch's hidden units / channels instead of one block per image (C <= 1024, hid <= 64;
 * other shapes run kad_se_mlp and leave hidden untouched).  Same result as kad_se_mlp up to
 * fp32 summation order.  Same reference as kad_se_mlp (kadc_fused_sm75.py:1518-1542). */
int kad_se_mlp_ws(const float *partial, int tiles, float inv_count, const float *w1, const float *b1,
                  const float *w2, const float *b2, float *att, int n, int c, int hid, float *hidden, void *stream);

/* Layer 1 of kad_se_mlp alone: hidden[n][hid] = relu(W1 (inv_count * sum_t partial[n][t]) + b1)
 * (C <= 1024), one wave per (hidden unit, 4 images).  With kad_se_scale it splits the SE MLP at
 * the hidden layer (kad_conv.py:105-109: Linear, ReLU | Linear, Sigmoid, then y *= att).  Same
 * reference as kad_se_mlp (kadc_fused_sm75.py:1518-1542). */
int kad_se_hidden(const float *partial, int tiles, float inv_count, const float *w1, const float *b1, float *hidden,
                  int n, int c, int hid, void *stream);

/* NCHW out = x * att, att[n][c] = sigmoid(W2[c] . hidden[n] + b2[c]) (also written to att):
 * layer 2 of the SE MLP computed by the blocks of the channel scale for the planes they touch
 * (planes of >= 64 pixels; otherwise a layer-2 launch, then kad_channel_scale; hid <= 64).
 * Reference: the second Linear + Sigmoid of k_se_mlp (kadc_fused_sm75.py:1518-1542) and
 * k_apply_tiled (:1203-1217). */
int kad_se_scale(const void *x, const float *hidden, const float *w2, const float *b2, float *att, void *out, int n,
                 int c, int h, int w, int hid, int dtype, void *stream);

/* The whole SE block over an NCHW x in two launches, x read from HBM once:
 *   g = mean_hw(x), hidden = relu(W1 g + b1), att = sigmoid(W2 hidden + b2), out = x * att.
 * Launch 1: plane means and each 32-channel block's share of W1 g (hpart: n * (C / 32) * 64
 * floats, caller-owned); launch 2: every block forms hidden from its image's shares, then att of
 * its channels (also written to att [n][C]) and the scale, its planes re-read from the L2 of the
 * XCD that read them first.  Fixed-order sums; no state kept between calls.  Needs
 * kad_se_nchw_fits (C % 32 == 0, hid <= 64, H W >= 8).  The reference's k_gap_partial + k_se_mlp
 * + k_apply_tiled (acceleration/kadc_fused_sm75.py:1203-1217,1518-1542) for kad_conv.py:105-109. */
int kad_se_nchw_fits(int n, int c, int h, int w, int hid);
int kad_se_nchw(const void *x, void *out, const float *w1, const float *b1, const float *w2, const float *b2,
                float *att, float *hpart, int n, int c, int h, int w, int hid, int dtype, void *stream);

/* out = x * att[n][c] (NCHW, or NHWC with channel stride x_cs).
 * Reference k_apply_tiled (acceleration/kadc_fused_sm75.py:1203-1217). */
int kad_channel_scale(const void *x, const float *att, void *out, int n, int c, int h, int w, int layout, int x_cs,
                      int dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* Branch merge: bilinear upsample + channel attention + concat + residual   */
/* ------------------------------------------------------------------------ */
/* NCHW [N][C][H][W] -> NHWC [N][H][W][out_cs], channels >= C written 0: the
 * layout the DSC kernels read.  The reference keeps NCHW throughout and has no
 * counterpart; this is the entry used when a caller hands over NCHW tensors. */
int kad_to_nhwc(const void *x, void *out, int n, int c, int h, int w, int out_cs, int dtype, void *stream);

/* Channels-last [N][H][W] with pixel stride x_cs (>= c; a channel slice of a
 * wider buffer, or a dense tensor whose C is not a multiple of 8) -> NHWC with
 * channel stride out_cs (a multiple of 8), channels >= c written 0.  Replaces the two passes (a dense copy, then kad_to_nhwc) that a
 * channels-last input of C % 8 != 0 needed.  Like kad_to_nhwc it has no
 * counterpart in the reference, which keeps NCHW. */
int kad_nhwc_pad(const void *x, int x_cs, void *out, int out_cs, int n, int c, int h, int w, int dtype, void *stream);

#define KAD_MAX_BRANCHES 4

typedef struct kad_merge_args {
  void *out;               /* [N][C][H][W] (NCHW) or [N][H][W][C] (NHWC), dtype */
  const void *residual;    /* same layout as out, or NULL */
  const float *gate;       /* [C] per-channel output multiplier, or NULL */
  int n, c, h, w, layout, dtype, nbranch;
  int c_begin, c_end;      /* output channels written: [c_begin, c_end); 0, 0 = all of [0, C) */
  const void *br_z[KAD_MAX_BRANCHES];    /* NHWC [N][h_b][w_b][cs_b], dtype */
  const float *br_att[KAD_MAX_BRANCHES]; /* [N][c_b] or NULL */
  int br_c[KAD_MAX_BRANCHES], br_c_off[KAD_MAX_BRANCHES];
  int br_h[KAD_MAX_BRANCHES], br_w[KAD_MAX_BRANCHES], br_cs[KAD_MAX_BRANCHES];
  float br_coeff[KAD_MAX_BRANCHES];
  int out_cs, res_cs;      /* NHWC only: pixel strides (elements) of out and residual; 0 = c.  Lets
                              the output be a channel slice of a wider buffer (a concat).  NCHW: 0 */
} kad_merge_args;

/* out[n, c] = gate[c] * (residual + sum over branches b with c in [c_off_b, c_off_b + c_b):
 *   coeff_b * att_b[n, c - c_off_b] * bilinear_up(z_b)[c - c_off_b])
 * for c in [c_begin, c_end); other channels of out are not touched, so one
 * call per branch can merge each branch as soon as it is ready.
 * KADConv's tail `F.interpolate(..., align_corners=False)`, `torch.cat` and `+ x`
 * (kad_conv.py:117-121); reference k_upsample_bilinear_att + k_cat_residual_att0
 * (acceleration/kadc_fused_sm75.py:1245-1331). */
int kad_branch_merge(const kad_merge_args *a, void *stream);

/* In place, for the full-resolution branch whose DSC wrote its output straight
 * into channels [c_off, c_off + c) of out (img_c channels per image):
 *   out[n, c_off + j] = att[n, j] * out[n, c_off + j] + residual[n, c_off + j].
 * residual has out's layout and shape (or NULL).  The reference's
 * k_cat_residual_att0 (acceleration/kadc_fused_sm75.py:1245-1331) for branch 0. */
int kad_scale_residual(void *out, const float *att, const void *residual, int n, int c, int h, int w, int img_c,
                       int c_off, int layout, int dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* KAD-CNet-S network ops (NHWC feature maps with explicit channel strides)  */
/* ------------------------------------------------------------------------ */

/* Plain 3x3 convolution (stride <= 2) whose output has the op's dtype, on the
 * kad_dcn_args machinery (offset / mask ignored): KAD-CNet's `Conv` with k = 3
 * after Conv-BN fusion, act(W * x + b) (KAD-CNet/models/common.py:43-57,
 * fused by yolo.py:574-585).  a->relu selects the activation: 0 none,
 * 1 ReLU, 2 SiLU (x * sigmoid(x), the `Conv.default_act`).  Grouped convs are
 * passed with block-diagonal dense weights.  The reference runs these on
 * cuDNN (KAD-CNet/inference/acceleration/kadc_fused_sm75.py:616-629). */
int kad_conv_fwd(const kad_dcn_args *a, void *stream);

/* The network's stem: the same 3x3 Conv for an NCHW image with 1-3 channels,
 * read as it is (x: [N][Cin][H][W] contiguous, 16-bit; x_cs ignored) and written
 * NHWC (out_cs), so the input needs no channels-last copy.  pad 1, stride 1 or 2,
 * Cout <= 64, W a multiple of 8; bias and activation only (post_* NULL).
 * Weights packed by kad_dcn_pack_weights.  Stands in for the first Conv of
 * KAD-CNet (models/common.py:43-57, `Conv(3, c, 3, 2)` of the yaml's first
 * row), run by cuDNN in the reference (kadc_fused_sm75.py:616-629). */
int kad_stem_conv_fwd(const kad_dcn_args *a, void *stream);

#define KAD_RS_AVG 0      /* average pool, zero padding counted (count_include_pad=True) */
#define KAD_RS_MAX 1      /* max pool, padding ignored */
#define KAD_RS_NEAREST 2  /* nearest upsample by the integer factor s: out[y][x] = in[y / s][x / s] */
#define KAD_RS_MAX3 3     /* SPPELAN's chain of three max pools (k odd, s = 1, p = k / 2, ho = h, wo = w):
                             out channels [0, c) = pool(x), [c, 2c) = pool(pool(x)), [2c, 3c) =
                             pool(pool(pool(x))) in one call (out_cs >= 3 c) */

typedef struct kad_resample_args {
  const void *x;         /* NHWC [N][H][W][x_cs], dtype (channels [0, c) used) */
  void *out;             /* NHWC [N][Ho][Wo][out_cs], dtype (channels [0, c) written) */
  int n, c, h, w, ho, wo, x_cs, out_cs;
  int mode;              /* KAD_RS_* */
  int k, s, p;           /* pool: kernel, stride, padding (floor mode); nearest: s = factor */
  int dtype;
} kad_resample_args;

/* Pools, nearest upsampling and channel-slice copies (k = s = 1, p = 0, AVG) of
 * NHWC maps, reading and writing channel slices of wider tensors in place.
 * Stands in for AConv's avg_pool2d(x, 2, 1, 0) (KAD-CNet/models/common.py:65-67),
 * SPPELAN's max pools (common.py:187-193,563-577), the neck's
 * nn.Upsample(None, 2, 'nearest') and torch.cat (common.py:535-542), and the
 * reference's Triton helpers for them (acceleration/kadc_fused_sm75.py:197-430). */
int kad_nhwc_resample(const kad_resample_args *a, void *stream);

#define KAD_MAX_LEVELS 4
typedef struct kad_decode_args {
  const void *head[KAD_MAX_LEVELS]; /* level l: NHWC [N][lh][lw][head_cs], box logits in channels
                                       [0, 4 * reg_max) (side j's bins at reg_max * j + b), class
                                       logits in [box_ch, box_ch + nc) */
  int lh[KAD_MAX_LEVELS], lw[KAD_MAX_LEVELS], head_cs[KAD_MAX_LEVELS];
  int anchor_off[KAD_MAX_LEVELS];   /* first anchor of level l (levels in order, cells row-major) */
  float stride[KAD_MAX_LEVELS];
  void *out;                        /* [N][4 + nc][A], dtype: (cx, cy, w, h) * stride, then sigmoid(cls) */
  int n, nl, nc, reg_max, box_ch, dtype;
} kad_decode_args;

/* DDetect's inference output y = cat(dist2bbox(DFL(box), anchors, xywh) * strides,
 * sigmoid(cls)) for all levels (KAD-CNet/models/yolo.py:102-127; DFL
 * models/common.py:232-244; make_anchors / dist2bbox
 * utils/tal/anchor_generator.py:8-32, grid offset 0.5).  The reference's
 * fused Triton decode is KAD-CNet/inference/acceleration/kadc_head_decode.py:9-88. */
int kad_ddetect_decode(const kad_decode_args *a, void *stream);

#define KAD_NMS_MAX 32768
/* 64-bit words of the pairwise suppression mask kad_nms needs for n boxes. */
int64_t kad_nms_mask_words(int n);

/* Greedy non-maximum suppression of n <= KAD_NMS_MAX boxes [n][4] (x1, y1, x2,
 * y2, fp32) already sorted by descending score: keep[i] = 1 when no kept box
 * before i has IoU > iou_thr with box i (IoU = inter / (area_i + area_j - inter),
 * fp32), else 0.  mask: kad_nms_mask_words(n) words of caller scratch.  The
 * torchvision.ops.nms call of non_max_suppression (KAD-CNet/utils/general.py:961). */
int kad_nms(const float *boxes, unsigned long long *mask, unsigned char *keep, int n, float iou_thr, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KADCONV_HIP_H_ */
