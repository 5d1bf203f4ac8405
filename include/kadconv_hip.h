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
 *  - no mutable global state: calls from different host threads on different
 *    streams do not interfere.
 */
#ifndef KADCONV_HIP_H_
#define KADCONV_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KAD_ABI_VERSION 1

/* element types */
#define KAD_F32 0
#define KAD_F16 1
#define KAD_BF16 2

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
  int64_t off_sn, off_sp, off_sc;
  int64_t mask_sn, mask_sp, mask_sc;
  int n, cin, cout, h, w, stride, pad;
  int x_cs;               /* channel stride of x (multiple of 8; >= Cin) */
  int out_layout;         /* KAD_NHWC or KAD_NCHW */
  int out_cs;             /* channel stride of out for NHWC (>= Cout) */
  int dtype;              /* KAD_F32 / KAD_F16 / KAD_BF16 (x, wpack, out) */
  int relu;               /* nonzero: ReLU between post_add and post_scale */
} kad_dcn_args;

/* out = post_scale * act((deform_conv3x3(x, offset, mask, W) + bias) * post_mul + post_add).
 * Stands in for kadc_dcn16.cpp:247-289 `forward*`/`forward_*_unsafe`
 * (kernel kadc_dcn16_kernel.cu:92-314) and for torchvision.ops.deform_conv2d
 * as called at KAD-Conv/kadconv/kad_conv.py:66-67. */
int kad_dcn_fwd(const kad_dcn_args *a, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KADCONV_HIP_H_ */
