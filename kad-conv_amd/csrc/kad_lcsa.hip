// LCSA (Low-Cost Spatial Attention), the mask generator of DSC:
//   mask = sigmoid( conv1x1_{C->9}( dwconv_{11x1}( relu(bn( dwconv_{1x11}( mean_w(x)[h] + mean_h(x)[w] ))))))
// (KAD-Conv/kadconv/kad_conv.py:18-39, 65; twin RCA in KAD-CNet/models/module/ops.py:12-37).
//
// The broadcast sum s[h, w] = a[h] + b[w] never exists here.  The 1x11
// depthwise conv of it is separable (the reference's fast path uses the same
// identity, acceleration/kadc_fused_sm75.py:861-878):
//   t[c, h, w] = a[c, h] * S_c(w) + B_c(w) + b1[c],
//   S_c(w) = sum of the taps that land inside the row, B_c(w) = (w1 * b)(w).
// So the only full-resolution work is u = relu(bn(t)) (3 ops), the 11-tap
// vertical conv and the 9 x C projection, done per image column in LDS.
//
// Two kernels: kad_axial_means reads the NHWC feature map once and writes the
// row means a[n, h, c] and column means b[n, w, c]; kad_lcsa_mask turns them
// into the fp32 mask [N, H, W, 9] (pixel-major, sigmoid applied).
#include "kad_common.h"

namespace kad {

constexpr int AX_THREADS = 256;

// grid.x = H + W lines, grid.y = N.  Line l < H is row l (mean over w);
// otherwise column l - H (mean over h).  Threads stride over channels, so each
// step reads consecutive channels of one pixel (coalesced in NHWC).
template <typename T>
__global__ __launch_bounds__(AX_THREADS) void axial_means_kernel(const T* x, float* rowm, float* colm, int c, int h,
                                                                int w, int cs) {
  const int n = blockIdx.y;
  const int l = blockIdx.x;
  const T* base = x + (int64_t)n * h * w * cs;
  if (l < h) {
    const float inv = 1.f / (float)w;
    for (int ch = threadIdx.x; ch < c; ch += AX_THREADS) {
      float acc = 0.f;
      const T* p = base + (int64_t)l * w * cs + ch;
      for (int j = 0; j < w; ++j) acc += to_f32(p[(int64_t)j * cs]);
      rowm[((int64_t)n * h + l) * c + ch] = acc * inv;
    }
  } else {
    const int col = l - h;
    const float inv = 1.f / (float)h;
    for (int ch = threadIdx.x; ch < c; ch += AX_THREADS) {
      float acc = 0.f;
      const T* p = base + (int64_t)col * cs + ch;
      for (int i = 0; i < h; ++i) acc += to_f32(p[(int64_t)i * w * cs]);
      colm[((int64_t)n * w + col) * c + ch] = acc * inv;
    }
  }
}

// Parameter block layout (fp32), built once by the host from the LCSA weights:
//   w1[C][11] | b1[C] | bn_a[C] | bn_b[C] | w3[C][11] | b3[C] | w4[9][C] | b4[9]
// with bn_a = gamma / sqrt(var + eps), bn_b = beta - mean * bn_a (eval-mode BN).
struct LcsaParams {
  const float *w1, *b1, *bna, *bnb, *w3, *b3, *w4, *b4;
  __device__ LcsaParams(const float* p, int c)
      : w1(p), b1(p + 11 * c), bna(p + 12 * c), bnb(p + 13 * c), w3(p + 14 * c), b3(p + 25 * c),
        w4(p + 26 * c), b4(p + 35 * c) {}
};

constexpr int LM_THREADS = 256;
constexpr int BAND = 11;
constexpr int HALF_BAND = 5;

// grid = (W, N).  One block per image column; rows processed in chunks of hc
// so that u [(hc + 10) x C] and v [hc x C] fit the dynamic LDS budget.
__global__ __launch_bounds__(LM_THREADS) void lcsa_mask_kernel(const float* rowm, const float* colm,
                                                              const float* params, float* mask, int c, int h,
                                                              int w, int hc) {
  extern __shared__ float lds[];
  const int col = blockIdx.x;
  const int n = blockIdx.y;
  const LcsaParams prm(params, c);
  float* sS = lds;             // [C]
  float* sB = sS + c;          // [C]
  float* u = sB + c;           // [(hc + 10)][C]
  float* v = u + (hc + 2 * HALF_BAND) * c;  // [hc][C]
  const float* bcol = colm + (int64_t)n * w * c;
  for (int ch = threadIdx.x; ch < c; ch += LM_THREADS) {
    float S = 0.f, B = 0.f;
#pragma unroll
    for (int k = 0; k < BAND; ++k) {
      const int ww = col + k - HALF_BAND;
      if (ww >= 0 && ww < w) {
        const float wk = prm.w1[ch * BAND + k];
        S += wk;
        B += wk * bcol[(int64_t)ww * c + ch];
      }
    }
    sS[ch] = S;
    sB[ch] = B + prm.b1[ch];
  }
  __syncthreads();
  const float* arow = rowm + (int64_t)n * h * c;
  for (int h0 = 0; h0 < h; h0 += hc) {
    const int rows = (h - h0) < hc ? (h - h0) : hc;
    const int urows = rows + 2 * HALF_BAND;
    // u for rows [h0 - 5, h0 + rows + 5); rows outside the image are the vertical conv's zero padding
    for (int e = threadIdx.x; e < urows * c; e += LM_THREADS) {
      const int r = e / c, ch = e - (e / c) * c;
      const int hh = h0 - HALF_BAND + r;
      float val = 0.f;
      if (hh >= 0 && hh < h) {
        const float t = arow[(int64_t)hh * c + ch] * sS[ch] + sB[ch];
        val = fmaxf(t * prm.bna[ch] + prm.bnb[ch], 0.f);
      }
      u[r * c + ch] = val;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < rows * c; e += LM_THREADS) {
      const int r = e / c, ch = e - (e / c) * c;
      float acc = prm.b3[ch];
#pragma unroll
      for (int k = 0; k < BAND; ++k) acc += prm.w3[ch * BAND + k] * u[(r + k) * c + ch];
      v[r * c + ch] = acc;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < rows * 9; e += LM_THREADS) {
      const int r = e / 9, j = e - (e / 9) * 9;
      float acc = prm.b4[j];
      const float* wj = prm.w4 + j * c;
      const float* vr = v + r * c;
      for (int ch = 0; ch < c; ++ch) acc += wj[ch] * vr[ch];
      mask[(((int64_t)n * h + h0 + r) * w + col) * 9 + j] = sigmoidf_(acc);
    }
    __syncthreads();
  }
}

}  // namespace kad

using namespace kad;

extern "C" int64_t kad_lcsa_params_elems(int c) { return c > 0 ? 35 * (int64_t)c + 9 : 0; }

extern "C" int kad_axial_means(const void* x, float* rowm, float* colm, int n, int c, int h, int w, int x_cs,
                               int dtype, void* stream) {
  KAD_CHECK_ARG(x && rowm && colm, "kad_axial_means: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0 && x_cs >= c, "kad_axial_means: bad shape");
  dim3 grid(h + w, n);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case KAD_F32: hipLaunchKernelGGL(axial_means_kernel<float>, grid, dim3(AX_THREADS), 0, st, (const float*)x, rowm, colm, c, h, w, x_cs); break;
    case KAD_F16: hipLaunchKernelGGL(axial_means_kernel<half_t>, grid, dim3(AX_THREADS), 0, st, (const half_t*)x, rowm, colm, c, h, w, x_cs); break;
    case KAD_BF16: hipLaunchKernelGGL(axial_means_kernel<bf16_t>, grid, dim3(AX_THREADS), 0, st, (const bf16_t*)x, rowm, colm, c, h, w, x_cs); break;
    default: return fail(KAD_EINVAL, "kad_axial_means: unknown dtype %d", dtype);
  }
  return check_launch("kad_axial_means");
}

extern "C" int kad_lcsa_mask(const float* rowm, const float* colm, const float* params, float* mask, int n, int c,
                             int h, int w, void* stream) {
  KAD_CHECK_ARG(rowm && colm && params && mask, "kad_lcsa_mask: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0, "kad_lcsa_mask: bad shape");
  // LDS budget 48 KB: (2C + (2 hc + 10) C) floats
  const int budget = 48 * 1024 / 4;
  int hc = (budget / c - 2 - 2 * HALF_BAND) / 2;
  KAD_CHECK_ARG(hc >= 1, "kad_lcsa_mask: C=%d too large for one LDS column", c);
  if (hc > h) hc = h;
  const size_t lds = (size_t)(2 * c + (2 * hc + 2 * HALF_BAND) * c) * sizeof(float);
  hipLaunchKernelGGL(lcsa_mask_kernel, dim3(w, n), dim3(LM_THREADS), lds, (hipStream_t)stream, rowm, colm, params,
                     mask, c, h, w, hc);
  return check_launch("kad_lcsa_mask");
}
