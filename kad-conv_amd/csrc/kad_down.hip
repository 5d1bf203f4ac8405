// KADDown input pass: the three pooled branch inputs at the output
// resolution, stacked along channels, so that the whole op is this pass plus
// one 1x1 GEMM.
//
// KADDown (builder-defined; no reference operator, definition in
// oracle/kadconv_oracle.py:kaddown_forward) is
//     y = sigmoid(gate) * sum_b softmax(alpha)_b * up_b(conv1x1_b(avgpool(x, 2^(b+1))))
// with up_b bilinear (align_corners=False) to (H/2, W/2), identity for b = 0.
// A 1x1 convolution commutes with a bilinear resize (the resize weights of an
// output pixel sum to 1, so the bias passes through), hence
//     y = [g a_0 W_0 | g a_1 W_1 | g a_2 W_2] . [p2; up(p4); up(p8)] + g sum_b a_b b_b
// with g = sigmoid(gate) per output channel and p_s = avgpool(x, s): one GEMM
// with K = 3 C over the stacked input u built here.  The GEMM does 2.3x the
// branch-resolution flops (branches 1 and 2 at H/2 x W/2), but no partial
// outputs are written, re-read and merged.
//
// One block per (image, channel) plane: the 2x2 means p2 are formed from the
// plane's input rows (8-byte reads when W % 4 == 0) and kept in LDS as fp32;
// p4 = 2x2 means of p2 and p8 = 2x2 means of p4 (floor(H/4) = floor(floor(H/2)/2),
// likewise for 8, so these equal avg_pool2d of x with kernel 4 and 8); then the
// resized planes are written.  HBM traffic per plane: H W reads, nb (H/2)(W/2)
// writes.
#include "kad_common.h"

namespace kad {

constexpr int KD_THREADS = 256;
constexpr int KD_MAX_LDS = 160 * 1024;

// VEC: W % 4 == 0, Wo even and both pointers aligned to their vector width.
template <typename T, bool VEC>
__global__ __launch_bounds__(KD_THREADS) void kaddown_prep_kernel(const T* __restrict__ x, T* __restrict__ u, int C,
                                                                  int H, int W, int nb) {
  extern __shared__ __align__(16) float ksm[];
  const int Ho = H >> 1, Wo = W >> 1, H4 = H >> 2, W4 = W >> 2, H8 = H >> 3, W8 = W >> 3;
  const int P = Ho * Wo;
  float* p2 = ksm;
  float* p4 = p2 + P;
  float* p8 = p4 + H4 * W4;
  const int plane = blockIdx.x, n = plane / C, c = plane - n * C;
  const T* xp = x + (int64_t)plane * H * W;
  T* ub = u + ((int64_t)n * nb * C + c) * P;  // branch b plane at ub + b C P
  const int tid = threadIdx.x;

  // ---- p2 = 2x2 means (branch 0 output as is) ---------------------------------------------------------
  if constexpr (VEC) {  // two outputs per step from 4-element input pieces, 2-element output pairs
    typedef T t4 __attribute__((ext_vector_type(4)));
    typedef T t2 __attribute__((ext_vector_type(2)));
    // batches of KU steps per thread: every load of a batch is issued before the first use
    // (one round trip per batch; a 100 x 100 plane is one batch)
    constexpr int KU = 8;
    for (int t0 = tid; t0 < P / 2; t0 += KU * KD_THREADS) {
      t4 r0[KU], r1[KU];
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const int t = t0 + u * KD_THREADS;
        if (t < P / 2) {
          const int i = 2 * t, y = i / Wo, xo = i - y * Wo;
          r0[u] = *(const t4*)(xp + (2 * y) * W + 2 * xo);
          r1[u] = *(const t4*)(xp + (2 * y + 1) * W + 2 * xo);
        }
      }
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const int t = t0 + u * KD_THREADS;
        if (t < P / 2) {
          const int i = 2 * t;
          const float v0 = 0.25f * ((to_f32(r0[u][0]) + to_f32(r0[u][1])) + (to_f32(r1[u][0]) + to_f32(r1[u][1])));
          const float v1 = 0.25f * ((to_f32(r0[u][2]) + to_f32(r0[u][3])) + (to_f32(r1[u][2]) + to_f32(r1[u][3])));
          p2[i] = v0;
          p2[i + 1] = v1;
          t2 o;
          o[0] = from_f32<T>(v0);
          o[1] = from_f32<T>(v1);
          *(t2*)(ub + i) = o;
        }
      }
    }
  } else {
    for (int i = tid; i < P; i += KD_THREADS) {
      const int y = i / Wo, xo = i - y * Wo;
      const T* r0 = xp + (2 * y) * W + 2 * xo;
      const float v = 0.25f * ((to_f32(r0[0]) + to_f32(r0[1])) + (to_f32(r0[W]) + to_f32(r0[W + 1])));
      p2[i] = v;
      ub[i] = from_f32<T>(v);
    }
  }
  if (nb < 2) return;
  __syncthreads();
  for (int i = tid; i < H4 * W4; i += KD_THREADS) {
    const int y = i / W4, xo = i - y * W4;
    const float* r = p2 + (2 * y) * Wo + 2 * xo;
    p4[i] = 0.25f * ((r[0] + r[1]) + (r[Wo] + r[Wo + 1]));
  }
  __syncthreads();
  if (nb > 2) {
    for (int i = tid; i < H8 * W8; i += KD_THREADS) {
      const int y = i / W8, xo = i - y * W8;
      const float* r = p4 + (2 * y) * W4 + 2 * xo;
      p8[i] = 0.25f * ((r[0] + r[1]) + (r[W4] + r[W4 + 1]));
    }
    __syncthreads();
  }
  // ---- bilinear resize of p4 (and p8) to Ho x Wo --------------------------------------------------------
  // A wave walks output rows (its lanes along the row's columns), so a row's source rows and weight
  // are wave-uniform; each lane's source columns and weights are computed once per column.  Same
  // formulas and order of operations as per-pixel src_index.
  const float sy4 = (float)H4 / (float)Ho, sx4 = (float)W4 / (float)Wo;
  const float sy8 = (float)H8 / (float)Ho, sx8 = (float)W8 / (float)Wo;
  const int lane = tid & 63, wave = tid >> 6;
  for (int x0c = 0; x0c < Wo; x0c += 64) {
    const int xo = x0c + lane;
    const bool col_ok = xo < Wo;
    int ax0, ax1, bx0 = 0, bx1 = 0;
    float alx, blx = 0.f;
    src_index(col_ok ? xo : 0, W4, Wo, sx4, ax0, ax1, alx);
    if (nb > 2) src_index(col_ok ? xo : 0, W8, Wo, sx8, bx0, bx1, blx);
    for (int y = wave; y < Ho; y += KD_THREADS / 64) {
      int y0, y1;
      float ly;
      src_index(y, H4, Ho, sy4, y0, y1, ly);
      const float* r0 = p4 + y0 * W4;
      const float* r1 = p4 + y1 * W4;
      const float v4 = (1.f - ly) * ((1.f - alx) * r0[ax0] + alx * r0[ax1]) +
                       ly * ((1.f - alx) * r1[ax0] + alx * r1[ax1]);
      float v8 = 0.f;
      if (nb > 2) {
        src_index(y, H8, Ho, sy8, y0, y1, ly);
        const float* s0 = p8 + y0 * W8;
        const float* s1 = p8 + y1 * W8;
        v8 = (1.f - ly) * ((1.f - blx) * s0[bx0] + blx * s0[bx1]) + ly * ((1.f - blx) * s1[bx0] + blx * s1[bx1]);
      }
      if (col_ok) {
        const int i = y * Wo + xo;
        ub[(int64_t)C * P + i] = from_f32<T>(v4);
        if (nb > 2) ub[(int64_t)2 * C * P + i] = from_f32<T>(v8);
      }
    }
  }
}

static size_t kd_lds(int h, int w) {
  return (size_t)((h >> 1) * (w >> 1) + (h >> 2) * (w >> 2) + (h >> 3) * (w >> 3)) * sizeof(float);
}

template <typename T>
static int launch_kaddown_prep(const void* x, void* u, int n, int c, int h, int w, int nb, hipStream_t st) {
  const size_t lds = kd_lds(h, w);
  const bool vec = w % 4 == 0 && (w >> 1) % 2 == 0 && (uintptr_t)x % (4 * sizeof(T)) == 0 &&
                   (uintptr_t)u % (2 * sizeof(T)) == 0;
  if (vec) {
    allow_lds(kaddown_prep_kernel<T, true>, lds);
    hipLaunchKernelGGL((kaddown_prep_kernel<T, true>), dim3(n * c), dim3(KD_THREADS), lds, st, (const T*)x, (T*)u, c,
                       h, w, nb);
  } else {
    allow_lds(kaddown_prep_kernel<T, false>, lds);
    hipLaunchKernelGGL((kaddown_prep_kernel<T, false>), dim3(n * c), dim3(KD_THREADS), lds, st, (const T*)x, (T*)u, c,
                       h, w, nb);
  }
  return check_launch("kad_kaddown_prep");
}

}  // namespace kad

using namespace kad;

extern "C" int kad_kaddown_prep(const void* x, void* u, int n, int c, int h, int w, int nb, int dtype, void* stream) {
  KAD_CHECK_ARG(x && u, "kad_kaddown_prep: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && nb >= 1 && nb <= 3, "kad_kaddown_prep: bad n=%d c=%d nb=%d", n, c, nb);
  KAD_CHECK_ARG(h >= (1 << nb) && w >= (1 << nb), "kad_kaddown_prep: %dx%d is smaller than the %d-pixel pool of branch %d",
                h, w, 1 << nb, nb - 1);
  KAD_CHECK_ARG(kd_lds(h, w) <= (size_t)KD_MAX_LDS,
                "kad_kaddown_prep: %dx%d planes exceed the LDS staging limit (%d bytes of fp32 pools)", h, w,
                KD_MAX_LDS);
  KAD_CHECK_ARG((int64_t)n * c < (1ll << 31), "kad_kaddown_prep: too many planes");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case KAD_F32: return launch_kaddown_prep<float>(x, u, n, c, h, w, nb, st);
    case KAD_F16: return launch_kaddown_prep<half_t>(x, u, n, c, h, w, nb, st);
    case KAD_BF16: return launch_kaddown_prep<bf16_t>(x, u, n, c, h, w, nb, st);
    default: return fail(KAD_EINVAL, "kad_kaddown_prep: unknown dtype %d", dtype);
  }
}
