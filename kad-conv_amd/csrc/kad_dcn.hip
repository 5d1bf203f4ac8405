// Modulated deformable 3x3 convolution (DCNv2) fused into an MFMA GEMM.
//
// Semantics: torchvision.ops.deform_conv2d as called by DSC.forward
// (KAD-Conv/kadconv/kad_conv.py:63-67), one offset group; sampling rule as
// restated by the reference at acceleration/kadc_dcn_direct.py:57-107: a
// sample is 0 when py <= -1, py >= H, px <= -1 or px >= W, else the four
// corners around floor(p) are blended and corners outside the image read 0.
// The BatchNorm/ReLU/branch-scale epilogue and the per-tile GAP partial sums
// that the reference fuses into its CUDA kernel (kadc_dcn16_kernel.cu:45-90,
// 270-300) are fused here too, with deterministic partials instead of float
// atomics.
//
// GEMM view: out[p, co] = sum_k S[p, k] * Wt[k, co] with k = (chunk, tap, c32),
// M = output pixels, N = Cout, K = 9 * roundup(Cin, 32).
//   * A operand (S, the modulated bilinear samples) is built directly in
//     registers in the MFMA A-fragment layout: lane (row r = lane & 15,
//     k-group g = lane >> 4) gathers 8 consecutive channels of one (pixel, tap)
//     from the NHWC input (four 16-byte corner loads) and blends them.
//   * B operand (weights) is read from the packed [Cout_pad][Cin_pad/32][9][32]
//     buffer, 16 contiguous bytes per lane.
//   * Per-(pixel, tap) bilinear corner indices and weights (mask and validity
//     folded in) are computed once per block into LDS.
// Any consistent assignment of k to (lane group, slot) gives the same dot
// product, so A and B only have to agree with each other; the accumulator
// layout (lane -> column lane & 15, rows 4 * (lane >> 4) + i) is the MFMA
// output layout.
#include "kad_common.h"

namespace kad {

constexpr int DCN_TILE = 128;   // output pixels per block (flattened, one image)
constexpr int DCN_THREADS = 256;
constexpr int DCN_WM = 2;       // 16-pixel A fragments per wave (4 waves x 2 x 16 = 128)

struct __align__(16) SampleInfo {
  int idx[4];    // corner pixel indices y*W+x (clamped in-image; weight 0 when invalid)
  float w[4];    // bilinear weight * mask, 0 for corners outside the image
};

// ---- per-dtype fragment helpers ------------------------------------------------
template <typename T> struct DcnOps;

template <> struct DcnOps<half_t> {
  typedef half8_t frag;
  template <bool PLAIN>
  static __device__ __forceinline__ frag gather(const half_t* base, const SampleInfo& s, int cs, int ch, bool ok) {
    if (!ok) return frag{};
    if (PLAIN) return *(const frag*)(base + (int64_t)s.idx[0] * cs + ch) * (half_t)s.w[0];
    const half_t* p0 = base + (int64_t)s.idx[0] * cs + ch;
    const half_t* p1 = base + (int64_t)s.idx[1] * cs + ch;
    const half_t* p2 = base + (int64_t)s.idx[2] * cs + ch;
    const half_t* p3 = base + (int64_t)s.idx[3] * cs + ch;
    frag v0 = *(const frag*)p0, v1 = *(const frag*)p1, v2 = *(const frag*)p2, v3 = *(const frag*)p3;
    frag r = v0 * (half_t)s.w[0];
    r += v1 * (half_t)s.w[1];
    r += v2 * (half_t)s.w[2];
    r += v3 * (half_t)s.w[3];
    return r;
  }
  static __device__ __forceinline__ frag load_b(const half_t* p) { return *(const frag*)p; }
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct DcnOps<bf16_t> {
  typedef bf16x8_t frag;
  template <bool PLAIN>
  static __device__ __forceinline__ frag gather(const bf16_t* base, const SampleInfo& s, int cs, int ch, bool ok) {
    if (!ok) return frag{};
    if (PLAIN) {
      frag v = *(const frag*)(base + (int64_t)s.idx[0] * cs + ch);
      return s.w[0] != 0.f ? v : frag{};
    }
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      frag v = *(const frag*)(base + (int64_t)s.idx[c] * cs + ch);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += s.w[c] * (float)v[j];
    }
    frag r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (bf16_t)acc[j];
    return r;
  }
  static __device__ __forceinline__ frag load_b(const bf16_t* p) { return *(const frag*)p; }
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

struct f32x8 { floatx4 lo, hi; };

template <> struct DcnOps<float> {
  typedef f32x8 frag;
  template <bool PLAIN>
  static __device__ __forceinline__ frag gather(const float* base, const SampleInfo& s, int cs, int ch, bool ok) {
    frag r;
    r.lo = floatx4{0.f, 0.f, 0.f, 0.f};
    r.hi = r.lo;
    if (!ok) return r;
#pragma unroll
    for (int c = 0; c < (PLAIN ? 1 : 4); ++c) {
      const float* p = base + (int64_t)s.idx[c] * cs + ch;
      floatx4 a = *(const floatx4*)p;
      floatx4 b = *(const floatx4*)(p + 4);
      r.lo += a * s.w[c];
      r.hi += b * s.w[c];
    }
    return r;
  }
  static __device__ __forceinline__ frag load_b(const float* p) {
    frag r;
    r.lo = *(const floatx4*)p;
    r.hi = *(const floatx4*)(p + 4);
    return r;
  }
  // 8 MFMA steps of k=4: step j consumes slot j of every lane group, i.e.
  // k = 8 * group + j on both operands.
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[j], b.lo[j], c, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[j], b.hi[j], c, 0, 0, 0);
    return c;
  }
};

// ---- kernel ------------------------------------------------------------------------
// PLAIN = true computes an ordinary 3x3 convolution (integer taps, no
// offsets or mask): used for DSC's offset branch, conv_offset (kad_conv.py:55-56).
template <typename T, typename OutT, int NBF, bool PLAIN>
__global__ __launch_bounds__(DCN_THREADS) void dcn_fwd_kernel(kad_dcn_args a, int ho, int wo, int tiles,
                                                             int nchunk, int cout_pad) {
  typedef DcnOps<T> Ops;
  typedef typename Ops::frag frag;
  __shared__ SampleInfo si[9][DCN_TILE];
  __shared__ float gap_red[4][NBF * 16];

  const int tile = blockIdx.x;
  const int co0 = blockIdx.y * NBF * 16;
  const int n = blockIdx.z;
  const int P = ho * wo;
  const int p0 = tile * DCN_TILE;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // ---- prologue: bilinear corners/weights per (tap, pixel) -------------------------
  for (int q = tid; q < 9 * DCN_TILE; q += DCN_THREADS) {
    const int k = q / DCN_TILE;
    const int pl = q - k * DCN_TILE;
    const int p = p0 + pl;
    SampleInfo s;
    s.idx[0] = s.idx[1] = s.idx[2] = s.idx[3] = 0;
    s.w[0] = s.w[1] = s.w[2] = s.w[3] = 0.f;
    if (p < P && PLAIN) {
      const int oy = p / wo, ox = p - (p / wo) * wo;
      const int iy = oy * a.stride - a.pad + k / 3, ix = ox * a.stride - a.pad + (k - (k / 3) * 3);
      if (iy >= 0 && iy < a.h && ix >= 0 && ix < a.w) {
        s.idx[0] = iy * a.w + ix;
        s.w[0] = 1.f;
      }
    } else if (p < P) {
      const int oy = p / wo, ox = p - (p / wo) * wo;
      const int ky = k / 3, kx = k - (k / 3) * 3;
      const float dy = a.offset[n * a.off_sn + (int64_t)p * a.off_sp + (2 * k) * a.off_sc];
      const float dx = a.offset[n * a.off_sn + (int64_t)p * a.off_sp + (2 * k + 1) * a.off_sc];
      const float m = a.mask ? a.mask[n * a.mask_sn + (int64_t)p * a.mask_sp + k * a.mask_sc] : 1.f;
      const float py = (float)(oy * a.stride - a.pad + ky) + dy;
      const float px = (float)(ox * a.stride - a.pad + kx) + dx;
      if (py > -1.f && py < (float)a.h && px > -1.f && px < (float)a.w) {
        const float fy = floorf(py), fx = floorf(px);
        const int y0 = (int)fy, x0 = (int)fx, y1 = y0 + 1, x1 = x0 + 1;
        const float ly = py - fy, lx = px - fx, hy = 1.f - ly, hx = 1.f - lx;
        const bool vy0 = y0 >= 0, vy1 = y1 <= a.h - 1, vx0 = x0 >= 0, vx1 = x1 <= a.w - 1;
        const int cy0 = vy0 ? y0 : 0, cy1 = vy1 ? y1 : a.h - 1;
        const int cx0 = vx0 ? x0 : 0, cx1 = vx1 ? x1 : a.w - 1;
        s.idx[0] = cy0 * a.w + cx0;
        s.idx[1] = cy0 * a.w + cx1;
        s.idx[2] = cy1 * a.w + cx0;
        s.idx[3] = cy1 * a.w + cx1;
        s.w[0] = (vy0 && vx0) ? hy * hx * m : 0.f;
        s.w[1] = (vy0 && vx1) ? hy * lx * m : 0.f;
        s.w[2] = (vy1 && vx0) ? ly * hx * m : 0.f;
        s.w[3] = (vy1 && vx1) ? ly * lx * m : 0.f;
      }
    }
    si[k][pl] = s;
  }
  __syncthreads();

  const T* xb = (const T*)a.x + (int64_t)n * a.h * a.w * a.x_cs;
  const T* wp = (const T*)a.wpack;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int cin8 = round_up(a.cin, 8);

  floatx4 acc[DCN_WM][NBF];
#pragma unroll
  for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
    for (int b = 0; b < NBF; ++b) acc[m][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int c = 0; c < nchunk; ++c) {
    const int ch = c * 32 + grp * 8;
    const bool ch_ok = ch < cin8;
#pragma unroll 1
    for (int k = 0; k < 9; ++k) {
      frag bf[NBF];
#pragma unroll
      for (int b = 0; b < NBF; ++b) {
        const int co = co0 + b * 16 + row;
        if (co < cout_pad)
          bf[b] = Ops::load_b(wp + ((int64_t)(co * nchunk + c) * 9 + k) * 32 + grp * 8);
        else
          bf[b] = Ops::template gather<true>(nullptr, si[0][0], 0, 0, false);
      }
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m) {
        const int pl = wave * (16 * DCN_WM) + m * 16 + row;
        const SampleInfo s = si[k][pl];
        frag af = Ops::template gather<PLAIN>(xb, s, a.x_cs, ch, ch_ok);
#pragma unroll
        for (int b = 0; b < NBF; ++b) acc[m][b] = Ops::mma(af, bf[b], acc[m][b]);
      }
    }
  }

  // ---- epilogue ------------------------------------------------------------------------
  float gsum[NBF];
#pragma unroll
  for (int b = 0; b < NBF; ++b) {
    gsum[b] = 0.f;
    const int co = co0 + b * 16 + row;
    const bool co_ok = co < a.cout;
    const float bias = (co_ok && a.bias) ? a.bias[co] : 0.f;
    const float mul = (co_ok && a.post_mul) ? a.post_mul[co] : 1.f;
    const float add = (co_ok && a.post_add) ? a.post_add[co] : 0.f;
    const float scl = (co_ok && a.post_scale) ? a.post_scale[co] : 1.f;
#pragma unroll
    for (int m = 0; m < DCN_WM; ++m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = p0 + wave * (16 * DCN_WM) + m * 16 + grp * 4 + i;
        float v = (acc[m][b][i] + bias) * mul + add;
        if (a.relu) v = fmaxf(v, 0.f);
        v *= scl;
        if (co_ok && p < P) {
          const OutT o = from_f32<OutT>(v);
          if (a.out_layout == KAD_NHWC)
            ((OutT*)a.out)[((int64_t)n * P + p) * a.out_cs + co] = o;
          else
            ((OutT*)a.out)[((int64_t)n * a.cout + co) * P + p] = o;
          gsum[b] += to_f32(o);
        }
      }
    }
  }
  if (a.gap_partial) {
#pragma unroll
    for (int b = 0; b < NBF; ++b) {
      float v = gsum[b];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (grp == 0) gap_red[wave][b * 16 + row] = v;
    }
    __syncthreads();
    for (int j = tid; j < NBF * 16; j += DCN_THREADS) {
      const int co = co0 + j;
      if (co < a.cout) {
        const float v = (gap_red[0][j] + gap_red[1][j]) + (gap_red[2][j] + gap_red[3][j]);
        a.gap_partial[((int64_t)n * tiles + tile) * a.cout + co] = v;
      }
    }
  }
}

// ---- weight packing ------------------------------------------------------------------
template <typename T>
__global__ void dcn_pack_kernel(const float* w, T* out, int cin, int cout, int nchunk, int cout_pad) {
  const int64_t total = (int64_t)cout_pad * nchunk * 9 * 32;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int c32 = (int)(i % 32);
    const int k = (int)((i / 32) % 9);
    const int chunk = (int)((i / (32 * 9)) % nchunk);
    const int co = (int)(i / ((int64_t)32 * 9 * nchunk));
    const int ci = chunk * 32 + c32;
    float v = 0.f;
    if (co < cout && ci < cin) v = w[((int64_t)co * cin + ci) * 9 + k];
    out[i] = from_f32<T>(v);
  }
}

template <typename T, typename OutT, int NBF, bool PLAIN>
static int launch_dcn(const kad_dcn_args& a, hipStream_t st, int ho, int wo) {
  const int tiles = kad_dcn_tiles(ho, wo);
  const int nchunk = ceil_div(a.cin, 32);
  const int cout_pad = round_up(a.cout, 16);
  dim3 grid(tiles, ceil_div(a.cout, NBF * 16), a.n);
  hipLaunchKernelGGL((dcn_fwd_kernel<T, OutT, NBF, PLAIN>), grid, dim3(DCN_THREADS), 0, st, a, ho, wo, tiles, nchunk, cout_pad);
  return check_launch("kad_dcn_fwd");
}

template <typename T>
static int dispatch_dcn(const kad_dcn_args& a, hipStream_t st, int ho, int wo) {
  const int nbf = ceil_div(a.cout, 16);
  switch (nbf < 8 ? nbf : 8) {
    case 1: return launch_dcn<T, T, 1, false>(a, st, ho, wo);
    case 2: return launch_dcn<T, T, 2, false>(a, st, ho, wo);
    case 3: return launch_dcn<T, T, 3, false>(a, st, ho, wo);
    case 4: return launch_dcn<T, T, 4, false>(a, st, ho, wo);
    case 5: return launch_dcn<T, T, 5, false>(a, st, ho, wo);
    case 6: return launch_dcn<T, T, 6, false>(a, st, ho, wo);
    case 7: return launch_dcn<T, T, 7, false>(a, st, ho, wo);
    default: return launch_dcn<T, T, 8, false>(a, st, ho, wo);
  }
}

}  // namespace kad

using namespace kad;

extern "C" int64_t kad_dcn_wpack_elems(int cin, int cout) {
  if (cin <= 0 || cout <= 0) return 0;
  return (int64_t)round_up(cout, 16) * ceil_div(cin, 32) * 9 * 32;
}

extern "C" int kad_dcn_tiles(int ho, int wo) { return ceil_div(ho * wo, DCN_TILE); }

extern "C" int kad_dcn_pack_weights(const float* w, void* wpack, int cin, int cout, int dtype, void* stream) {
  KAD_CHECK_ARG(w && wpack, "kad_dcn_pack_weights: null pointer");
  KAD_CHECK_ARG(cin > 0 && cout > 0, "kad_dcn_pack_weights: cin=%d cout=%d must be positive", cin, cout);
  const int nchunk = ceil_div(cin, 32), cout_pad = round_up(cout, 16);
  const int64_t total = kad_dcn_wpack_elems(cin, cout);
  const int blocks = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case KAD_F32: hipLaunchKernelGGL(dcn_pack_kernel<float>, dim3(blocks), dim3(256), 0, st, w, (float*)wpack, cin, cout, nchunk, cout_pad); break;
    case KAD_F16: hipLaunchKernelGGL(dcn_pack_kernel<half_t>, dim3(blocks), dim3(256), 0, st, w, (half_t*)wpack, cin, cout, nchunk, cout_pad); break;
    case KAD_BF16: hipLaunchKernelGGL(dcn_pack_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st, w, (bf16_t*)wpack, cin, cout, nchunk, cout_pad); break;
    default: return fail(KAD_EINVAL, "kad_dcn_pack_weights: unknown dtype %d", dtype);
  }
  return check_launch("kad_dcn_pack_weights");
}

static int validate_dcn(const kad_dcn_args* a, bool need_offset, int* ho_out, int* wo_out) {
  KAD_CHECK_ARG(a, "null args");
  KAD_CHECK_ARG(a->x && a->wpack && a->out && (a->offset || !need_offset), "null tensor pointer");
  KAD_CHECK_ARG(a->n > 0 && a->cin > 0 && a->cout > 0 && a->h > 0 && a->w > 0,
                "bad shape n=%d cin=%d cout=%d h=%d w=%d", a->n, a->cin, a->cout, a->h, a->w);
  KAD_CHECK_ARG(a->stride >= 1 && a->pad >= 0, "bad stride=%d pad=%d", a->stride, a->pad);
  KAD_CHECK_ARG(a->x_cs % 8 == 0 && a->x_cs >= round_up(a->cin, 8),
                "x channel stride %d must be a multiple of 8 and >= roundup(cin=%d, 8)", a->x_cs, a->cin);
  KAD_CHECK_ARG(a->out_layout == KAD_NCHW || (a->out_layout == KAD_NHWC && a->out_cs >= a->cout),
                "bad output layout %d / channel stride %d", a->out_layout, a->out_cs);
  const int ho = (a->h + 2 * a->pad - 3) / a->stride + 1;
  const int wo = (a->w + 2 * a->pad - 3) / a->stride + 1;
  KAD_CHECK_ARG(ho > 0 && wo > 0, "empty output");
  KAD_CHECK_ARG((int64_t)a->h * a->w < (1ll << 31) && (int64_t)ho * wo * 9 < (1ll << 31), "image too large");
  const uintptr_t align = (uintptr_t)a->x | (uintptr_t)a->wpack;
  KAD_CHECK_ARG(align % 16 == 0, "x and wpack must be 16-byte aligned");
  *ho_out = ho;
  *wo_out = wo;
  return KAD_OK;
}

template <typename T>
static int dispatch_conv3x3(const kad_dcn_args& a, hipStream_t st, int ho, int wo) {
  const int nbf = ceil_div(a.cout, 16);
  switch (nbf < 8 ? nbf : 8) {
    case 1: return launch_dcn<T, float, 1, true>(a, st, ho, wo);
    case 2: return launch_dcn<T, float, 2, true>(a, st, ho, wo);
    case 3: return launch_dcn<T, float, 3, true>(a, st, ho, wo);
    case 4: return launch_dcn<T, float, 4, true>(a, st, ho, wo);
    default: return launch_dcn<T, float, 8, true>(a, st, ho, wo);
  }
}

extern "C" int kad_conv3x3_fwd(const kad_dcn_args* a, void* stream) {
  int ho = 0, wo = 0;
  int rc = validate_dcn(a, false, &ho, &wo);
  if (rc) return fail(rc, "kad_conv3x3_fwd: %s", kad_last_error());
  hipStream_t st = (hipStream_t)stream;
  switch (a->dtype) {
    case KAD_F32: return dispatch_conv3x3<float>(*a, st, ho, wo);
    case KAD_F16: return dispatch_conv3x3<half_t>(*a, st, ho, wo);
    case KAD_BF16: return dispatch_conv3x3<bf16_t>(*a, st, ho, wo);
    default: return fail(KAD_EINVAL, "kad_conv3x3_fwd: unknown dtype %d", a->dtype);
  }
}

extern "C" int kad_dcn_fwd(const kad_dcn_args* a, void* stream) {
  int ho = 0, wo = 0;
  int rc = validate_dcn(a, true, &ho, &wo);
  if (rc) return fail(rc, "kad_dcn_fwd: %s", kad_last_error());
  hipStream_t st = (hipStream_t)stream;
  switch (a->dtype) {
    case KAD_F32: return dispatch_dcn<float>(*a, st, ho, wo);
    case KAD_F16: return dispatch_dcn<half_t>(*a, st, ho, wo);
    case KAD_BF16: return dispatch_dcn<bf16_t>(*a, st, ho, wo);
    default: return fail(KAD_EINVAL, "kad_dcn_fwd: unknown dtype %d", a->dtype);
  }
}
