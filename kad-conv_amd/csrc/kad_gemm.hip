// Pointwise (1x1) convolution as an MFMA GEMM, with an optional fused
// s x s average pool on the input and a fused bias + activation epilogue.
//
//   out[n, co, p] = act( sum_ci W[co, ci] * avgpool_s(x)[n, ci, p] + b[co] )
//
// Serves three places on the path:
//  * KADConv's per-branch 1x1 projection after F.avg_pool2d(x, 2**i)
//    (KAD-Conv/kadconv/kad_conv.py:101,115), writing the branch input NHWC;
//  * the fused 1x1 conv + SiLU of KAD-CNet's Conv after Conv-BN fusion
//    (KAD-CNet/models/common.py:43-57; reference kernels
//    KAD-CNet/inference/acceleration/kadc_gemm_silu.cu:125-176 and
//    acceleration/kadc_fused_sm75.py:504-532);
//  * the per-branch projections of the builder-defined KADDown op.
//
// avg_pool2d here is floor mode with stride = kernel (kad_conv.py:115): output
// (H // s, W // s), trailing rows/columns dropped.
//
// GEMM: M = pooled pixels of one image (tile 128), N = Cout (tile 16 * NBF),
// K = Cin in steps of 32.  The pooled A tile [128 px][32 ch] is staged in LDS
// (transposed on the way in for NCHW input, so every lane's MFMA A fragment is
// 8 K-contiguous halves); the B fragment (weights, packed [Cout_pad][Cin_pad]
// with Cin_pad = roundup(Cin, 32)) is one 16-byte load per lane.
#include "kad_common.h"

namespace kad {

constexpr int GM_TILE = 128;
constexpr int GM_THREADS = 256;
constexpr int GM_LDS_STRIDE = 40;  // halves per pixel row of the A tile (32 + 8 pad: spreads banks)

template <typename T> struct GemmOps;
template <> struct GemmOps<half_t> {
  typedef half8_t frag;
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct GemmOps<bf16_t> {
  typedef bf16x8_t frag;
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// fp32 path keeps fp32 in LDS and uses the k=4 fp32 MFMA 8 times per k-step.
template <typename T> struct LdsT { typedef T type; };

template <typename T>
__device__ __forceinline__ float load_f(const T* p) { return to_f32(*p); }

template <typename T, int NBF>
__global__ __launch_bounds__(GM_THREADS) void gemm1x1_kernel(kad_gemm_args a, int hp, int wp, int tiles,
                                                            int cin_pad) {
  __shared__ float as32[(sizeof(T) == 4) ? GM_TILE * 33 : 1];
  __shared__ T ash[(sizeof(T) == 2) ? GM_TILE * GM_LDS_STRIDE : 1];
  const int tile = blockIdx.x;
  const int co0 = blockIdx.y * NBF * 16;
  const int n = blockIdx.z;
  const int P = hp * wp;
  const int p0 = tile * GM_TILE;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = lane & 15, grp = lane >> 4;
  const int s = a.pool;
  const float inv = 1.f / (float)(s * s);
  const T* x = (const T*)a.x;
  const T* wt = (const T*)a.wpack;

  floatx4 acc[2][NBF];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int b = 0; b < NBF; ++b) acc[m][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < cin_pad; k0 += 32) {
    __syncthreads();
    // ---- stage pooled A tile: 128 px x 32 ch -------------------------------------------
    // NCHW: consecutive lanes take consecutive pixels of one channel plane (coalesced);
    // NHWC: consecutive lanes take consecutive channels of one pixel.
    for (int e = tid; e < GM_TILE * 32; e += GM_THREADS) {
      int pl, c;
      if (a.in_layout == KAD_NCHW) {
        pl = e & (GM_TILE - 1);
        c = e >> 7;
      } else {
        c = e & 31;
        pl = e >> 5;
      }
      const int ci = k0 + c;
      const int p = p0 + pl;
      float v = 0.f;
      if (ci < a.cin && p < P) {
        const int py = p / wp, px = p - (p / wp) * wp;
        if (a.in_layout == KAD_NCHW) {
          const T* base = x + ((int64_t)n * a.cin + ci) * a.h * a.w;
          for (int dy = 0; dy < s; ++dy)
            for (int dx = 0; dx < s; ++dx) v += load_f(base + (int64_t)(py * s + dy) * a.w + px * s + dx);
        } else {
          const T* base = x + (int64_t)n * a.h * a.w * a.x_cs + ci;
          for (int dy = 0; dy < s; ++dy)
            for (int dx = 0; dx < s; ++dx)
              v += load_f(base + ((int64_t)(py * s + dy) * a.w + px * s + dx) * a.x_cs);
        }
        v *= inv;
      }
      if (sizeof(T) == 4)
        as32[pl * 33 + c] = v;
      else
        ash[pl * GM_LDS_STRIDE + c] = from_f32<T>(v);
    }
    __syncthreads();
    // ---- MFMA --------------------------------------------------------------------------
    if constexpr (sizeof(T) == 2) {
      typedef typename GemmOps<T>::frag frag;
      frag bf[NBF];
#pragma unroll
      for (int b = 0; b < NBF; ++b) {
        const int co = co0 + b * 16 + row;
        bf[b] = *(const frag*)(wt + (int64_t)co * cin_pad + k0 + grp * 8);
      }
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int pl = wave * 32 + m * 16 + row;
        const frag af = *(const frag*)(&ash[pl * GM_LDS_STRIDE + grp * 8]);
#pragma unroll
        for (int b = 0; b < NBF; ++b) acc[m][b] = GemmOps<T>::mma(af, bf[b], acc[m][b]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float bv[NBF];
#pragma unroll
        for (int b = 0; b < NBF; ++b) {
          const int co = co0 + b * 16 + row;
          bv[b] = ((const float*)wt)[(int64_t)co * cin_pad + k0 + grp * 8 + j];
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const int pl = wave * 32 + m * 16 + row;
          const float av = as32[pl * 33 + grp * 8 + j];
#pragma unroll
          for (int b = 0; b < NBF; ++b)
            acc[m][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[b], acc[m][b], 0, 0, 0);
        }
      }
    }
  }

  // ---- epilogue: bias, activation, store; zero the NHWC padding channels -------------
#pragma unroll
  for (int b = 0; b < NBF; ++b) {
    const int co = co0 + b * 16 + row;
    const bool co_ok = co < a.cout;
    const bool pad_ch = !co_ok && a.out_layout == KAD_NHWC && co < a.out_cs;
    const float bias = (co_ok && a.bias) ? a.bias[co] : 0.f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = p0 + wave * 32 + m * 16 + grp * 4 + i;
        if (p >= P) continue;
        float v = acc[m][b][i] + bias;
        if (a.act == 1) v = v * sigmoidf_(v);
        if (co_ok) {
          if (a.out_layout == KAD_NHWC)
            ((T*)a.out)[((int64_t)n * P + p) * a.out_cs + co] = from_f32<T>(v);
          else
            ((T*)a.out)[((int64_t)n * a.cout + co) * P + p] = from_f32<T>(v);
        } else if (pad_ch) {
          ((T*)a.out)[((int64_t)n * P + p) * a.out_cs + co] = from_f32<T>(0.f);
        }
      }
    }
  }
}

template <typename T>
__global__ void gemm_pack_kernel(const float* w, T* out, int cin, int cout, int cin_pad, int cout_pad) {
  const int64_t total = (int64_t)cout_pad * cin_pad;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int ci = (int)(i % cin_pad), co = (int)(i / cin_pad);
    out[i] = from_f32<T>((co < cout && ci < cin) ? w[(int64_t)co * cin + ci] : 0.f);
  }
}

template <typename T, int NBF>
static int launch_gemm(const kad_gemm_args& a, hipStream_t st, int hp, int wp) {
  const int P = hp * wp;
  const int tiles = ceil_div(P, GM_TILE);
  const int ncols = a.out_layout == KAD_NHWC ? (a.out_cs > a.cout ? a.out_cs : a.cout) : a.cout;
  dim3 grid(tiles, ceil_div(ncols, NBF * 16), a.n);
  hipLaunchKernelGGL((gemm1x1_kernel<T, NBF>), grid, dim3(GM_THREADS), 0, st, a, hp, wp, tiles,
                     round_up(a.cin, 32));
  return check_launch("kad_gemm1x1_fwd");
}

template <typename T>
static int dispatch_gemm(const kad_gemm_args& a, hipStream_t st, int hp, int wp) {
  const int ncols = a.out_layout == KAD_NHWC ? (a.out_cs > a.cout ? a.out_cs : a.cout) : a.cout;
  const int nbf = ceil_div(ncols, 16);
  switch (nbf < 8 ? nbf : 8) {
    case 1: return launch_gemm<T, 1>(a, st, hp, wp);
    case 2: return launch_gemm<T, 2>(a, st, hp, wp);
    case 3: return launch_gemm<T, 3>(a, st, hp, wp);
    case 4: return launch_gemm<T, 4>(a, st, hp, wp);
    case 5: return launch_gemm<T, 5>(a, st, hp, wp);
    case 6: return launch_gemm<T, 6>(a, st, hp, wp);
    case 7: return launch_gemm<T, 7>(a, st, hp, wp);
    default: return launch_gemm<T, 8>(a, st, hp, wp);
  }
}

}  // namespace kad

using namespace kad;

extern "C" int64_t kad_gemm_wpack_elems(int cin, int cout) {
  if (cin <= 0 || cout <= 0) return 0;
  // rows cover every 16-wide column block a launch can touch (NHWC padding included)
  return (int64_t)round_up(round_up(cout, 8), 128) * round_up(cin, 32);
}

extern "C" int kad_gemm_pack_weights(const float* w, void* wpack, int cin, int cout, int dtype, void* stream) {
  KAD_CHECK_ARG(w && wpack, "kad_gemm_pack_weights: null pointer");
  KAD_CHECK_ARG(cin > 0 && cout > 0, "kad_gemm_pack_weights: bad shape cin=%d cout=%d", cin, cout);
  const int cin_pad = round_up(cin, 32), cout_pad = round_up(round_up(cout, 8), 128);
  const int64_t total = (int64_t)cin_pad * cout_pad;
  const int blocks = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case KAD_F32: hipLaunchKernelGGL(gemm_pack_kernel<float>, dim3(blocks), dim3(256), 0, st, w, (float*)wpack, cin, cout, cin_pad, cout_pad); break;
    case KAD_F16: hipLaunchKernelGGL(gemm_pack_kernel<half_t>, dim3(blocks), dim3(256), 0, st, w, (half_t*)wpack, cin, cout, cin_pad, cout_pad); break;
    case KAD_BF16: hipLaunchKernelGGL(gemm_pack_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st, w, (bf16_t*)wpack, cin, cout, cin_pad, cout_pad); break;
    default: return fail(KAD_EINVAL, "kad_gemm_pack_weights: unknown dtype %d", dtype);
  }
  return check_launch("kad_gemm_pack_weights");
}

extern "C" int kad_gemm1x1_fwd(const kad_gemm_args* a, void* stream) {
  KAD_CHECK_ARG(a, "kad_gemm1x1_fwd: null args");
  KAD_CHECK_ARG(a->x && a->wpack && a->out, "kad_gemm1x1_fwd: null tensor pointer");
  KAD_CHECK_ARG(a->n > 0 && a->cin > 0 && a->cout > 0 && a->h > 0 && a->w > 0 && a->pool >= 1,
                "kad_gemm1x1_fwd: bad shape n=%d cin=%d cout=%d h=%d w=%d pool=%d", a->n, a->cin, a->cout, a->h,
                a->w, a->pool);
  KAD_CHECK_ARG(a->in_layout == KAD_NCHW || (a->in_layout == KAD_NHWC && a->x_cs >= a->cin),
                "kad_gemm1x1_fwd: bad input layout/channel stride");
  KAD_CHECK_ARG(a->out_layout == KAD_NCHW || (a->out_layout == KAD_NHWC && a->out_cs >= a->cout &&
                                              a->out_cs <= round_up(round_up(a->cout, 8), 128)),
                "kad_gemm1x1_fwd: bad output layout/channel stride");
  KAD_CHECK_ARG(a->act == 0 || a->act == 1, "kad_gemm1x1_fwd: act must be 0 (none) or 1 (SiLU)");
  const int hp = a->h / a->pool, wp = a->w / a->pool;
  KAD_CHECK_ARG(hp > 0 && wp > 0, "kad_gemm1x1_fwd: pool %d larger than the image", a->pool);
  KAD_CHECK_ARG(((uintptr_t)a->wpack) % 16 == 0, "kad_gemm1x1_fwd: wpack must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  switch (a->dtype) {
    case KAD_F32: return dispatch_gemm<float>(*a, st, hp, wp);
    case KAD_F16: return dispatch_gemm<half_t>(*a, st, hp, wp);
    case KAD_BF16: return dispatch_gemm<bf16_t>(*a, st, hp, wp);
    default: return fail(KAD_EINVAL, "kad_gemm1x1_fwd: unknown dtype %d", a->dtype);
  }
}
