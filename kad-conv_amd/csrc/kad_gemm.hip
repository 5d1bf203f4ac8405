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

// ---- NCHW fast path -------------------------------------------------------------------------
// 16-bit NCHW input and output, no pooling, P = H * W a multiple of 4.
//
// Block = 256 threads (4 waves) x 128 pixels of one image x 256 output
// channels; wave w owns channels [64 w, 64 w + 64) of the block's range and all
// 128 pixels.  Per 32-channel k-step the input tile [32 ci][128 px] goes to LDS
// exactly as it lies in memory (16-byte pieces along the pixels, coalesced).
// No transpose pass: MFMA column c of pixel fragment j (j = 0..7) is pixel
// 8 c + j, so lane (c, g) reads rows 8 g .. 8 g + 7 at pixels 8 c .. 8 c + 7
// (eight 16-byte LDS reads) and an 8 x 8 transpose of 16-bit values in its own
// registers gives its B operand (8 channels of one pixel) for all eight
// fragments.  The accumulator of fragment j in lane (c, g) holds channels
// 4 g + i at pixel 8 c + j, so every lane ends with eight consecutive pixels per
// output channel: one 16-byte store (two 8-byte stores when P % 8 != 0).
// A (weights, rows = output channels) is one 16-byte load per lane and
// fragment from the packed [Cout_pad][Cin_pad] layout, prefetched one k-step
// ahead like the input tile.  Work items are ordered so the channel blocks of
// one pixel tile run back to back on the same XCD (shared L2).
constexpr int GN_PX = 128;         // pixels per tile
constexpr int GN_WCO = 64;         // output channels per wave
constexpr int GN_CO = 4 * GN_WCO;  // output channels per block

template <typename T> struct Raw16 { typedef half8_t type; };
template <> struct Raw16<bf16_t> { typedef bf16x8_t type; };

template <bool V16>
__device__ __forceinline__ intx4 ld_px8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (V16) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  } else {  // 8-byte aligned halves
    typedef int intx2 __attribute__((ext_vector_type(2)));
    const intx2 lo = __builtin_bit_cast(intx2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
    const intx2 hi = __builtin_bit_cast(intx2, __builtin_amdgcn_raw_buffer_load_b64(r, off + 8, 0, 0));
    return intx4{lo[0], lo[1], hi[0], hi[1]};
  }
}

template <typename T, bool V16>
__global__ __launch_bounds__(256, 2) void gemm_nchw_kernel(kad_gemm_args a, int P, int tiles_px, int co_blocks,
                                                           int total, int cin_pad) {
  typedef typename GemmOps<T>::frag frag;
  __shared__ __align__(16) T xs[2][32 * GN_PX];  // [ci][px] per stage
  const int bid = blockIdx.x;
  const int wi = (bid & 7) * (int)(gridDim.x >> 3) + (bid >> 3);  // contiguous band of work per XCD
  if (wi >= total) return;  // whole block, before any barrier
  const int cb = wi % co_blocks, t2 = wi / co_blocks;
  const int n = t2 / tiles_px, p0 = (t2 - n * tiles_px) * GN_PX;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, g = lane >> 4;
  const int co_w = cb * GN_CO + wave * GN_WCO;
  const int nk = cin_pad / 32;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((int64_t)a.n * a.cin * P * 2));
  const int cout_pk = round_up(round_up(a.cout, 8), 128);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.wpack, (uint32_t)((int64_t)cout_pk * cin_pad * 2));
  // staging pieces: rows tid / 16 and 16 + tid / 16, pixels 8 (tid % 16) .. + 8
  const int sr = tid >> 4, sq = tid & 15;
  const uint32_t xrow = (uint32_t)(P * 2);
  const uint32_t xo0 = (uint32_t)((((int64_t)n * a.cin + sr) * P + p0 + 8 * sq) * 2);
  const uint32_t xo1 = xo0 + 16u * xrow;
  uint32_t wo[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int co = co_w + 16 * m + c;
    wo[m] = co < cout_pk ? (uint32_t)((co * cin_pad + 8 * g) * 2) : KAD_OOB;
  }
  // Loads for a step past the last one read zeros (out-of-range offsets): the
  // prefetch is issued unconditionally, so no branch splits the wait counts.
  auto ld_x = [&](int ks, intx4& v0, intx4& v1) {
    const int r = ks * 32 + sr;
    const uint32_t step = (uint32_t)ks * 32u * xrow;
    v0 = ld_px8<V16>(rx, r < a.cin ? xo0 + step : KAD_OOB);
    v1 = ld_px8<V16>(rx, r + 16 < a.cin ? xo1 + step : KAD_OOB);
  };
  auto ld_w = [&](int ks, frag (&w)[4]) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
      w[m] = __builtin_bit_cast(frag, __builtin_amdgcn_raw_buffer_load_b128(
                                          rw, (wo[m] == KAD_OOB || ks >= nk) ? KAD_OOB : wo[m] + (uint32_t)ks * 64u, 0, 0));
  };
  auto st_x = [&](int s, const intx4& v0, const intx4& v1) {
    *(intx4*)&xs[s][sr * GN_PX + 8 * sq] = v0;
    *(intx4*)&xs[s][(sr + 16) * GN_PX + 8 * sq] = v1;
  };

  floatx4 acc[4][8];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  intx4 v0, v1;
  frag wa[4], wb[4];
  ld_x(0, v0, v1);
  ld_w(0, wa);
  st_x(0, v0, v1);
  __syncthreads();
  // one k-step: prefetch step ks + 1 (input pieces, weights into wnx), multiply
  // step ks from LDS stage ks & 1 with weights wc, then stage the prefetched tile
  auto step = [&](int ks, const frag (&wc)[4], frag (&wnx)[4]) {
    const int s = ks & 1;
    ld_x(ks + 1, v0, v1);  // rows past Cin (and so every row of step nk) read zeros
    ld_w(ks + 1, wnx);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of this step's MFMAs
    typedef typename Raw16<T>::type raw_t;
    raw_t raw[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) raw[r] = *(const raw_t*)&xs[s][(8 * g + r) * GN_PX + 8 * c];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      frag b;
#pragma unroll
      for (int r = 0; r < 8; ++r) b[r] = raw[r][j];  // channel 8 g + r of pixel 8 c + j
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m][j] = GemmOps<T>::mma(wc[m], b, acc[m][j]);
    }
    __builtin_amdgcn_sched_barrier(0);  // the prefetched tile is stored after the MFMAs, not before
    st_x(s ^ 1, v0, v1);  // stage s ^ 1 was last read before the previous barrier
    __syncthreads();
  };
  for (int ks = 0; ks < nk; ks += 2) {  // unrolled by two: the weight buffers swap roles without copies
    step(ks, wa, wb);
    if (ks + 1 < nk) step(ks + 1, wb, wa);
  }

  // ---- epilogue: bias, activation, eight consecutive pixels per channel ----------------------------
  const int px = p0 + 8 * c;
  const int nvalid = P - px;  // pixels of this lane's run inside the image (>= 8: full run)
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int co = co_w + 16 * m + 4 * g + i;
      if (co >= a.cout || nvalid <= 0) continue;
      const float bias = a.bias ? a.bias[co] : 0.f;
      typename Raw16<T>::type o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float v = acc[m][j][i] + bias;
        if (a.act == 1) v = v * __builtin_amdgcn_rcpf(1.f + __expf(-v));  // SiLU; 16-bit output
        o[j] = from_f32<T>(v);
      }
      T* dst = (T*)a.out + ((int64_t)n * a.cout + co) * P + px;
      if (nvalid >= 8) {
        if constexpr (V16) {
          *(intx4*)dst = __builtin_bit_cast(intx4, o);
        } else {
          typedef int intx2 __attribute__((ext_vector_type(2)));
          const intx4 q = __builtin_bit_cast(intx4, o);
          *(intx2*)dst = intx2{q[0], q[1]};
          *(intx2*)(dst + 4) = intx2{q[2], q[3]};
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < nvalid) dst[j] = o[j];
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
static int launch_gemm_nchw(const kad_gemm_args& a, hipStream_t st) {
  const int P = a.h * a.w;
  const int tiles_px = ceil_div(P, GN_PX), co_blocks = ceil_div(a.cout, GN_CO);
  const int total = a.n * tiles_px * co_blocks;
  const int cin_pad = round_up(a.cin, 32);
  dim3 grid(round_up(total, 8));
  if (P % 8 == 0)
    hipLaunchKernelGGL((gemm_nchw_kernel<T, true>), grid, dim3(256), 0, st, a, P, tiles_px, co_blocks, total, cin_pad);
  else
    hipLaunchKernelGGL((gemm_nchw_kernel<T, false>), grid, dim3(256), 0, st, a, P, tiles_px, co_blocks, total, cin_pad);
  return check_launch("kad_gemm1x1_fwd");
}

// The NCHW fast path covers 16-bit NCHW -> NCHW without pooling when P % 4 == 0
// (8-byte aligned pixel runs) and every buffer offset fits 31 bits.
static bool nchw_fast_ok(const kad_gemm_args& a) {
  const int64_t P = (int64_t)a.h * a.w;
  const int64_t cout_pk = round_up(round_up(a.cout, 8), 128);
  return a.dtype != KAD_F32 && a.pool == 1 && a.in_layout == KAD_NCHW && a.out_layout == KAD_NCHW && P % 4 == 0 &&
         ((uintptr_t)a.x % 8) == 0 && ((uintptr_t)a.out % 8) == 0 && (int64_t)a.n * a.cin * P * 2 < (1ll << 31) &&
         cout_pk * round_up(a.cin, 32) * 2 < (1ll << 31);
}

template <typename T>
static int dispatch_gemm(const kad_gemm_args& a, hipStream_t st, int hp, int wp) {
  if constexpr (sizeof(T) == 2)
    if (nchw_fast_ok(a)) return launch_gemm_nchw<T>(a, st);
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
