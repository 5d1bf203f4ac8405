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
#include <type_traits>

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
  auto epilogue = [&](auto act_tag) {  // activation as a template argument: no per-value branch
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int b = 0; b < NBF; ++b) {
      const int co = co0 + b * 16 + row;
      const bool co_ok = co < a.cout;
      // NHWC: channels [cout, roundup(cout, 8)) are the output's zero padding; the rest of a
      // wider channel stride (other slices of a concat buffer) is left untouched
      const bool pad_ch = !co_ok && a.out_layout == KAD_NHWC && co < a.out_cs && co < round_up(a.cout, 8);
      const float bias = (co_ok && a.bias) ? a.bias[co] : 0.f;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int p = p0 + wave * 32 + m * 16 + grp * 4 + i;
          if (p >= P) continue;
          float v = acc[m][b][i] + bias;
          if constexpr (ACT == 1) v = v * sigmoidf_(v);
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
  };
  if (a.act == 1) epilogue(std::integral_constant<int, 1>{});
  else epilogue(std::integral_constant<int, 0>{});
}

// ---- NCHW fast path -------------------------------------------------------------------------
// 16-bit NCHW input and output, no pooling, P = H * W a multiple of 4.
//
// Block = NW waves (4 or 8) x 128 pixels of one image x 64 NW output
// channels; wave w owns channels [64 w, 64 w + 64) of the block's range and all
// 128 pixels (8 waves cover Cout = 512 in one block, so the input tile is read
// from memory once).  K runs in 32-channel steps.  The input tile of a step,
// [32 ci][128 px] exactly as it lies in memory (16-byte pieces along the pixels
// when P % 8 == 0, else 4-byte pieces), goes through a ring of three LDS stages
// filled by buffer -> LDS loads (no registers in between); each wave's weight
// fragments (one 16-byte load per lane and fragment from the packed
// [Cout_pad][Cin_pad] layout, L2-resident) go straight to registers, three
// buffers rotating with the stages.  Both are issued two steps ahead; a step
// opens with "own loads of this step landed" (vmcnt) + barrier.  LDS then
// carries only the input tile: one write and NW reads per step.
// No transpose pass: MFMA column c of pixel fragment j (j = 0..7) is pixel
// 8 c + j, so lane (c, g) reads rows 8 g .. 8 g + 7 at pixels 8 c .. 8 c + 7
// (eight 16-byte LDS reads) and an 8 x 8 transpose of 16-bit values in its own
// registers gives its B operand (8 channels of one pixel) for all eight
// fragments.  The accumulator of fragment j in lane (c, g) holds channels
// 4 g + i at pixel 8 c + j, so every lane ends with eight consecutive pixels per
// output channel: one 16-byte store (two 8-byte stores when P % 8 != 0).
// Work items are ordered so the channel blocks of one pixel tile run back to
// back on the same XCD (shared L2).  The 64-pixel tile (PXT below) is the same
// scheme with runs of 4 pixels: four fragments, 8-byte LDS reads and stores.
constexpr int GN_WCO = 64;  // output channels per wave

template <typename T, int JP> struct RawRun;  // JP consecutive 16-bit pixels of one channel row
template <> struct RawRun<half_t, 8> { typedef half8_t type; };
template <> struct RawRun<bf16_t, 8> { typedef bf16x8_t type; };
template <> struct RawRun<half_t, 4> { typedef half_t type __attribute__((ext_vector_type(4))); };
template <> struct RawRun<bf16_t, 4> { typedef bf16_t type __attribute__((ext_vector_type(4))); };

// PXT = 128: lane runs of 8 pixels, 4 x 8 accumulator tiles per wave, two blocks per CU.
// PXT = 64: lane runs of 4 pixels (MFMA column c of pixel fragment j is pixel 4 c + j), 4 x 4
// accumulator tiles per wave, three blocks per CU: half the work per wave, so a launch's last
// round of blocks is shorter and small launches fill more of the chip.
template <int PXT> constexpr int gn_min_blocks() { return PXT == 128 ? 2 : 3; }

template <typename T, bool V16, int NW, int PXT>
__global__ __launch_bounds__(64 * NW, (8 / NW) * gn_min_blocks<PXT>() / 2) void gemm_nchw_kernel(
    kad_gemm_args a, int P, int tiles_px, int co_blocks, int total, int cin_pad) {
  static_assert(PXT == 128 || PXT == 64, "pixel tile");
  constexpr int JP = PXT / 16;  // pixels per lane run = pixel fragments per wave
  typedef typename GemmOps<T>::frag frag;
  typedef typename RawRun<T, JP>::type raw_t;
  constexpr int STAGE = 32 * PXT * 2;  // input tile bytes per stage
  // one object per stage: the compiler tracks the loads into each separately
  __shared__ __align__(16) char st0[STAGE];
  __shared__ __align__(16) char st1[STAGE];
  __shared__ __align__(16) char st2[STAGE];
  const int bid = blockIdx.x;
  const int wi = (bid & 7) * (int)(gridDim.x >> 3) + (bid >> 3);  // contiguous band of work per XCD
  if (wi >= total) return;  // whole block, before any barrier
  const int cb = wi % co_blocks, t2 = wi / co_blocks;
  const int n = t2 / tiles_px, p0 = (t2 - n * tiles_px) * PXT;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar offsets below)
  const int co_w = (cb * NW + wave) * GN_WCO;
  const int nk = cin_pad / 32;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((int64_t)a.n * a.cin * P * 2));
  const int cout_pk = round_up(round_up(a.cout, 8), 128);
  // the fragment-ordered copy behind the row layout
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc((const T*)a.wpack + (int64_t)cout_pk * cin_pad, (uint32_t)((int64_t)cout_pk * cin_pad * 2));

  // Input pieces (PB = 16 bytes when P % 8 == 0, else 4): a tile row of PXT pixels is
  // LPR lanes of one load, so one load covers RQ = 64 / LPR rows; wave w stages rows
  // RPW w .. + RPW, its load q rows RPW w + RQ q + lr (lr = lane / LPR) at pixels
  // p0 + lpx ..  The row base goes in the wave-uniform soffset, the lane part (pixels,
  // lr rows) in voffset, which is out of range for pixels past the image row or rows
  // past Cin: such lanes read zeros and no load reaches past the tensor.
  constexpr int PB = V16 ? 16 : 4, LPR = PXT * 2 / PB, RQ = 64 / LPR;
  constexpr int RPW = 32 / NW, XQ = RPW / RQ;
  static_assert(XQ >= 1 && RPW % RQ == 0, "input pieces");
  const int lr = lane / LPR, lpx = (PB / 2) * (lane % LPR);
  const uint32_t prow = (uint32_t)P * 2u;  // bytes per channel row
  const uint32_t xlane = p0 + lpx < P ? (uint32_t)lr * prow + (uint32_t)(p0 + lpx) * 2u : KAD_OOB;
  const int64_t xrow0 = (int64_t)n * a.cin + RPW * wave;  // first row of this wave's pieces (step 0)
  uint32_t woff[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int co = co_w + 16 * m + c;
    woff[m] = co < cout_pk ? (uint32_t)(((((co_w >> 4) + m) * nk) * 64 + lane) * 16) : KAD_OOB;
  }
  constexpr int L = XQ + 4;  // loads per wave per step
  // Loads of step kk: input into stage st, weights into w; a step past the last
  // one (or a row past Cin) reads zeros, so every path issues the same loads.
  // soffset stays the uniform row base (< 2^31, so the sum with KAD_OOB cannot
  // wrap into range).
  auto issue = [&](int kk, char* st, frag (&w)[4]) {
    if constexpr (RQ == 1) {  // one row per load, rows wave-uniform: a short rolled loop keeps the offsets in scalars
      const int rows = kk < nk ? min(a.cin - (kk * 32 + RPW * wave), RPW) : 0;  // valid rows of this wave
      uint32_t soff = (uint32_t)((xrow0 + kk * 32) * P * 2);
      char* dst = st + RPW * wave * PXT * 2;
#pragma unroll 1
      for (int q = 0; q < XQ; ++q) {
        dma4(rx, dst, q < rows ? xlane : KAD_OOB, soff);
        soff += prow;
        dst += PXT * 2;
      }
    } else {
#pragma unroll
      for (int q = 0; q < XQ; ++q) {
        const bool ok = kk < nk && kk * 32 + RPW * wave + RQ * q + lr < a.cin;
        char* dst = st + (RPW * wave + RQ * q) * PXT * 2;
        const uint32_t soff = (uint32_t)((xrow0 + kk * 32 + RQ * q) * P * 2);
        if constexpr (V16)
          dma16(rx, dst, ok ? xlane : KAD_OOB, soff);
        else
          dma4(rx, dst, ok ? xlane : KAD_OOB, soff);
      }
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t o = (woff[m] == KAD_OOB || kk >= nk) ? KAD_OOB : woff[m] + (uint32_t)kk * 1024u;
      w[m] = __builtin_bit_cast(frag, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, 0));
    }
  };

  floatx4 acc[4][JP];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < JP; ++j) acc[m][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // step kk: wait for this wave's loads of step kk (those of step kk + 1, L per
  // wave, may stay in flight) and for every wave's LDS reads of the previous
  // step, then barrier; refill the stage and weight buffer of the previous step
  // with step kk + 2; multiply.
  auto step = [&](int kk, const char* cur, char* refill, const frag (&wf)[4], frag (&wrefill)[4]) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(L) : "memory");
    issue(kk + 2, refill, wrefill);
    raw_t raw[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) raw[r] = *(const raw_t*)(cur + ((8 * g + r) * PXT + JP * c) * 2);
#pragma unroll
    for (int j = 0; j < JP; ++j) {
      frag b;
#pragma unroll
      for (int r = 0; r < 8; ++r) b[r] = raw[r][j];  // channel 8 g + r of pixel JP c + j
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m][j] = GemmOps<T>::mma(wf[m], b, acc[m][j]);
    }
  };
  frag w0[4], w1[4], w2[4];
  issue(0, st0, w0);
  issue(1, st1, w1);
  const int nk3 = nk / 3 * 3;
  for (int kk = 0; kk < nk3; kk += 3) {  // branch-free body: exact wait counts
    step(kk, st0, st2, w0, w2);
    step(kk + 1, st1, st0, w1, w0);
    step(kk + 2, st2, st1, w2, w1);
  }
  if (nk3 < nk) step(nk3, st0, st2, w0, w2);
  if (nk3 + 1 < nk) step(nk3 + 1, st1, st0, w1, w0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the block

  // ---- epilogue: bias, activation, JP consecutive pixels per channel ------------------------------
  const int px = p0 + JP * c;
  const int nvalid = P - px;  // pixels of this lane's run inside the image (>= JP: full run)
  // every bias first: loads and stores share one in-order counter, so a load
  // issued after a store would make its wait include that store's write
  float bias[4][4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int co = co_w + 16 * m + 4 * g + i;
      bias[m][i] = (a.bias && co < a.cout) ? a.bias[co] : 0.f;
    }
  auto epilogue = [&](auto act_tag) {  // activation as a template argument: no per-value branch
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int co = co_w + 16 * m + 4 * g + i;
        if (co >= a.cout || nvalid <= 0) continue;
        raw_t o;
#pragma unroll
        for (int j = 0; j < JP; ++j) {
          float v = acc[m][j][i] + bias[m][i];
          if constexpr (ACT == 1) v = v * __builtin_amdgcn_rcpf(1.f + __expf(-v));  // SiLU; 16-bit output
          o[j] = from_f32<T>(v);
        }
        T* dst = (T*)a.out + ((int64_t)n * a.cout + co) * P + px;
        if (nvalid >= JP) {
          typedef int intx2 __attribute__((ext_vector_type(2)));
          if constexpr (JP == 4) {
            *(intx2*)dst = __builtin_bit_cast(intx2, o);  // P % 4 == 0: 8-byte aligned
          } else if constexpr (V16) {
            *(intx4*)dst = __builtin_bit_cast(intx4, o);
          } else {
            const intx4 q = __builtin_bit_cast(intx4, o);
            *(intx2*)dst = intx2{q[0], q[1]};
            *(intx2*)(dst + 4) = intx2{q[2], q[3]};
          }
        } else {
#pragma unroll
          for (int j = 0; j < JP; ++j)
            if (j < nvalid) dst[j] = o[j];
        }
      }
    }
  };
  if (a.act == 1) epilogue(std::integral_constant<int, 1>{});
  else epilogue(std::integral_constant<int, 0>{});
}

// Packed weights: rows [Cout_pad][Cin_pad] (the general kernel, the pyramid),
// then the same values in MFMA fragment order for the NCHW fast path: per
// (16-channel block cb, 32-channel step ks) one 1 KB chunk at
// ((cb * nk + ks) * 64 + lane) * 8 elements, lane = r + 16 g holding
// W[16 cb + r][32 ks + 8 g .. + 8], so a wave's fragment load is one
// contiguous 1 KB read.
template <typename T>
__global__ void gemm_pack_kernel(const float* w, T* out, int cin, int cout, int cin_pad, int cout_pad) {
  const int64_t total = (int64_t)cout_pad * cin_pad;
  const int nk = cin_pad / 32;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int ci = (int)(i % cin_pad), co = (int)(i / cin_pad);
    const T v = from_f32<T>((co < cout && ci < cin) ? w[(int64_t)co * cin + ci] : 0.f);
    out[i] = v;
    const int lane = (co & 15) + 16 * ((ci & 31) >> 3);
    out[total + ((int64_t)((co >> 4) * nk + (ci >> 5)) * 64 + lane) * 8 + (ci & 7)] = v;
  }
}

// ---- NHWC fast path ---------------------------------------------------------------------------------
// 16-bit NHWC input and output, no pooling, Cin a multiple of 8 (whole 16-byte channel pieces).
// In NHWC both MFMA operands are contiguous 16-byte runs:
//  * A = weights, 16 output channels x 32 input channels: lane (r, g) holds row r's input
//    channels 8g .. 8g + 7, from the block's copy of its fragment-ordered weights in LDS (WLDS:
//    one copy per block, one barrier), else straight from the packed [Cout_pad][Cin_pad] rows;
//  * B = input, 32 input channels x 16 pixels: lane (c, g) loads pixel c's channels 8g .. 8g + 7
//    straight from memory into registers (four lanes cover a pixel's 64 contiguous bytes of the
//    k-step).
// A wave owns 64 pixels (4 pixel fragments) x 16 NB output channels.  The accumulator of
// (pixel fragment m, channel fragment f) in lane (c, g) holds output channels 16 f + 4 g .. + 3
// of pixel 16 m + c: one 8-byte store.  The next k-step's operands are loaded before this step's
// MFMAs.  Input channels past Cin inside a k-step are read as 0 (they may belong to another slice
// of a concat buffer); weight rows past Cout are zero in the packing.
constexpr int GH_PXW = 64;    // pixels per wave
constexpr int GH_WAVES = 4;   // waves per block

// WLDS: the block's four waves share one channel block and take four pixel tiles; the block first
// copies its weight fragments (the packing's fragment-ordered part: NB x Cin_pad / 32 chunks of
// 1 KB, contiguous) into LDS, so per k-step a wave loads only its pixel fragments from memory and
// reads the weights from LDS (without it every wave fetched the same weights through the vector
// memory path, which bounded the big launches).
template <typename T, int NB, bool WLDS>
__global__ __launch_bounds__(64 * GH_WAVES) void gemm_nhwc_kernel(kad_gemm_args a, int P, int tiles_px, int co_blocks,
                                                                 int total, int cin_pad, int stage) {
  typedef typename GemmOps<T>::frag frag;
  extern __shared__ __align__(16) char gh_smem[];  // WLDS: [NB][nk][64 lanes][16 bytes]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nk = cin_pad / 32;
  int cb, t;
  if constexpr (WLDS) {
    // Blocks are dealt to the 8 XCDs round robin (block b to XCD b % 8), each with its own L2:
    // blocks b, b + 8, ... b + 8 (co_blocks - 1) take the same four pixel tiles with each channel
    // block, so a tile's pixels are fetched into one L2 only.
    const int ntg = ceil_div(total / co_blocks, GH_WAVES), b = blockIdx.x;
    const int tg = (b / (8 * co_blocks)) * 8 + (b & 7);
    if (tg >= ntg) return;  // the whole block, before its barrier
    cb = (b >> 3) % co_blocks;
    t = tg * GH_WAVES + wave;
    const int cpad16 = round_up(round_up(a.cout, 8), 128) / 16;  // 16-column blocks in the packing
    const T* frags = (const T*)a.wpack + (int64_t)cpad16 * 16 * cin_pad;
    const int nchunk = NB * nk * 64;  // 16-byte pieces
    for (int e0 = 0; e0 < nchunk; e0 += 8 * 64 * GH_WAVES) {
      intx4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + u * 64 * GH_WAVES + threadIdx.x, ch = e >> 6, f = ch / nk, cb16 = cb * NB + f;
        v[u] = intx4{0, 0, 0, 0};
        if (e < nchunk && cb16 < cpad16)
          v[u] = *(const intx4*)(frags + ((int64_t)(cb16 * nk + (ch - f * nk)) * 64 + (e & 63)) * 8);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + u * 64 * GH_WAVES + threadIdx.x;
        if (e < nchunk) *(intx4*)(gh_smem + (size_t)e * 16) = v[u];
      }
    }
    __syncthreads();
    if (t * co_blocks >= total) return;  // no tile for this wave (after the block's only barrier)
  } else {
    const int item = blockIdx.x * GH_WAVES + wave;
    if (item >= total) return;
    cb = item % co_blocks;  // the channel blocks of a pixel tile run in neighbouring waves
    t = item / co_blocks;
  }
  const int n = t / tiles_px, p0 = (t - n * tiles_px) * GH_PXW;
  const int co0 = cb * NB * 16;
  const int c = lane & 15, g = lane >> 4;
  const T* x = (const T*)a.x + (int64_t)n * P * a.x_cs;
  const T* wt = (const T*)a.wpack;
  const T* xp[4];
  bool pok[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int p = p0 + 16 * m + c;
    pok[m] = p < P;
    xp[m] = x + (int64_t)(pok[m] ? p : 0) * a.x_cs + 8 * g;
  }
  const T* wr[NB];
  const int wrows = round_up(round_up(a.cout, 8), 128);  // rows of the packed [Cout_pad][Cin_pad] part
#pragma unroll
  for (int f = 0; f < NB; ++f) {
    const int co = co0 + 16 * f + c;  // rows past the packing (discarded columns) read row 0
    wr[f] = wt + (int64_t)(co < wrows ? co : 0) * cin_pad + 8 * g;
  }
  floatx4 acc[4][NB];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int f = 0; f < NB; ++f) acc[m][f] = floatx4{0.f, 0.f, 0.f, 0.f};
  const frag zero = frag{};
  frag xa[4], wa[NB];
  auto load = [&](int k0, frag* xv, frag* wv) {
    const bool kok = k0 + 8 * g < a.cin;
#pragma unroll
    for (int m = 0; m < 4; ++m) xv[m] = (pok[m] && kok) ? *(const frag*)(xp[m] + k0) : zero;
    if constexpr (!WLDS) {
#pragma unroll
      for (int f = 0; f < NB; ++f) wv[f] = *(const frag*)(wr[f] + k0);
    }
  };
  load(0, xa, wa);
  for (int k0 = 0; k0 < cin_pad; k0 += 32) {
    frag xn[4], wn[NB];
    const bool more = k0 + 32 < cin_pad;
    if (more) load(k0 + 32, xn, wn);
    if constexpr (WLDS) {
#pragma unroll
      for (int f = 0; f < NB; ++f) wa[f] = *(const frag*)(gh_smem + ((f * nk + (k0 >> 5)) * 64 + lane) * 16);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int f = 0; f < NB; ++f) acc[m][f] = GemmOps<T>::mma(wa[f], xa[m], acc[m][f]);
    if (more) {
#pragma unroll
      for (int m = 0; m < 4; ++m) xa[m] = xn[m];
      if constexpr (!WLDS) {
#pragma unroll
        for (int f = 0; f < NB; ++f) wa[f] = wn[f];
      }
    }
  }
  // ---- epilogue: bias, activation, 8-byte stores of 4 channels; zero the pad channels ----------
  const int cpad = round_up(a.cout, 8) < a.out_cs ? round_up(a.cout, 8) : a.out_cs;
  T* out = (T*)a.out + (int64_t)n * P * a.out_cs;
  if constexpr (WLDS) {
    if (stage) {
      // Through the wave's own LDS tile [64 pixels][16 NB (+ 8 pad)]: a lane's 8-byte pieces (4
      // channels of one pixel, 16 pixels per store) left the output lines partly written, and the
      // memory side wrote about twice the output bytes; read back, consecutive lanes store
      // consecutive 16-byte pieces of each pixel's channel run.  out_cs % 8 == 0, 16-byte aligned.
      // stage 1: the tiles behind the weights; 2: in the weights' place, once every wave of the
      // block is done with them (waves without a tile have ended and are not waited for).
      constexpr int OBS = 16 * NB + 8;
      T* stg = (T*)(gh_smem + (stage == 1 ? NB * nk * 1024 : 0)) + wave * 64 * OBS;
      if (stage == 2) __syncthreads();
      auto stage_tile = [&](auto act_tag) {
        constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
        for (int f = 0; f < NB; ++f) {
          const int co = co0 + 16 * f + 4 * g;
          float b[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) b[i] = (a.bias && co + i < a.cout) ? a.bias[co + i] : 0.f;
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            T o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float v = acc[m][f][i] + b[i];
              if constexpr (ACT == 1) v = v * sigmoidf_(v);
              o[i] = from_f32<T>(co + i < a.cout ? v : 0.f);
            }
            *(half4_t*)(stg + (16 * m + c) * OBS + 16 * f + 4 * g) = __builtin_bit_cast(half4_t, o);
          }
        }
      };
      if (a.act == 1) stage_tile(std::integral_constant<int, 1>{});
      else stage_tile(std::integral_constant<int, 0>{});
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int nch = cpad - co0 < 16 * NB ? cpad - co0 : 16 * NB;  // a multiple of 8
      const int ppp = nch >> 3;                                       // 16-byte pieces per pixel
      for (int i = lane; i < 64 * ppp; i += 64) {
        const int px = i / ppp, j = i - px * ppp;
        if (p0 + px < P) *(intx4*)(out + (int64_t)(p0 + px) * a.out_cs + co0 + 8 * j) = *(const intx4*)(stg + px * OBS + 8 * j);
      }
      return;
    }
  }
  auto epilogue = [&](auto act_tag) {  // activation as a template argument: no per-value branch
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int f = 0; f < NB; ++f) {
      const int co = co0 + 16 * f + 4 * g;
      if (co >= cpad) continue;
      float b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) b[i] = (a.bias && co + i < a.cout) ? a.bias[co + i] : 0.f;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (!pok[m]) continue;
        T o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = acc[m][f][i] + b[i];
          if constexpr (ACT == 1) v = v * sigmoidf_(v);
          o[i] = from_f32<T>(co + i < a.cout ? v : 0.f);
        }
        T* dst = out + (int64_t)(p0 + 16 * m + c) * a.out_cs + co;
        if (co + 4 <= cpad) {
          *(half4_t*)dst = __builtin_bit_cast(half4_t, o);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (co + i < cpad) dst[i] = o[i];
        }
      }
    }
  };
  if (a.act == 1) epilogue(std::integral_constant<int, 1>{});
  else epilogue(std::integral_constant<int, 0>{});
}

// The NHWC fast path covers 16-bit NHWC -> NHWC without pooling when Cin and the input channel
// stride are multiples of 8 (16-byte pieces) and the output stride a multiple of 4 (8-byte stores).
static bool nhwc_fast_ok(const kad_gemm_args& a) {
  return a.dtype != KAD_F32 && a.pool == 1 && a.in_layout == KAD_NHWC && a.out_layout == KAD_NHWC &&
         a.cin % 8 == 0 && a.x_cs % 8 == 0 && a.out_cs % 4 == 0 && ((uintptr_t)a.x % 16) == 0 &&
         ((uintptr_t)a.out % 8) == 0;
}

#ifndef KAD_GH_WLDS_KB
#define KAD_GH_WLDS_KB 64
#endif
#ifndef KAD_GH_STAGE
#define KAD_GH_STAGE 1
#endif
template <typename T, int NB>
static void launch_gemm_nhwc_nb(const kad_gemm_args& a, hipStream_t st) {
  const int P = a.h * a.w, cin_pad = round_up(a.cin, 32);
  const int tiles_px = ceil_div(P, GH_PXW), co_blocks = ceil_div(round_up(a.cout, 8), NB * 16);
  const int total = a.n * tiles_px * co_blocks;
  const size_t wlds = (size_t)NB * (cin_pad / 32) * 1024;  // the block's weight fragments
  if (wlds <= (size_t)KAD_GH_WLDS_KB * 1024) {
    // The output staged through LDS when 16-byte pieces line up (one tile per wave behind the
    // weights) and the extra LDS keeps the blocks per CU that the registers allow (three at NB <= 4,
    // two at NB = 5): staging that cost a block per CU measured slower (360 -> 128 @100^2: 51 -> 71
    // us) than the writes it saves.
    // Where the weights take at least as much LDS as the tiles, the tiles reuse it after a barrier.
    const size_t stg = (size_t)GH_WAVES * 64 * (16 * NB + 8) * sizeof(T);
    const bool aligned = KAD_GH_STAGE && a.out_cs % 8 == 0 && ((uintptr_t)a.out & 15) == 0;
    const int stage = !aligned ? 0 : wlds >= stg ? 2 : (wlds + stg) * (NB <= 4 ? 3 : 2) <= 160 * 1024 ? 1 : 0;
    const size_t lds = wlds + (stage == 1 ? stg : 0);
    allow_lds(gemm_nhwc_kernel<T, NB, true>, lds);
    hipLaunchKernelGGL((gemm_nhwc_kernel<T, NB, true>), dim3(co_blocks * round_up(ceil_div(a.n * tiles_px, GH_WAVES), 8)),
                       dim3(64 * GH_WAVES), lds, st, a, P, tiles_px, co_blocks, total, cin_pad, stage);
  } else {
    hipLaunchKernelGGL((gemm_nhwc_kernel<T, NB, false>), dim3(ceil_div(total, GH_WAVES)), dim3(64 * GH_WAVES), 0, st,
                       a, P, tiles_px, co_blocks, total, cin_pad, 0);
  }
}

// Output-channel fragments per wave (channel blocks of 16 NB): the fewest padded columns plus 16
// per channel block, among the widths whose weight fragments fit the LDS staging (NB x Cin_pad / 32
// KB <= 64), ties to the narrower block; then a launch of fewer than 200 blocks narrows its channel
// blocks.  Measured at batch 16, fp16 (us for NB = 1 .. 5): 512 -> 288 at 25^2: 28.7 23.2 18.3 19.6
// 28.5 (NB = 5 does not fit the staging); 384 -> 216 at 50^2: 59.7 43.7 37.2 33.9 28.9; 256 -> 144
// at 100^2: 104.9 73.4 53.8 61.5 57.9; 432 -> 256 at 25^2: 21.1 16.5 15.8 16.8 20.9.  NB <= 5: from
// NB = 6 the accumulators and the prefetched fragments take more than 256 registers, one wave per
// SIMD, and the loads' latency is no longer hidden (NB = 8 measured 1.1-1.8x slower than 4 or 5).
static int nhwc_pick_nb(int cout, int cin_pad, long tiles) {
  const int c8 = round_up(cout, 8), nk = cin_pad / 32;
  int best = 1;
  long best_cost = -1;
  for (int nb = 1; nb <= 5; ++nb) {
    if (nb > 1 && (long)nb * nk * 1024 > (long)KAD_GH_WLDS_KB * 1024) break;
    const int blocks = ceil_div(c8, nb * 16);
    const long cost = (long)blocks * nb * 16 + 16L * blocks;
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = nb;
    }
  }
  while (best > 1 && ceil_div(tiles, GH_WAVES) * ceil_div(c8, best * 16) < 200) --best;
  return best;
}

template <typename T>
static int launch_gemm_nhwc(const kad_gemm_args& a, hipStream_t st) {
  switch (nhwc_pick_nb(a.cout, round_up(a.cin, 32), (long)a.n * ceil_div(a.h * a.w, GH_PXW))) {
    case 1: launch_gemm_nhwc_nb<T, 1>(a, st); break;
    case 2: launch_gemm_nhwc_nb<T, 2>(a, st); break;
    case 3: launch_gemm_nhwc_nb<T, 3>(a, st); break;
    case 4: launch_gemm_nhwc_nb<T, 4>(a, st); break;
    default: launch_gemm_nhwc_nb<T, 5>(a, st); break;
  }
  return check_launch("kad_gemm1x1_fwd");
}

template <typename T, int NBF>
static int launch_gemm(const kad_gemm_args& a, hipStream_t st, int hp, int wp) {
  const int P = hp * wp;
  const int tiles = ceil_div(P, GM_TILE);
  const int ncols = a.out_layout == KAD_NHWC ? round_up(a.cout, 8) : a.cout;
  dim3 grid(tiles, ceil_div(ncols, NBF * 16), a.n);
  hipLaunchKernelGGL((gemm1x1_kernel<T, NBF>), grid, dim3(GM_THREADS), 0, st, a, hp, wp, tiles,
                     round_up(a.cin, 32));
  return check_launch("kad_gemm1x1_fwd");
}

template <typename T, int NW, int PXT>
static void launch_gemm_nchw_nw(const kad_gemm_args& a, hipStream_t st) {
  const int P = a.h * a.w;
  const int tiles_px = ceil_div(P, PXT), co_blocks = ceil_div(a.cout, NW * GN_WCO);
  const int total = a.n * tiles_px * co_blocks;
  const int cin_pad = round_up(a.cin, 32);
  dim3 grid(round_up(total, 8));
  if (P % 8 == 0)
    hipLaunchKernelGGL((gemm_nchw_kernel<T, true, NW, PXT>), grid, dim3(64 * NW), 0, st, a, P, tiles_px, co_blocks,
                       total, cin_pad);
  else
    hipLaunchKernelGGL((gemm_nchw_kernel<T, false, NW, PXT>), grid, dim3(64 * NW), 0, st, a, P, tiles_px, co_blocks,
                       total, cin_pad);
}

// 4-wave blocks, two per CU: independent blocks drift apart, so one block's LDS
// reads and barrier waits overlap the other's MFMAs (8-wave blocks, one per CU,
// keep both waves of a SIMD in lockstep and measured slower: 50-55 us against
// 47.7 us for [16,512,50,50]).  What remains per block (MI355X, 2 blocks per
// CU): ~1.6k cycles per k-step against 0.5k of MFMA per wave, and an epilogue of
// ~14k cycles that is mostly SiLU (exp and rcp are quarter-rate: ~6k cycles per
// wave for its 128 values) run by both blocks of a CU at the same time.
//
// Pixel tile: 128 for launches of at least two full rounds of 128-pixel blocks (two per CU),
// else 64 (three blocks per CU, half the work per block).  Measured (MI355X, fp16, us, 128 -> 64):
// [16,512,50,50] -> 512 + SiLU 43-45 -> 40-42; [8,256,100,100] -> 256 27 -> 25; [2,512,26,26]
// -> 512 20.5 -> 11.7; [8,768,50,50] -> 512 unchanged (30-33); [8,256,100,100] -> 512 45-46 -> 47.
template <typename T>
static int launch_gemm_nchw(const kad_gemm_args& a, hipStream_t st) {
  const int64_t items128 = (int64_t)a.n * ceil_div(a.h * a.w, 128) * ceil_div(a.cout, 4 * GN_WCO);
  if (items128 >= 2 * 2 * 256)
    launch_gemm_nchw_nw<T, 4, 128>(a, st);
  else
    launch_gemm_nchw_nw<T, 4, 64>(a, st);
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
  if constexpr (sizeof(T) == 2) {
    if (nchw_fast_ok(a)) return launch_gemm_nchw<T>(a, st);
    if (nhwc_fast_ok(a)) return launch_gemm_nhwc<T>(a, st);
  }
  const int ncols = a.out_layout == KAD_NHWC ? round_up(a.cout, 8) : a.cout;
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
  // rows cover every 16-wide column block a launch can touch (NHWC padding included);
  // row layout followed by the fragment-ordered copy
  return 2 * (int64_t)round_up(round_up(cout, 8), 128) * round_up(cin, 32);
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
  KAD_CHECK_ARG(a->out_layout == KAD_NCHW || (a->out_layout == KAD_NHWC && a->out_cs >= a->cout),
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
