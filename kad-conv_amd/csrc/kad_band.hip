// Band pyramid: KADConv's three branch projections from a 16-bit NCHW input,
// one block per (image, band of 4 full rows).
//
//   y_b = conv1x1_b(avg_pool2d(x, 2^b)) + bias_b,  b = 0, 1, 2
//   (KAD-Conv/kadconv/kad_conv.py:101,115), plus LCSA's axial partial sums of
//   every y_b (kad_conv.py:26-27).
//
// The general pyramid kernel (kad_pyramid.hip) works on 4 x 32 tiles; at the
// KADConv(256) shape it is bound by per-block latency (barriers behind late
// loads, a long epilogue) at a fifth of HBM speed.  This kernel streams a
// whole 4-row band (4 W pixels, W <= 128) of every input channel as one
// contiguous 8 W-byte run per channel, so:
//  * the x slice of a K step (32 channels) is 32 contiguous runs, loaded two
//    steps ahead into registers (16-byte pieces, 64 KB in flight per CU) and
//    written into one of two LDS stages [32 ch][512 px] in the image's own
//    pixel order: no transpose pass;
//  * MFMA operands: weights are the A operand (16 output channels x 32 input
//    channels, the fragment-ordered packed copy, one 16-byte load per lane);
//    pixels are the B operand, built with no transpose pass: lane (c, g) reads
//    channels 8 g .. 8 g + 7 of the 8 pixels 8 c .. 8 c + 7 of a 128-pixel
//    group (eight 16-byte LDS reads), and fragment j takes element j of each,
//    i.e. column c of fragment j is pixel 8 c + j;
//  * the 2 x 2 and 4 x 4 means are formed once per K step by a pooling pass
//    (fp32 sums of the 16-bit inputs, one rounding to 16 bits, as PyTorch's
//    avg_pool2d) into small LDS slices [32 ch][2 x 64] and [32 ch][32]; the
//    pooled branches' MFMAs run one step behind, so one barrier per step
//    covers both;
//  * the epilogue stages all three y_b of the band in LDS (16-bit, pad
//    channels zero), stores them as contiguous 16-byte runs (the band is
//    contiguous in every NHWC output), and forms the row partial sums per
//    32 >> b column slice and the column partial sums over the band's rows
//    from the rounded values, in the layout of kad_pyramid_tiles (ntx column
//    slices of 32 >> b columns, nty = H / 4 row slices).
// Wave w: branch-0 pixel group w / 2 (x all 16 * MH output channels of half
// w % 2), and for w < 2 MH the pooled branches' output fragment w.
#include <type_traits>

#include "kad_common.h"

namespace kad {

constexpr int BD_WAVES = 4, BD_THREADS = 64 * BD_WAVES;  // one wave per SIMD: up to 512 registers each
constexpr int BD_SLOT = 512;                         // pixels per channel in an x stage (4 rows x W, W <= 128)
constexpr int BD_XS = 32 * BD_SLOT;                  // elements per x stage (32 KB)
constexpr int BD_XSA = BD_XS + 4096;                 // allocated per stage: the epilogue stages outputs there too
constexpr int BD_P2 = 32 * 128;                      // 2 x 2 means: [32 ch][2 pooled rows x 64]
constexpr int BD_P4 = 32 * 32;                       // 4 x 4 means: [32 ch][32]

template <typename T> struct BdOps;
template <> struct BdOps<half_t> {
  typedef half8_t frag;
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct BdOps<bf16_t> {
  typedef bf16x8_t frag;
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// 4 x 16-bit values at p (8-byte aligned) as fp32.
template <typename T>
__device__ __forceinline__ void ld4f(const T* p, float* v) {
  typedef T t4 __attribute__((ext_vector_type(4)));
  const t4 q = *(const t4*)p;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (float)q[i];
}

// MF = 16-channel output fragments per branch (2, 4 or 6).
template <typename T, int MF>
__global__ __launch_bounds__(BD_THREADS, 1) void band_pyramid_kernel(kad_pyramid_args a, int nbands, int nk) {
  typedef typename BdOps<T>::frag frag;
  typedef T t2 __attribute__((ext_vector_type(2)));
  typedef T t4 __attribute__((ext_vector_type(4)));
  // one __shared__ object per x stage: the buffer -> LDS loads into one stage are then known not to
  // alias reads of the others, so the compiler's wait counts stay per stage
  __shared__ __align__(16) T xsA[BD_XSA];
  __shared__ __align__(16) T xsB[BD_XSA];
  __shared__ __align__(16) T xsC[BD_XSA];
  __shared__ __align__(16) T p2s[2 * BD_P2];
  __shared__ __align__(16) T p4s[2 * BD_P4];
  __shared__ __align__(16) float s_bias[3][128];  // the branches' biases (0 past Cout)

  const int bid = blockIdx.x;
  const int n = bid / nbands, band = bid - n * nbands;
  const int tid = threadIdx.x, lane = tid & 63, cl = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int W = a.w, HW = a.h * a.w, W1 = W >> 1, W2 = W >> 2, bandpx = 4 * W;
  const int cin = a.cin;
  // biases: loaded first (the oldest load of the wave), written to LDS before the first step
  float bias_v[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int t = tid + BD_THREADS * u, b = t >> 7, c = t & 127;
    bias_v[u] = (b < 3 && a.bias[b] != nullptr && c < a.cout[b]) ? a.bias[b][c] : 0.f;
  }

  // ---- x: wave w moves channels 8 w .. 8 w + 7 of each step; lane l the l-th 16-byte piece of a
  // channel's band (pieces past the band read 0), landing at [channel][8 l] of the stage -----------------
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((int64_t)a.n * cin * HW * 2));
  const uint32_t xlane = 8 * lane < bandpx ? 16u * lane : KAD_OOB;
  const int64_t xrow0 = (int64_t)n * cin + 8 * wave;  // plane of this wave's first channel (step 0)
  auto dma_x = [&](int k, T* st) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int ci = 32 * k + 8 * wave + u;
      const uint32_t soff = (uint32_t)((xrow0 + 32 * k + u) * HW + (int64_t)band * bandpx) * 2u;
      dma16(rx, (char*)(st + (8 * wave + u) * BD_SLOT), ci < cin ? xlane : KAD_OOB, ci < cin ? soff : 0u);
    }
  };

  // ---- roles and weights --------------------------------------------------------------------------
  // Waves 0-2 (role A): branch-0 pixel group w (128 pixels, every output fragment) on step k, and
  // output fragments 2 w, 2 w + 1 of branch 2 (the 4 x 4 means, 2 pixel fragments) on step k - 1.
  // Wave 3 (role B): branch 1 (the 2 x 2 means, one 128-pixel group) on step k - 1, and branch 0's tail
  // (the band's last 4 W - 128 q_full <= 16 pixels, one pixel fragment) on step k.
  // Both roles keep MF x 8 main accumulators and up to MF extra ones.
  const bool role_a = wave < 3;
  const int ngrp = bandpx >> 7, tail = bandpx - 128 * ngrp;
  const bool main_b0 = role_a && wave < ngrp;  // branch-0 group of this wave holds pixels
  const bool x_tail = !role_a && tail > 0;
  __amdgpu_buffer_rsrc_t rw[3];
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const int cout_pk = round_up(round_up(a.cout[b], 8), 128);
    rw[b] = make_rsrc((const T*)a.wpack[b] + (int64_t)cout_pk * nk * 32, (uint32_t)(cout_pk * nk * 32 * 2));
  }
  // every wave issues the same loads per step (fragments it does not use read out of range): the K
  // loop's explicit wait counts are constants
  auto wfrag = [&](int b, int mf, int ks, bool on) __attribute__((always_inline)) -> frag {
    const uint32_t off = (on && ks >= 0 && ks < nk) ? (uint32_t)(((mf * nk + ks) * 64 + lane) * 16) : KAD_OOB;
    return __builtin_bit_cast(frag, __builtin_amdgcn_raw_buffer_load_b128(rw[b], off, 0, 0));
  };
  constexpr int NXS = MF < 4 ? 4 : MF;  // extra slots: role A needs 4 (2 fragments x 2 pixel fragments)
  frag wm[MF], wx[NXS];
  // RA: role A (compile-time, so each role's loop is code of its own)
  auto load_w = [&](auto ra, int k) __attribute__((always_inline)) {
    constexpr bool RA = decltype(ra)::value;
#pragma unroll
    for (int m = 0; m < MF; ++m)  // main: branch 0 at step k (A); branch 1 at step k - 1 (B)
      wm[m] = RA ? wfrag(0, m, k, main_b0) : wfrag(1, m, k - 1, true);
#pragma unroll
    for (int m = 0; m < NXS; ++m)  // extra slot m: A: branch-2 fragment 2 w + (m & 1) at step k - 1;
      wx[m] = RA ? wfrag(2, 2 * wave + (m & 1), k - 1, m < 4 && 2 * wave + (m & 1) < MF)
                 : wfrag(0, m, k, x_tail && m < MF);  // B: branch-0 tail, fragment m, at step k
  };

  floatx4 acc[MF][8], accx[NXS];
#pragma unroll
  for (int m = 0; m < MF; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < NXS; ++m) accx[m] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Both roles run the same MFMA sequences (one copy of each accumulator chain; only the operand
  // sources differ by role):
  // main: 8 pixel fragments of a 128-pixel group x MF output fragments.  Role A reads the x stage,
  // role B the 2 x 2 means of step k - 1, each from a pointer based on one __shared__ object (a
  // pointer selected between two objects would make the compiler wait for every load into LDS)
  auto mfma_main = [&](auto ra, int k, const T* cur) __attribute__((always_inline)) {
    constexpr bool RA = decltype(ra)::value;
    frag raw[8];
    if constexpr (RA) {
      const T* s = cur + 8 * g * BD_SLOT + 128 * wave + 8 * cl;
#pragma unroll
      for (int r = 0; r < 8; ++r) raw[r] = *(const frag*)(s + r * BD_SLOT);
    } else {
      const T* s = p2s + ((k - 1) & 1) * BD_P2 + 8 * g * 128 + 8 * cl;
#pragma unroll
      for (int r = 0; r < 8; ++r) raw[r] = *(const frag*)(s + r * 128);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      frag b;
#pragma unroll
      for (int r = 0; r < 8; ++r) b[r] = raw[r][j];
#pragma unroll
      for (int m = 0; m < MF; ++m) acc[m][j] = BdOps<T>::mma(wm[m], b, acc[m][j]);
    }
  };
  // extra: slot m multiplies wx[m] by pixel fragment bx[(m >> 1) & 1].  Role A: the two fragments of
  // the 4 x 4 means of step k - 1 (pixel 2 c + j of fragment j), slot 2 j + e = branch-2 fragment 2 w + e.
  // Role B: the branch-0 tail of step k (pixel 128 ngrp + c) in both.
  auto mfma_extra = [&](auto ra, int k, const T* cur) __attribute__((always_inline)) {
    constexpr bool RA = decltype(ra)::value;
    frag bx[2];
    if constexpr (RA) {
      const T* s4 = p4s + ((k - 1) & 1) * BD_P4 + 8 * g * 32 + 2 * cl;
      t2 raw4[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) raw4[r] = *(const t2*)(s4 + r * 32);
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        bx[0][r] = raw4[r][0];
        bx[1][r] = raw4[r][1];
      }
    } else {
      const T* s = cur + 8 * g * BD_SLOT + 128 * ngrp + cl;
#pragma unroll
      for (int r = 0; r < 8; ++r) bx[0][r] = s[r * BD_SLOT];
      bx[1] = bx[0];
    }
#pragma unroll
    for (int m = 0; m < NXS; ++m) accx[m] = BdOps<T>::mma(wx[m], bx[(m >> 1) & 1], accx[m]);
  };

  // ---- pooling pass: 2 x 2 and 4 x 4 means of step k into the pooled slices ---------------------------
  // task 2 (ch * nseg + s) + pr = (channel, 8-column segment s, pooled row pr): the two pooled rows of
  // a segment sit in adjacent lanes (the 4 x 4 sums swap them by DPP).  Columns past the row's end read
  // the next row's pixels; they only reach pooled columns >= W / 2 (or W / 4), whose outputs are dropped.
  const int nseg = ceil_div(W1, 8), ntask = 64 * nseg;
  auto pool_pass = [&](int k, const T* cur) __attribute__((always_inline)) {
    for (int t = tid; t < ntask; t += BD_THREADS) {  // t and t ^ 1 run in one iteration, in adjacent lanes
      const int ptask = t >> 1, ppr = t & 1;
      const int pch = ptask / nseg, pseg = ptask - pch * nseg;
      const T* s = cur + pch * BD_SLOT + 16 * pseg + 2 * ppr * W;
      float s2[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float r0[4], r1[4];
        ld4f(s + 4 * u, r0);
        ld4f(s + W + 4 * u, r1);
        s2[2 * u] = ((r0[0] + r0[1]) + r1[0]) + r1[1];
        s2[2 * u + 1] = ((r0[2] + r0[3]) + r1[2]) + r1[3];
      }
      t4 lo, hi;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        lo[m] = from_f32<T>(s2[m] * 0.25f);
        hi[m] = from_f32<T>(s2[4 + m] * 0.25f);
      }
      T* d2 = p2s + (k & 1) * BD_P2 + pch * 128 + 64 * ppr + 8 * pseg;
      *(t4*)d2 = lo;
      *(t4*)(d2 + 4) = hi;
      float so[8];
#pragma unroll
      for (int m = 0; m < 8; ++m)
        so[m] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s2[m]), 0xB1, 0xf, 0xf, false));
      if (ppr == 0) {
        t4 q;
#pragma unroll
        for (int m = 0; m < 4; ++m)
          q[m] = from_f32<T>(((s2[2 * m] + s2[2 * m + 1]) + (so[2 * m] + so[2 * m + 1])) * 0.0625f);
        *(t4*)(p4s + (k & 1) * BD_P4 + pch * 32 + 4 * pseg) = q;
      }
    }
  };

  // ---- K loop ---------------------------------------------------------------------------------------
  // Step k (0 .. nk; step nk only finishes the pooled branches): wait for this wave's loads of input
  // step k (loads of later steps may stay in flight: LW per wave) and every wave's LDS traffic of the
  // previous step, barrier; refill the stage read in step k - 1 with input step k + 2; multiply branch 0
  // on step k and the pooled branches on step k - 1; load the next step's weights; pool step k.
  // Loads per wave per step: 8 x pieces + MF + NXS weight fragments; the wait of step k lets the weights
  // of step k - 1 (already consumed), the pieces of step k + 1 and the weights of step k stay outstanding.
  constexpr int LW = 2 * (MF + NXS) + 8;
  for (int t = tid; t < (2 * BD_P2 + 2 * BD_P4) / 8; t += BD_THREADS)  // finite operands for step 0
    *(intx4*)(t < 2 * BD_P2 / 8 ? p2s + 8 * t : p4s + 8 * (t - 2 * BD_P2 / 8)) = intx4{0, 0, 0, 0};
  auto step = [&](auto ra, int k, T* cur, T* refill) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(LW) : "memory");
    dma_x(k + 2, refill);
    // unconditional chains (a conditional one made the register allocator alternate the accumulators
    // between two register sets): where a role has nothing to add its weight fragments read 0 and its
    // operands finite values (zero pieces or the zeroed pooled slices), so the sums do not change
    mfma_main(ra, k, cur);
    mfma_extra(ra, k, cur);
    load_w(ra, k + 1);
    if (k < nk) pool_pass(k, cur);
  };
  // The two roles run separate copies of the loop (same barriers, same loads per step): an LDS read
  // whose pointer could come from either role's buffer would alias the loads in flight into the next
  // stages and make the compiler wait for all of them.  Steps 0 .. nk, padded to a multiple of 3 with
  // steps whose loads all read out of range (their weights are 0): every step copy runs
  // unconditionally, so the accumulators keep one register set.
  auto kloop = [&](auto ra) __attribute__((always_inline)) {
    dma_x(0, xsA);
    load_w(ra, -1);
    dma_x(1, xsB);
    load_w(ra, 0);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = tid + BD_THREADS * u;
      if (t < 3 * 128) s_bias[t >> 7][t & 127] = bias_v[u];
    }
    for (int k = 0; k <= nk; k += 3) {
      step(ra, k, xsA, xsC);
      step(ra, k + 1, xsB, xsA);
      step(ra, k + 2, xsC, xsB);
    }
  };
  if (role_a) kloop(std::true_type{});
  else kloop(std::false_type{});
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");  // no load into LDS outlives the loop

  // ---- epilogue: stage every branch's band outputs in LDS (bias added, 16-bit; pad channels come out
  // 0 because their weights and biases are 0), store them as contiguous runs (the band is contiguous
  // in every NHWC output), then form the LCSA partial sums from the rounded values in the layout of
  // kad_pyramid_tiles: row sums per column slice of 32 >> b columns (ntx slices), column sums over the
  // band's rows (slice `band` of nty).  Staging: branch-0 pixel p at [(p - 128 q) cs0] of object
  // q = min(p / 128, 2) (xsA, xsB, xsC: the tail after group 2 in xsC); branch 1 (both pooled rows) at
  // [128 cs0 + (r W / 2 + c) cs1] of xsA; branch 2 at [max(4 W - 256, 0) cs0 + c cs2] of xsC.
  const int cs0 = a.out_cs[0], cs1 = a.out_cs[1], cs2 = a.out_cs[2];
  auto obj = [&](int q) __attribute__((always_inline)) -> T* {  // q wave-uniform
    return q == 0 ? xsA : (q == 1 ? xsB : xsC);
  };
  // branch-b value at (band row r, column x), for x in a 4-column chunk starting at x0: the chunk's
  // pixels share one object (the 128-pixel boundaries r W + x = 128 k fall on multiples of 4 of x), so
  // the object is chosen from x0 (wave-uniform in the sums below) without divergent selects
  auto zat0 = [&](int r, int x0, int x) __attribute__((always_inline)) -> T* {
    const int q = min(__builtin_amdgcn_readfirstlane(r * W + x0) >> 7, 2);
    return obj(q) + (r * W + x - 128 * q) * cs0;
  };
  T* const z1s = xsA + 128 * cs0;
  auto zat1 = [&](int r, int, int x) __attribute__((always_inline)) -> T* { return z1s + (r * W1 + x) * cs1; };
  T* const z2s = xsC + max(bandpx - 256, 0) * cs0;
  auto zat2 = [&](int, int, int x) __attribute__((always_inline)) -> T* { return z2s + x * cs2; };
  auto bias4 = [&](int b, int m) __attribute__((always_inline)) -> floatx4 {  // channels 16 m + 4 g ..
    return *(const floatx4*)&s_bias[b][(16 * m + 4 * g) & 127];
  };
  auto put4 = [&](T* dst, const floatx4& v, const floatx4& bias) __attribute__((always_inline)) {
    t4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = from_f32<T>(v[i] + bias[i]);
    *(t4*)dst = o;
  };
  if (role_a) {
    if (main_b0) {  // branch 0, pixels 128 w + 8 c + j
      T* zb = obj(wave) + 8 * cl * cs0 + 4 * g;
#pragma unroll
      for (int m = 0; m < MF; ++m) {
        if (16 * m + 4 * g >= cs0) continue;
        const floatx4 bv = bias4(0, m);
#pragma unroll
        for (int j = 0; j < 8; ++j) put4(zb + j * cs0 + 16 * m, acc[m][j], bv);
      }
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {  // branch 2, fragment 2 w + e, pixels 2 c + j
      const int mf = 2 * wave + e;
      if (mf >= MF || 16 * mf + 4 * g >= cs2) continue;
      const floatx4 bv = bias4(2, mf);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (2 * cl + j < W2) put4(z2s + (2 * cl + j) * cs2 + 16 * mf + 4 * g, accx[2 * j + e], bv);
    }
  } else {
    const int pr = cl >> 3;
#pragma unroll
    for (int m = 0; m < MF; ++m) {  // branch 1, pooled row c / 8, columns 8 (c & 7) + j
      if (16 * m + 4 * g >= cs1) continue;
      const floatx4 bv = bias4(1, m);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int pc = 8 * (cl & 7) + j;
        if (pc < W1) put4(z1s + (pr * W1 + pc) * cs1 + 16 * m + 4 * g, acc[m][j], bv);
      }
    }
    if (x_tail && cl < tail) {  // branch-0 tail, pixel 128 ngrp + c
#pragma unroll
      for (int m = 0; m < MF; ++m)
        if (16 * m + 4 * g < cs0) put4(obj(min(ngrp, 2)) + (128 * (ngrp - min(ngrp, 2)) + cl) * cs0 + 16 * m + 4 * g, accx[m], bias4(0, m));
    }
  }
  __syncthreads();

  // stores: contiguous LDS spans to contiguous output runs, every LDS read of a round before its stores
  auto copy = [&](const T* src, T* dst, int pieces) __attribute__((always_inline)) {
    for (int t0 = tid; t0 < pieces; t0 += 4 * BD_THREADS) {
      intx4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *(const intx4*)(src + 8 * min(t0 + u * BD_THREADS, pieces - 1));
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (t0 + u * BD_THREADS < pieces) *(intx4*)(dst + 8 * (t0 + u * BD_THREADS)) = v[u];
    }
  };
  {
    T* o0 = (T*)a.out[0] + ((int64_t)n * a.h + 4 * band) * W * cs0;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int npx = q < 2 ? min(128, bandpx - 128 * q) : bandpx - 256;
      if (npx > 0) copy(obj(q), o0 + 128 * q * cs0, npx * cs0 / 8);
    }
    T* o1 = (T*)a.out[1] + ((int64_t)n * (a.h >> 1) + 2 * band) * W1 * cs1;
    copy(z1s, o1, 2 * W1 * cs1 / 8);
    T* o2 = (T*)a.out[2] + ((int64_t)n * (a.h >> 2) + band) * W2 * cs2;
    copy(z2s, o2, W2 * cs2 / 8);
  }

  // partial sums of branch B from its staged values.  Wave w takes column slice i = w (CW = 32 >> B
  // columns, LPS = CW / 4 chunks of 4), lane = (channel group gr = lane / 4, column u = lane & 3 of
  // the chunk).  Per chunk a lane adds the band's rows of its column (in row order) into the column
  // sum it writes, and each row's value into that row's partial (chunks in order); the chunk's four
  // lanes then add their row partials by DPP (quad swaps: every lane of the quad ends with the same sum).
  auto sums = [&](auto bt, auto zat) __attribute__((always_inline)) {
    constexpr int B = decltype(bt)::value, R = 4 >> B, CW = 32 >> B, LPS = CW / 4;
    if (a.rowpart[B] == nullptr) return;
    const int wbb = W >> B, cout = a.cout[B], ngr = ceil_div(cout, 8);
    const int u = lane & 3, gr = lane >> 2;
    const bool lane_on = gr < ngr;
    for (int i = wave; i < a.ntx; i += BD_WAVES) {
      float rs[R][8];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) rs[r][e] = 0.f;
#pragma unroll 1
      for (int c = 0; c < LPS; ++c) {  // rolled: the epilogue runs once per block
        const int x0 = CW * i + 4 * c, x = x0 + u;
        if (x0 >= wbb) break;
        const bool ok = lane_on && x < wbb;
        t4 v[2 * R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const T* z = zat(r, x0, ok ? x : x0) + 8 * (lane_on ? gr : 0);
          v[2 * r] = *(const t4*)z;
          v[2 * r + 1] = *(const t4*)(z + 4);
        }
        float cs_[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float f0 = ok ? (float)v[2 * r][e] : 0.f, f1 = ok ? (float)v[2 * r + 1][e] : 0.f;
            cs_[e] += f0;
            cs_[4 + e] += f1;
            rs[r][e] += f0;
            rs[r][4 + e] += f1;
          }
        if (ok) {
          float* dst = a.colpart[B] + (((int64_t)n * a.nty + band) * wbb + x) * cout + 8 * gr;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (8 * gr + e < cout) dst[e] = cs_[e];
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float vv = rs[r][e];
          vv += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(vv), 0xB1, 0xf, 0xf, false));  // lane ^ 1
          vv += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(vv), 0x4E, 0xf, 0xf, false));  // lane ^ 2
          rs[r][e] = vv;
        }
      if (lane_on && u == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float* dst = a.rowpart[B] + (((int64_t)n * a.ntx + i) * (a.h >> B) + R * band + r) * cout + 8 * gr;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (8 * gr + e < cout) dst[e] = rs[r][e];
        }
      }
    }
  };
  sums(std::integral_constant<int, 0>{}, zat0);
  sums(std::integral_constant<int, 1>{}, zat1);
  sums(std::integral_constant<int, 2>{}, zat2);
}

template <typename T, int MF>
static void launch_band(const kad_pyramid_args& a, hipStream_t st) {
  const int nbands = a.h / 4, nk = round_up(a.cin, 32) / 32;
  hipLaunchKernelGGL((band_pyramid_kernel<T, MF>), dim3(a.n * nbands), dim3(BD_THREADS), 0, st, a, nbands, nk);
}

// The band kernel's launch, or 1 when the arguments are not a case it handles (the caller then
// runs the general pyramid kernel): 16-bit NCHW input, three branches, H and W multiples of 4,
// W <= 128, every branch at most 96 output channels (out_cs <= 32 MH), the band's outputs staged
// within the LDS budget, ntx / nty from kad_pyramid_tiles.
int band_pyramid(const kad_pyramid_args& a, hipStream_t st) {
  if (a.in_layout != KAD_NCHW || (a.dtype != KAD_F16 && a.dtype != KAD_BF16) || a.nb != 3) return 1;
  if (a.h % 4 || a.w % 4 || a.w < 8 || a.w > 100 || a.h < 4) return 1;
  if ((4 * a.w) % 128 > 16) return 1;  // at most 3 full pixel groups and a tail of one fragment
  if ((int64_t)a.n * a.cin * a.h * a.w * 2 >= (1ll << 31) || (uintptr_t)a.x % 16) return 1;
  int mf = 0;
  for (int b = 0; b < 3; ++b) mf = max(mf, ceil_div(a.cout[b], 16));
  const int mh = ceil_div(mf, 2);
  if (mh > 3) return 1;
  for (int b = 0; b < 3; ++b)
    if (a.out_cs[b] > 32 * mh) return 1;
  // epilogue staging: 128 branch-0 pixels per stage object (the last also the tail, then branch 2),
  // branch 1 behind the first
  if (128 * a.out_cs[0] + a.w * a.out_cs[1] > BD_XSA ||
      max(4 * a.w - 256, 0) * a.out_cs[0] + (a.w / 4) * a.out_cs[2] > BD_XSA)
    return 1;
  if (a.dtype == KAD_F16) {
    if (mh == 1) launch_band<half_t, 2>(a, st);
    else if (mh == 2) launch_band<half_t, 4>(a, st);
    else launch_band<half_t, 6>(a, st);
  } else {
    if (mh == 1) launch_band<bf16_t, 2>(a, st);
    else if (mh == 2) launch_band<bf16_t, 4>(a, st);
    else launch_band<bf16_t, 6>(a, st);
  }
  return check_launch("kad_pyramid_proj (band)");
}

}  // namespace kad
