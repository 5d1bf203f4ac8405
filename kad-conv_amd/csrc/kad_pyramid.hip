// One-pass branch pyramid for KADConv: the input is read once and every
// branch's avg-pool + 1x1 projection is computed from the same tile
// (KAD-Conv/kadconv/kad_conv.py:101,115: y_i = conv1x1_i(avg_pool2d(x, 2^i))),
// together with the LCSA axial partial sums of every y_i (kad_conv.py:26-27,39).
//
// Tile: 4 rows x 32 columns of x (128 px).  Branch b sees (4 >> b) x (32 >> b)
// pooled pixels of it (floor-mode windows never straddle tiles because tiles are
// aligned to the largest window, 4).  Per K step of 32 input channels the block
// stages in LDS: the x slice [128 px][32 ch] (transposed on the way in from
// NCHW), its 2x2 and 4x4 averages, and the three branches' weight slices; the
// four waves then run v_mfma_f32_16x16x32 in a 2 x 2 split (pixel halves x
// column halves).  The epilogue goes through LDS: bias, 16-byte NHWC stores of
// y_b (pad channels zeroed) and deterministic per-tile row / column sums of the
// fp32 results, from which kad_lcsa_mask forms the axial means.
//
// The reference runs these as separate cuDNN 1x1 convs after separate pooling
// kernels, one branch per stream (acceleration/kadc_fused_parallel.py:74-103,
// kadc_fused_sm75.py:707-726) and reduces rows/columns again inside LCSA
// (kadc_fused_sm75.py:830-888).
#include "kad_common.h"

namespace kad {

int band_pyramid(const kad_pyramid_args& a, hipStream_t st);  // kad_band.hip; 1 = not its case

constexpr int PY_TR = 4, PY_TC = 32, PY_TILE = PY_TR * PY_TC;
constexpr int PY_THREADS = 256;

__device__ __forceinline__ int nbf_sel(const int* nbf, int b) { return b == 0 ? nbf[0] : (b == 1 ? nbf[1] : nbf[2]); }
__device__ __forceinline__ const void* sel3(const void* const* p, int b) { return b == 0 ? p[0] : (b == 1 ? p[1] : p[2]); }

template <typename T> struct PyLds { static constexpr int lda = 40; };   // 32 + 8 halves (80 B rows)
template <> struct PyLds<float> { static constexpr int lda = 36; };      // 32 + 4 floats

template <typename T>
__device__ __forceinline__ floatx4 py_mma(const T* a, const T* b, floatx4 c) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
    return c;
  } else if constexpr (__is_same(T, half_t)) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8_t*)a, *(const half8_t*)b, c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8_t*)a, *(const bf16x8_t*)b, c, 0, 0, 0);
  }
}

// Eight elements of T held in registers as raw bits: one uint4 for 16-bit
// types, two for fp32 (only .lo used by 16-bit types).
struct Raw8 { uint4 lo, hi; };

template <typename T>
__device__ __forceinline__ T raw_get(const Raw8& r, int j) {
  if constexpr (sizeof(T) == 2) {
    const unsigned w = j < 2 ? r.lo.x : j < 4 ? r.lo.y : j < 6 ? r.lo.z : r.lo.w;
    const unsigned short hbits = (unsigned short)((j & 1) ? (w >> 16) : (w & 0xffffu));
    return __builtin_bit_cast(T, hbits);
  } else {
    const uint4& q = j < 4 ? r.lo : r.hi;
    const int k = j & 3;
    const unsigned w = k == 0 ? q.x : k == 1 ? q.y : k == 2 ? q.z : q.w;
    return __builtin_bit_cast(T, w);
  }
}

// Eight elements of T packed as raw bits (inverse of raw_get).
template <typename T>
__device__ __forceinline__ Raw8 raw_pack(const T (&t)[8]) {
  Raw8 r;
  if constexpr (sizeof(T) == 2) {
    unsigned w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (unsigned)__builtin_bit_cast(unsigned short, t[2 * j]) |
             ((unsigned)__builtin_bit_cast(unsigned short, t[2 * j + 1]) << 16);
    r.lo = uint4{w[0], w[1], w[2], w[3]};
    r.hi = uint4{0u, 0u, 0u, 0u};
  } else {
    r.lo = uint4{__builtin_bit_cast(unsigned, t[0]), __builtin_bit_cast(unsigned, t[1]),
                 __builtin_bit_cast(unsigned, t[2]), __builtin_bit_cast(unsigned, t[3])};
    r.hi = uint4{__builtin_bit_cast(unsigned, t[4]), __builtin_bit_cast(unsigned, t[5]),
                 __builtin_bit_cast(unsigned, t[6]), __builtin_bit_cast(unsigned, t[7])};
  }
  return r;
}

// 8 consecutive elements at p, the first `valid` real, the rest 0.
template <typename T>
__device__ __forceinline__ Raw8 load8_raw(const T* p, int valid) {
  Raw8 r;
  r.lo = uint4{0u, 0u, 0u, 0u};
  r.hi = r.lo;
  const uintptr_t addr = (uintptr_t)p;
  if constexpr (sizeof(T) == 2) {
    if (valid == 8 && (addr & 15) == 0) {
      r.lo = *(const uint4*)p;
    } else if (valid == 8 && (addr & 7) == 0) {
      const uint2 a0 = ((const uint2*)p)[0], a1 = ((const uint2*)p)[1];
      r.lo = uint4{a0.x, a0.y, a1.x, a1.y};
    } else {
      unsigned w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const unsigned v = j < valid ? (unsigned)__builtin_bit_cast(unsigned short, p[j]) : 0u;
        w[j >> 1] |= (j & 1) ? (v << 16) : v;
      }
      r.lo = uint4{w[0], w[1], w[2], w[3]};
    }
  } else {
    if (valid == 8 && (addr & 15) == 0) {
      r.lo = ((const uint4*)p)[0];
      r.hi = ((const uint4*)p)[1];
    } else {
      unsigned w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = j < valid ? __builtin_bit_cast(unsigned, p[j]) : 0u;
      r.lo = uint4{w[0], w[1], w[2], w[3]};
      r.hi = uint4{w[4], w[5], w[6], w[7]};
    }
  }
  return r;
}

template <typename T>
__device__ __forceinline__ void store8_raw(T* d, const Raw8& r) {
  *(uint4*)d = r.lo;
  if constexpr (sizeof(T) == 4) *(uint4*)(d + 4) = r.hi;
}

template <typename T>
__device__ __forceinline__ Raw8 load8_full(const T* p) {
  Raw8 r;
  r.lo = *(const uint4*)p;
  if constexpr (sizeof(T) == 4) r.hi = *(const uint4*)(p + 4);
  else r.hi = uint4{0u, 0u, 0u, 0u};
  return r;
}

// 8 consecutive elements at p (8-byte aligned), the first `valid` (0, 4 or 8)
// real: two predicated 8-byte loads for 16-bit types, two 16-byte loads for
// fp32 -- no per-lane branching on alignment (rows with W % 4 == 0).
template <typename T>
__device__ __forceinline__ Raw8 load8_w4(const T* p, int valid) {
  Raw8 r;
  r.lo = uint4{0u, 0u, 0u, 0u};
  r.hi = r.lo;
  if constexpr (sizeof(T) == 2) {
    uint2 a0 = uint2{0u, 0u}, a1 = uint2{0u, 0u};
    if (valid >= 4) a0 = ((const uint2*)p)[0];
    if (valid == 8) a1 = ((const uint2*)p)[1];
    r.lo = uint4{a0.x, a0.y, a1.x, a1.y};
  } else {
    if (valid >= 4) r.lo = ((const uint4*)p)[0];
    if (valid == 8) r.hi = ((const uint4*)p)[1];
  }
  return r;
}

// An MFMA A/B fragment: 8 elements of T in registers.
template <typename T> struct PyFrag { T v[8]; };

template <typename T>
__device__ __forceinline__ PyFrag<T> frag_ld(const T* p) {
  PyFrag<T> f;
  if constexpr (sizeof(T) == 2) {
    *(uint4*)f.v = *(const uint4*)p;
  } else {
    *(floatx4*)f.v = *(const floatx4*)p;
    *(floatx4*)(f.v + 4) = *(const floatx4*)(p + 4);
  }
  return f;
}

template <typename T>
__device__ __forceinline__ floatx4 py_mma_f(const PyFrag<T>& a, const PyFrag<T>& b, floatx4 c) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[j], b.v[j], c, 0, 0, 0);
    return c;
  } else if constexpr (__is_same(T, half_t)) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                  0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
}

// fp16 pooling sums without separate conversions: v_fma_mix_f32 with f16 sources
// (op_sel_hi 1; op_sel picks the high half), multiplier 1.0 and one f32 rounding,
// so mix_add2(a, b) == (float)a + (float)b and mix_add1(a, c) == (float)a + c exactly.
template <int HI>
__device__ __forceinline__ float mix_add2(unsigned a, unsigned b) {
  float r;
  if constexpr (HI) asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
  else asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
template <int HI>
__device__ __forceinline__ float mix_add1(unsigned a, float c) {
  float r;
  if constexpr (HI) asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(a), "v"(c));
  else asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(a), "v"(c));
  return r;
}
__device__ __forceinline__ unsigned frag_word(const uint4& q, int w) { return w == 0 ? q.x : w == 1 ? q.y : w == 2 ? q.z : q.w; }

// Pooled input of branches 1 and 2, built straight into an A fragment (8
// channels from lane group offset g8, fp32 sums, one rounding to T): S = 2, the
// 2 x 2 window with top-left staged pixel q0; S = 4, the upper or lower half (two
// rows) of a 4 x 4 window divided by 16 -- the two halves are projected by the
// two pixel-half waves and their products added in the epilogue (linearity).
template <typename T, int S, int LDA>
__device__ __forceinline__ PyFrag<T> pooled_frag(const T* xs, int q0, int g8) {
  float acc8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc8[j] = 0.f;
  if constexpr (__is_same(T, half_t)) {  // same sums in the same order, conversions folded into the adds
    if constexpr (S == 2) {
      const uint4 s0 = *(const uint4*)(xs + q0 * LDA + g8), s1 = *(const uint4*)(xs + (q0 + 1) * LDA + g8);
      const uint4 s2 = *(const uint4*)(xs + (q0 + PY_TC) * LDA + g8);
      const uint4 s3 = *(const uint4*)(xs + (q0 + PY_TC + 1) * LDA + g8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        acc8[2 * w] = mix_add2<0>(frag_word(s0, w), frag_word(s1, w)) + mix_add2<0>(frag_word(s2, w), frag_word(s3, w));
        acc8[2 * w + 1] =
            mix_add2<1>(frag_word(s0, w), frag_word(s1, w)) + mix_add2<1>(frag_word(s2, w), frag_word(s3, w));
      }
    } else {
      uint4 sv[2 * S];
#pragma unroll
      for (int dy = 0; dy < 2; ++dy)
#pragma unroll
        for (int dx = 0; dx < S; ++dx) sv[dy * S + dx] = *(const uint4*)(xs + (q0 + dy * PY_TC + dx) * LDA + g8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float lo = mix_add2<0>(frag_word(sv[0], w), frag_word(sv[1], w));
        float hi = mix_add2<1>(frag_word(sv[0], w), frag_word(sv[1], w));
#pragma unroll
        for (int k = 2; k < 2 * S; ++k) {
          lo = mix_add1<0>(frag_word(sv[k], w), lo);
          hi = mix_add1<1>(frag_word(sv[k], w), hi);
        }
        acc8[2 * w] = lo;
        acc8[2 * w + 1] = hi;
      }
    }
  } else if constexpr (S == 2) {  // (a + b) + (c + d), as a 2x2 average is usually formed
    const PyFrag<T> s0 = frag_ld(xs + q0 * LDA + g8), s1 = frag_ld(xs + (q0 + 1) * LDA + g8);
    const PyFrag<T> s2 = frag_ld(xs + (q0 + PY_TC) * LDA + g8), s3 = frag_ld(xs + (q0 + PY_TC + 1) * LDA + g8);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc8[j] = (to_f32(s0.v[j]) + to_f32(s1.v[j])) + (to_f32(s2.v[j]) + to_f32(s3.v[j]));
  } else {  // half of a 4 x 4 window: rows q0 / PY_TC and the next, 4 columns
#pragma unroll
    for (int dy = 0; dy < 2; ++dy)
#pragma unroll
      for (int dx = 0; dx < S; ++dx) {
        const PyFrag<T> sv = frag_ld(xs + (q0 + dy * PY_TC + dx) * LDA + g8);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc8[j] += to_f32(sv.v[j]);
      }
  }
  PyFrag<T> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.v[j] = from_f32<T>(acc8[j] * (1.f / (float)(S * S)));
  return f;
}

// HB = MFMA column fragments per wave and branch (columns per block = 32 * HB).
// The widest column tiles get the whole register file (1 block per CU) instead of spilling.
template <typename T, int HB> struct PyOcc { static constexpr int v = HB <= (sizeof(T) == 4 ? 2 : 3) ? 2 : 1; };

// Weight chunks per K step of the pipelined 16-bit path: 3 branches x 2 HB
// fragments of 16 columns x 32 channels (1 KB each, MFMA lane order).
template <int HB> struct PyW { static constexpr int NCH = 6 * HB, BYTES = NCH * 1024; };

// dma = 1 (host-checked: 16-bit NCHW input, W % 4 == 0, offsets fit 31 bits):
// the K loop pipelines through LDS (weights by buffer -> LDS loads into a
// 3-stage ring, the x slice two steps ahead in registers); else the
// register-staged loop with one step of prefetch.
template <typename T, int HB>
__global__ __launch_bounds__(PY_THREADS, (PyOcc<T, HB>::v)) void pyramid_kernel(kad_pyramid_args a, int cin_pad,
                                                                                 int dma, int ncy, int grid8) {
  constexpr int LDA = PyLds<T>::lda;
  constexpr int NB = 32 * HB;              // output columns per branch per block
  constexpr int BTASKS = 3 * NB * 4;       // 16-byte weight pieces per K step (3 branches)
  constexpr int BPT = (BTASKS + PY_THREADS - 1) / PY_THREADS;
  constexpr int OBT = NB + 16 / (int)sizeof(T);   // epilogue staging row of y (T)
  constexpr bool H16 = sizeof(T) == 2;
  // 16-bit: the weight ring, one __shared__ object per stage (exact wait counts per stage)
  __shared__ __align__(16) char pw0[H16 ? PyW<HB>::BYTES : 16];
  __shared__ __align__(16) char pw1[H16 ? PyW<HB>::BYTES : 16];
  __shared__ __align__(16) char pw2[H16 ? PyW<HB>::BYTES : 16];
  // 16-bit pipelined path: the two x stages, a static object too (no wait on the weight loads to read it)
  __shared__ __align__(16) T xsd[H16 ? 2 * PY_TILE * LDA : 8];
  extern __shared__ __align__(16) char smem[];
  T* xs = (T*)smem;                   // register-staged path: [128][LDA]
  T* bs = xs + PY_TILE * LDA;         // register-staged path: [3][NB][LDA]
  // epilogue staging: y of branch 0 as T rows [128][OBT] in two 64-row halves, y of branch 1
  // [32][OBT], and the two fp32 half-window products of branch 2 [2][8][NB].  Pipelined path:
  // the three weight-ring stages (free after the K loop); register-staged path: dynamic LDS.
  constexpr int Y0H = 64 * OBT * (int)sizeof(T), Y1B = 32 * OBT * (int)sizeof(T);
  static_assert(!H16 || (Y0H <= PyW<HB>::BYTES && Y1B + 2 * 8 * NB * 4 <= PyW<HB>::BYTES),
                "epilogue staging must fit the weight ring stages");
  T* const y0a = (H16 && dma) ? (T*)pw0 : (T*)smem;
  T* const y0b = (H16 && dma) ? (T*)pw1 : (T*)(smem + Y0H);
  T* const y1s = (H16 && dma) ? (T*)pw2 : (T*)(smem + 2 * Y0H);
  float* const y2s = (float*)((char*)y1s + Y1B);

  // XCD-aware order: block b runs on XCD b % 8, which takes the contiguous run of tiles
  // [(b % 8) grid8 / 8, ...): the tiles of a row band (which share input lines) stay in one L2.
  const int bq = (int)(blockIdx.x & 7) * (grid8 >> 3) + (int)(blockIdx.x >> 3);
  if (bq >= a.ntx * a.nty * ncy * a.n) return;  // whole block, before any barrier
  const int tx = bq % a.ntx, r1 = bq / a.ntx, ty = r1 % a.nty, r2 = r1 / a.nty, cy = r2 % ncy, n = r2 / ncy;
  const int r0 = ty * PY_TR, c0 = tx * PY_TC;
  const int col0 = cy * NB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wa = wave & 1, wb = wave >> 1;
  const int row16 = lane & 15, grp = lane >> 4;
  const int nb = a.nb;

  int ncols[3], nbf[3];
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    int c = (b < nb ? a.out_cs[b] : 0) - col0;   // columns incl. zero pad channels
    c = c < 0 ? 0 : (c > NB ? NB : c);
    ncols[b] = c;
    nbf[b] = ceil_div(c, 16);
  }

  // The branches' biases for this block's columns: requested now, staged into LDS only at the
  // epilogue (a store here would hold the loading waves for a round trip before the K loop).
  static_assert(NB <= PY_THREADS, "one bias column per thread");
  __shared__ float s_bias[3][NB];
  float bias_r[3];
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const float* bp = b == 0 ? a.bias[0] : b == 1 ? a.bias[1] : a.bias[2];
    const int cb = b < nb ? a.cout[b] : 0;
    bias_r[b] = (tid < NB && bp && col0 + tid < cb) ? bp[col0 + tid] : 0.f;
  }

  // acc0: branch 0, this wave's pixel half x column half.  accp: the wave's pooled branch
  // (wb = 0: branch 1, wb = 1: branch 2), this wave's pixel half x all 2 HB column fragments,
  // so each pooled A fragment is formed by one wave instead of both column-half waves.
  floatx4 acc0[4][HB], accp[2 * HB];
#pragma unroll
  for (int j = 0; j < HB; ++j) {
    accp[j] = accp[HB + j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc0[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- register-staged prefetch of one K step (x slice + weight slices) ---------------------
  // Per-thread source pointers and validity are fixed across K steps; each step
  // advances them by 32 channels.
  const T* x = (const T*)a.x;
  const bool w4 = a.in_layout == KAD_NCHW && (a.w % 4) == 0;  // block-uniform: 8-byte aligned rows
  Raw8 xr[2];
  Raw8 br[BPT];
  const T* xp[2];
  int xvalid[2];      // elements of the 8-wide piece inside the image / channel range, before the K offset
  int xch[2];         // channel (NCHW) or channel-group start (NHWC) relative to k0
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int e = tid + t * PY_THREADS;
    if (a.in_layout == KAD_NCHW) {
      // lanes run along channels so the transposed LDS writes hit distinct banks
      const int ch = e & 31, rs = e >> 5, row = rs >> 2, seg = rs & 3;
      const int gy = r0 + row, gx = c0 + seg * 8;
      int valid = gy < a.h ? a.w - gx : 0;
      xvalid[t] = valid < 0 ? 0 : (valid > 8 ? 8 : valid);
      xch[t] = ch;
      xp[t] = x + (((int64_t)n * a.cin + ch) * a.h + (gy < a.h ? gy : 0)) * a.w + gx;
    } else {
      const int px = e >> 2, g = e & 3;
      const int gy = r0 + (px >> 5), gx = c0 + (px & 31);
      xvalid[t] = (gy < a.h && gx < a.w) ? 8 : 0;
      xch[t] = g * 8;
      xp[t] = x + (((int64_t)n * a.h + (gy < a.h ? gy : 0)) * a.w + (gx < a.w ? gx : 0)) * a.x_cs + g * 8;
    }
  }
  const int64_t xstep = a.in_layout == KAD_NCHW ? (int64_t)32 * a.h * a.w : 32;
  const T* bp_[BPT];
  bool bok[BPT];
#pragma unroll
  for (int t = 0; t < BPT; ++t) {
    const int e = tid + t * PY_THREADS;
    const int b = e / (NB * 4), r = e - b * (NB * 4), cl = r >> 2, g = r & 3;
    bok[t] = e < BTASKS && cl < nbf_sel(nbf, b) * 16;
    bp_[t] = bok[t] ? (const T*)sel3(a.wpack, b) + (int64_t)(col0 + cl) * cin_pad + g * 8 : nullptr;
  }
  auto load_step = [&](int k0) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      int valid;
      if (a.in_layout == KAD_NCHW) {
        valid = (k0 + xch[t] < a.cin) ? xvalid[t] : 0;
      } else {
        const int rem = a.cin - (k0 + xch[t]);
        valid = xvalid[t] ? (rem < 0 ? 0 : (rem > 8 ? 8 : rem)) : 0;
      }
      xr[t] = w4 ? load8_w4(xp[t] + (k0 / 32) * xstep, valid) : load8_raw(xp[t] + (k0 / 32) * xstep, valid);
    }
#pragma unroll
    for (int t = 0; t < BPT; ++t)
      if (bok[t]) br[t] = load8_full(bp_[t] + k0);
  };
  auto store_step = [&]() {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e = tid + t * PY_THREADS;
      if (a.in_layout == KAD_NCHW) {
        const int ch = e & 31, rs = e >> 5, row = rs >> 2, seg = rs & 3;
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[(row * PY_TC + seg * 8 + j) * LDA + ch] = raw_get<T>(xr[t], j);
      } else {
        const int px = e >> 2, g = e & 3;
        store8_raw(xs + px * LDA + g * 8, xr[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < BPT; ++t) {
      const int e = tid + t * PY_THREADS;
      const int b = e / (NB * 4), r = e - b * (NB * 4), cl = r >> 2, g = r & 3;
      if (e < BTASKS && cl < nbf_sel(nbf, b) * 16) {
        store8_raw(bs + (b * NB + cl) * LDA + g * 8, br[t]);
      }
    }
  };

  // one K step of MFMAs from the staged x slice (x_stage) and weights (bfrag(b, bf))
  auto mma_step = [&](const T* x_stage, auto bfrag) {
    // ---- A fragments: the slice (branch 0) and its 2x2 / 4x4 averages (branches 1, 2) ----------
    // wave (wa, wb) = pixel half x column half
    PyFrag<T> a0[4], ap;
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) a0[mm] = frag_ld(x_stage + ((wa * 4 + mm) * 16 + row16) * LDA + grp * 8);
    if (wb == 0) {  // branch 1: pooled (wa, row16)
      if (nb > 1) ap = pooled_frag<T, 2, LDA>(x_stage, (2 * wa) * PY_TC + 2 * row16, grp * 8);
    } else if (nb > 2) {  // branch 2: pooled pixel row16 of the 1 x 8 tile (rows >= 8 are padding), rows 2 wa, 2 wa + 1
      if (row16 < 8) {
        ap = pooled_frag<T, 4, LDA>(x_stage, (2 * wa) * PY_TC + 4 * row16, grp * 8);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) ap.v[j] = from_f32<T>(0.f);
      }
    }
#pragma unroll
    for (int bb = 0; bb < HB; ++bb) {
      const int bf = wb * HB + bb;
      if (bf < nbf[0]) {
        const PyFrag<T> bq = bfrag(0, bf);
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) acc0[mm][bb] = py_mma_f<T>(a0[mm], bq, acc0[mm][bb]);
      }
    }
    const int pbr = 1 + wb, nbp = wb == 0 ? nbf[1] : nbf[2];  // wave-uniform
#pragma unroll
    for (int bp = 0; bp < 2 * HB; ++bp)
      if (bp < nbp) accp[bp] = py_mma_f<T>(ap, bfrag(pbr, bp), accp[bp]);
  };
  auto bfrag_lds = [&](int b, int bf) { return frag_ld(bs + (b * NB + bf * 16 + row16) * LDA + grp * 8); };

  if constexpr (H16) {
    if (dma) {
      // ---- pipelined K loop (16-bit NCHW, W % 4 == 0) ---------------------------------------------
      // Weights: chunk (b, f) of step ks is 1 KB (fragment f) of the fragment-ordered copy behind the
      // row layout of branch b's packed buffer; wave w loads fragments w, w + 4, ... of every branch
      // straight into LDS slot b FB + f of the step's stage.  x: this thread's two 8-pixel pieces as four
      // 8-byte buffer loads (pieces past the image or channels past Cin read 0), two steps ahead.
      // Step ks opens with "own loads of step ks landed" + barrier; loads for steps past the last
      // read zeros, so every step issues the same loads and the wait count holds.
      constexpr int FB = 2 * HB, UPB = (FB + 3) / 4, TWMIN = 3 * (FB / 4);  // loads per branch / per wave (min)
      const int nk = cin_pad / 32;
      const int wv = __builtin_amdgcn_readfirstlane(wave);
      __amdgpu_buffer_rsrc_t rwb[3];
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        const int bb = b < nb ? b : 0;
        const int cpk = round_up(round_up(a.cout[bb], 8), 128);
        rwb[b] = make_rsrc((const T*)sel3(a.wpack, bb) + (int64_t)cpk * cin_pad, (uint32_t)((int64_t)cpk * cin_pad * 2));
      }
      uint32_t woff[3][UPB];
#pragma unroll
      for (int b = 0; b < 3; ++b)
#pragma unroll
        for (int u = 0; u < UPB; ++u) {
          const int f = wv + 4 * u;
          const bool ok = b < nb && f < nbf_sel(nbf, b);
          woff[b][u] = ok ? (uint32_t)(((((col0 >> 4) + f) * nk) * 64 + lane) * 16) : KAD_OOB;
        }
      const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)a.n * a.cin * a.h * a.w * 2));
      uint32_t xo[2];
      int xv[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int e = tid + t * PY_THREADS;
        const int ch = e & 31, rs = e >> 5, row = rs >> 2, seg = rs & 3;
        const int gy = r0 + row, gx = c0 + seg * 8;
        xo[t] = (uint32_t)(((((int64_t)n * a.cin + ch) * a.h + (gy < a.h ? gy : 0)) * a.w + gx) * 2);
        xv[t] = xvalid[t];  // 0, 4 or 8 (W % 4 == 0)
      }
      const uint32_t xstep_b = (uint32_t)(32 * a.h * a.w * 2);
      auto issue = [&](int ks, char* pw, uint4 (&xr2)[2]) {
#pragma unroll
        for (int b = 0; b < 3; ++b)
#pragma unroll
          for (int u = 0; u < UPB; ++u) {
            const int f = wv + 4 * u;
            if (f < FB) {  // wave-uniform: with FB % 4 != 0 the low waves take one fragment more
              const uint32_t o = (woff[b][u] == KAD_OOB || ks >= nk) ? KAD_OOB : woff[b][u] + (uint32_t)ks * 1024u;
              dma16(rwb[b], pw + (b * FB + f) * 1024, o, 0u);
            }
          }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const bool chok = ks < nk && ks * 32 + xch[t] < a.cin;
          const uint32_t o = xo[t] + (uint32_t)ks * xstep_b;
          typedef int intx2 __attribute__((ext_vector_type(2)));
          const intx2 lo = __builtin_bit_cast(intx2, __builtin_amdgcn_raw_buffer_load_b64(
                                                         rx, (chok && xv[t] >= 4) ? o : KAD_OOB, 0, 0));
          const intx2 hi = __builtin_bit_cast(intx2, __builtin_amdgcn_raw_buffer_load_b64(
                                                         rx, (chok && xv[t] == 8) ? o + 8 : KAD_OOB, 0, 0));
          xr2[t] = uint4{(unsigned)lo[0], (unsigned)lo[1], (unsigned)hi[0], (unsigned)hi[1]};
        }
      };
      auto store_x = [&](T* stage, const uint4 (&xr2)[2]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int e = tid + t * PY_THREADS;
          const int ch = e & 31, rs = e >> 5, row = rs >> 2, seg = rs & 3;
          Raw8 r;
          r.lo = xr2[t];
          r.hi = uint4{0u, 0u, 0u, 0u};
#pragma unroll
          for (int j = 0; j < 8; ++j) stage[(row * PY_TC + seg * 8 + j) * LDA + ch] = raw_get<T>(r, j);
        }
      };
      T* xs0 = xsd;
      T* xs1 = xsd + PY_TILE * LDA;
      uint4 xa[2], xb[2];
      issue(0, pw0, xa);
      issue(1, pw1, xb);
      store_x(xs0, xa);
      // step ks: stage ks % 3 for the weights, ks % 2 for x; x of step ks + 1 sits in registers
      auto step = [&](int ks, const char* pwc, char* pwr, const T* xcur, T* xnext, uint4 (&xnow)[2],
                      uint4 (&xload)[2]) {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(TWMIN + 4) : "memory");
        issue(ks + 2, pwr, xload);
        mma_step(xcur, [&](int b, int bf) { return *(const PyFrag<T>*)(pwc + ((b * FB + bf) * 64 + lane) * 16); });
        store_x(xnext, xnow);  // x of step ks + 1 into the stage read in step ks - 1
      };
      // rotation period 6 = lcm(3 weight stages, 2 x stages); x registers alternate xb (step ks + 1) / xa
      const int nk6 = nk / 6 * 6;
      for (int ks = 0; ks < nk6; ks += 6) {
        step(ks, pw0, pw2, xs0, xs1, xb, xa);
        step(ks + 1, pw1, pw0, xs1, xs0, xa, xb);
        step(ks + 2, pw2, pw1, xs0, xs1, xb, xa);
        step(ks + 3, pw0, pw2, xs1, xs0, xa, xb);
        step(ks + 4, pw1, pw0, xs0, xs1, xb, xa);
        step(ks + 5, pw2, pw1, xs1, xs0, xa, xb);
      }
      const int r6 = nk - nk6;
      if (r6 > 0) step(nk6, pw0, pw2, xs0, xs1, xb, xa);
      if (r6 > 1) step(nk6 + 1, pw1, pw0, xs1, xs0, xa, xb);
      if (r6 > 2) step(nk6 + 2, pw2, pw1, xs0, xs1, xb, xa);
      if (r6 > 3) step(nk6 + 3, pw0, pw2, xs1, xs0, xa, xb);
      if (r6 > 4) step(nk6 + 4, pw1, pw0, xs0, xs1, xb, xa);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the loop
    }
  }
  if (!H16 || !dma) {
  load_step(0);
  for (int k0 = 0; k0 < cin_pad; k0 += 32) {
    __syncthreads();  // the previous step's MFMAs are done with xs / bs
    store_step();
    if (k0 + 32 < cin_pad) load_step(k0 + 32);  // in flight while this step computes
    __syncthreads();
    mma_step(xs, bfrag_lds);
  }
  }

  // ---- epilogue -------------------------------------------------------------------------------------
  // acc layout: lane (row16, grp) holds column bf * 16 + row16 and tile pixels
  //   branch 0: (wa * 4 + mm) * 16 + grp * 4 + i  (tile row 2 wa + mm / 2, column (mm & 1) * 16 + grp * 4 + i)
  //   branch 1 (accp, wb = 0): wa * 16 + grp * 4 + i  (pooled row wa, column grp * 4 + i)
  //   branch 2 (accp, wb = 1): grp * 4 + i (< 8)      (pooled row 0, column grp * 4 + i; wa = half of the window)
  // 1. Each wave rounds its outputs (bias added) to T and stages them; the row sums of
  //    branches 0 and 1 come from the same rounded values in registers (+ shuffles across
  //    the 4 lane groups), masked to the tile's valid columns.
  // 2. After one barrier all threads store y as 16-byte NHWC pieces and form the column
  //    sums (and branch 2's row sums, whose window halves meet only here) from LDS.
  // The partial sums are fp32 sums of the rounded outputs, as pooling y in T does.  A tile
  // with no row of a pooled branch still writes zero column partials (the consumer reads
  // every slice).  The barriers wait for LDS traffic only.  No load into LDS is in flight
  // past the K loop.
#define PY_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")
  if (tid < NB) {
#pragma unroll
    for (int b = 0; b < 3; ++b) s_bias[b][tid] = bias_r[b];
  }
  PY_LDS_BARRIER();  // every wave is done with the K loop's LDS; the biases are staged
  int vcs[3], vrs[3];
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const int tr = PY_TR >> b, tc = PY_TC >> b;
    const int hbch = b < nb ? a.out_h[b] : 0, wbch = b < nb ? a.out_w[b] : 0;
    vcs[b] = (wbch - tx * tc) < tc ? (wbch - tx * tc) : tc;  // valid columns in this tile (may be <= 0)
    vrs[b] = (hbch - ty * tr) < tr ? (hbch - ty * tr) : tr;  // valid rows
  }
#pragma unroll
  for (int bb = 0; bb < HB; ++bb) {
    const int bf = wb * HB + bb;
    const int col = bf * 16 + row16, co = col0 + col;
    if (bf < nbf[0]) {
      const float bv = s_bias[0][col];
      T* yh = wa == 0 ? y0a : y0b;
      float sr[2] = {0.f, 0.f};
#pragma unroll
      for (int mm = 0; mm < 4; ++mm)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const T v = from_f32<T>(acc0[mm][bb][i] + bv);
          yh[(mm * 16 + grp * 4 + i) * OBT + col] = v;
          sr[mm >> 1] += ((mm & 1) * 16 + grp * 4 + i < vcs[0]) ? to_f32(v) : 0.f;
        }
      if (a.rowpart[0]) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {  // tile rows 2 wa + q
          float v = sr[q];
          v = sum_xor32(sum_xor16(v));
          const int r = 2 * wa + q;
          if (grp == 0 && co < a.cout[0] && r < vrs[0])
            a.rowpart[0][(((int64_t)n * a.ntx + tx) * a.out_h[0] + ty * PY_TR + r) * a.cout[0] + co] = v;
        }
      }
    }
  }
  // pooled branches: wave (wa, wb) holds branch 1 + wb over the column fragments bp < 2 HB
#pragma unroll
  for (int bp = 0; bp < 2 * HB; ++bp) {
    const int col = bp * 16 + row16, co = col0 + col;
    if (wb == 0 && bp < nbf[1]) {
      const float bv = s_bias[1][col];
      float sr = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const T v = from_f32<T>(accp[bp][i] + bv);
        y1s[(wa * 16 + grp * 4 + i) * OBT + col] = v;
        sr += (grp * 4 + i < vcs[1]) ? to_f32(v) : 0.f;
      }
      if (a.rowpart[1]) {
        sr = sum_xor32(sum_xor16(sr));
        if (grp == 0 && co < a.cout[1] && wa < vrs[1])
          a.rowpart[1][(((int64_t)n * a.ntx + tx) * a.out_h[1] + ty * (PY_TR >> 1) + wa) * a.cout[1] + co] = sr;
      }
    }
    if (wb == 1 && bp < nbf[2]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (grp * 4 + i < 8) y2s[(wa * 8 + grp * 4 + i) * NB + col] = accp[bp][i];
    }
  }
  PY_LDS_BARRIER();
  // staged y of branch b, pixel p, columns c8 .. c8 + 7 (branch 2: the halves added, bias, rounding)
#define PY_STAGED(B, P, C8, OUT)                                                                     \
  {                                                                                                  \
    if ((B) == 0) {                                                                                  \
      const T* sp_ = ((P) < 64 ? y0a + (P) * OBT : y0b + ((P) - 64) * OBT) + (C8);                   \
      OUT.lo = *(const uint4*)sp_;                                                                   \
      if constexpr (sizeof(T) == 4) OUT.hi = *(const uint4*)(sp_ + 4);                               \
    } else if ((B) == 1) {                                                                           \
      const T* sp_ = y1s + (P) * OBT + (C8);                                                         \
      OUT.lo = *(const uint4*)sp_;                                                                   \
      if constexpr (sizeof(T) == 4) OUT.hi = *(const uint4*)(sp_ + 4);                               \
    } else {                                                                                         \
      const floatx4* h0_ = (const floatx4*)(y2s + (P) * NB + (C8));                                  \
      const floatx4* h1_ = (const floatx4*)(y2s + (8 + (P)) * NB + (C8));                            \
      const floatx4 a0_ = h0_[0], a1_ = h0_[1], b0_ = h1_[0], b1_ = h1_[1];                          \
      T t_[8];                                                                                       \
      _Pragma("unroll") for (int j_ = 0; j_ < 4; ++j_) {                                             \
        t_[j_] = from_f32<T>(a0_[j_] + b0_[j_] + s_bias[2][(C8) + j_]);                              \
        t_[4 + j_] = from_f32<T>(a1_[j_] + b1_[j_] + s_bias[2][(C8) + 4 + j_]);                      \
      }                                                                                              \
      OUT = raw_pack<T>(t_);                                                                         \
    }                                                                                                \
  }
  constexpr int G8 = NB / 8;
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    if (ncols[b] == 0) continue;  // uniform across the block
    const int tr = PY_TR >> b, tc = PY_TC >> b;
    const int hbch = a.out_h[b], wbch = a.out_w[b], cout = a.cout[b], g8 = ncols[b] >> 3;
    const int vc = vcs[b], vr = vrs[b];
    // y_b: NHWC, 16-byte pieces of 8 channels (the pad channels come out zero)
    T* y = (T*)a.out[b];
    for (int e = tid; e < tr * tc * G8; e += PY_THREADS) {
      const int pl = e / G8, g = e - pl * G8;
      const int py_ = pl / tc;  // tc is a power of two
      const int gy = ty * tr + py_, gx = tx * tc + (pl - py_ * tc);
      if (g >= g8 || gy >= hbch || gx >= wbch) continue;
      Raw8 v;
      PY_STAGED(b, pl, g * 8, v);
      store8_raw(y + (((int64_t)n * hbch + gy) * wbch + gx) * a.out_cs[b] + col0 + g * 8, v);
    }
    if (!a.colpart[b]) continue;
    // column sums over the tile's valid rows (0 if it has none), columns c < vc
    float* colp = a.colpart[b];
    for (int e = tid; e < tc * G8; e += PY_THREADS) {
      const int c = e / G8, g = e - c * G8;
      if (c >= vc || g * 8 >= cout - col0) continue;
      float sc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int r = 0; r < vr; ++r) {
        Raw8 v;
        PY_STAGED(b, r * tc + c, g * 8, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] += to_f32(raw_get<T>(v, j));
      }
      float* d = colp + (((int64_t)n * a.nty + ty) * wbch + tx * tc + c) * cout + col0 + g * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (col0 + g * 8 + j < cout) d[j] = sc[j];
    }
    if (b == 2 && a.rowpart[2]) {  // one pooled row per tile: its sum over the valid columns
      static_assert(8 * G8 <= PY_THREADS && PY_TC >> 2 == 8, "thread (group g, column c) of the pooled row");
      const int g = tid >> 3, c = tid & 7;  // the 8 lanes of a group stay together (all in or out)
      if (g < G8) {
        float sr[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (vr > 0 && c < vc) {
          Raw8 v;
          PY_STAGED(2, c, g * 8, v);
#pragma unroll
          for (int j = 0; j < 8; ++j) sr[j] = to_f32(raw_get<T>(v, j));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          sr[j] += __shfl_xor(sr[j], 1);
          sr[j] += __shfl_xor(sr[j], 2);
          sr[j] += __shfl_xor(sr[j], 4);
        }
        if (c == 0 && vr > 0 && g * 8 < cout - col0) {
          float* d = a.rowpart[2] + (((int64_t)n * a.ntx + tx) * hbch + ty) * cout + col0 + g * 8;
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (col0 + g * 8 + j < cout) d[j] = sr[j];
        }
      }
    }
  }
#undef PY_STAGED
}
#undef PY_LDS_BARRIER

// Dynamic LDS (register-staged path): the K loop's x and weight stages or the
// epilogue staging (y of branches 0 and 1 as T rows, branch 2's fp32 window halves).
template <typename T, int HB>
static size_t pyramid_lds(int dma) {
  if (dma) return 0;  // pipelined path: static weight ring and x stages (the epilogue reuses the ring)
  const size_t lda = PyLds<T>::lda;
  const size_t stage = (size_t)(PY_TILE + 3 * 32 * HB) * lda * sizeof(T);
  const size_t obt = (size_t)(32 * HB + 16 / sizeof(T)) * sizeof(T);
  const size_t epi = (size_t)(128 + 32) * obt + (size_t)2 * 8 * 32 * HB * sizeof(float);
  return stage > epi ? stage : epi;
}

template <typename T, int HB>
static void launch_pyramid(const kad_pyramid_args& a, int cin_pad, int maxcols, hipStream_t st) {
  const int ncy = ceil_div(maxcols, 32 * HB);
  const int grid8 = round_up(a.ntx * a.nty * ncy * a.n, 8);
  dim3 grid(grid8);
  const int dma = sizeof(T) == 2 && a.in_layout == KAD_NCHW && a.w % 4 == 0 &&
                  (int64_t)a.n * a.cin * a.h * a.w * 2 < (1ll << 31) && (uint32_t)(32 * a.h * a.w * 2) > 0;
  const size_t lds = pyramid_lds<T, HB>(dma);
  allow_lds(pyramid_kernel<T, HB>, lds);
  hipLaunchKernelGGL((pyramid_kernel<T, HB>), grid, dim3(PY_THREADS), lds, st, a, cin_pad, dma, ncy, grid8);
}

template <typename T>
static int dispatch_pyramid(const kad_pyramid_args& a, int cin_pad, int maxcols, hipStream_t st) {
  const int hb = ceil_div(ceil_div(maxcols, 16), 2);
  switch (hb) {
    case 1: launch_pyramid<T, 1>(a, cin_pad, maxcols, st); break;
    case 2: launch_pyramid<T, 2>(a, cin_pad, maxcols, st); break;
    case 3: launch_pyramid<T, 3>(a, cin_pad, maxcols, st); break;
    default: launch_pyramid<T, 4>(a, cin_pad, maxcols, st); break;
  }
  return check_launch("kad_pyramid_proj");
}

}  // namespace kad

using namespace kad;

extern "C" int kad_pyramid_tiles(int h, int w, int* ntx, int* nty) {
  KAD_CHECK_ARG(ntx && nty && h > 0 && w > 0, "kad_pyramid_tiles: bad arguments");
  *ntx = ceil_div(w, PY_TC);
  *nty = ceil_div(h, PY_TR);
  return KAD_OK;
}

extern "C" int kad_pyramid_proj(const kad_pyramid_args* a, void* stream) {
  KAD_CHECK_ARG(a && a->x, "kad_pyramid_proj: null pointer");
  KAD_CHECK_ARG(a->nb >= 1 && a->nb <= 3, "kad_pyramid_proj: nb=%d must be 1..3", a->nb);
  KAD_CHECK_ARG(a->n > 0 && a->cin > 0 && a->h >= (1 << (a->nb - 1)) && a->w >= (1 << (a->nb - 1)),
                "kad_pyramid_proj: bad shape");
  KAD_CHECK_ARG(a->in_layout == KAD_NCHW || (a->in_layout == KAD_NHWC && a->x_cs >= a->cin),
                "kad_pyramid_proj: bad input layout");
  KAD_CHECK_ARG((int64_t)a->n * ceil_div(a->w, PY_TC) * ceil_div(a->h, PY_TR) * 8 < (1ll << 31),
                "kad_pyramid_proj: too many tiles");
  KAD_CHECK_ARG(a->ntx == ceil_div(a->w, PY_TC) && a->nty == ceil_div(a->h, PY_TR),
                "kad_pyramid_proj: ntx/nty must come from kad_pyramid_tiles");
  int maxcols = 0;
  for (int b = 0; b < a->nb; ++b) {
    KAD_CHECK_ARG(a->wpack[b] && a->out[b], "kad_pyramid_proj: branch %d has a null pointer", b);
    KAD_CHECK_ARG(a->cout[b] > 0 && a->out_cs[b] % 8 == 0 && a->out_cs[b] >= a->cout[b] &&
                      a->out_cs[b] <= round_up(round_up(a->cout[b], 8), 128),
                  "kad_pyramid_proj: branch %d: out_cs %d must be a multiple of 8 in [cout, roundup128]", b,
                  a->out_cs[b]);
    KAD_CHECK_ARG(a->out_h[b] == a->h >> b && a->out_w[b] == a->w >> b, "kad_pyramid_proj: branch %d size", b);
    KAD_CHECK_ARG((a->rowpart[b] == nullptr) == (a->colpart[b] == nullptr),
                  "kad_pyramid_proj: rowpart and colpart go together");
    KAD_CHECK_ARG(((uintptr_t)a->wpack[b] | (uintptr_t)a->out[b]) % 16 == 0,
                  "kad_pyramid_proj: wpack/out must be 16-byte aligned");
    maxcols = a->out_cs[b] > maxcols ? a->out_cs[b] : maxcols;
  }
  const int cin_pad = round_up(a->cin, 32);
  hipStream_t st = (hipStream_t)stream;
  const int band = band_pyramid(*a, st);  // 16-bit NCHW KADConv shapes: one block per 4-row band
  if (band != 1) return band;
  switch (a->dtype) {
    case KAD_F32: return dispatch_pyramid<float>(*a, cin_pad, maxcols, st);
    case KAD_F16: return dispatch_pyramid<half_t>(*a, cin_pad, maxcols, st);
    case KAD_BF16: return dispatch_pyramid<bf16_t>(*a, cin_pad, maxcols, st);
    default: return fail(KAD_EINVAL, "kad_pyramid_proj: unknown dtype %d", a->dtype);
  }
}
