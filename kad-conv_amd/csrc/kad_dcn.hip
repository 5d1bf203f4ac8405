// Modulated deformable 3x3 convolution (DCNv2) fused into an MFMA GEMM, and the
// plain 3x3 convolution that produces its offsets.
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
//
// One kernel template, three modes:
//  EXT    offsets (and mask) come from memory             -> kad_dcn_fwd
//  FUSED  offsets = conv_offset(x) computed in the block   -> kad_dsc_fwd
//  PLAIN  ordinary 3x3 convolution (no sampling)          -> kad_conv3x3_fwd
//
// Block = 512 threads (8 waves, two per SIMD, so one wave's LDS / memory waits
// overlap the other's MFMA and blend work) x one output tile of up to 128
// pixels (TH x TW, chosen per image size to waste few lanes) x 16 * NBF output
// channels; wave w owns tile pixels [16 w, 16 w + 16) and all the block's
// channels.
//  0. Loads that do not depend on anything are issued first: epilogue
//     parameters, the mask (and offsets in EXT mode), the first input chunk.
//  1. PLAIN / FUSED: the tile's 3x3 footprint (tile + 1-pixel ring, zero
//     padded) is staged per 32-channel chunk in LDS and convolved on MFMA
//     (integer taps need no sample records).  FUSED keeps the 18 offset
//     channels in LDS; PLAIN goes straight to the epilogue.
//  2. Every (tap, pixel) sample position is computed once (registers), and the
//     block reduces the bounding box of all live corners.  The input region =
//     that box, capped to the LDS budget around the tile (typical offsets fit).
//     Each sample's four region byte offsets and weights (bilinear x mask, 0
//     for out-of-image corners; fp16 except on the fp32 path) go to LDS once.
//     Samples outside a capped region are flagged and added by a rare pass
//     that reads global memory.
//  3. Per 32-channel chunk (next chunk prefetched into registers): the region
//     slice [pixels][32 ch] and, on 16-bit paths, the chunk's weights
//     [9 taps][cols][32] are staged in LDS; for each tap each lane builds its
//     MFMA A fragment (8 channels of one (pixel, tap)) from four 16-byte LDS
//     corner reads blended with packed FMAs, and the wave issues NBF
//     v_mfma_f32_16x16x32 against 16-byte B fragments.  Weight rows are
//     64 bytes, so their four 16-byte pieces are stored XOR-swizzled by
//     column (piece g of column c at slot g ^ ((c >> 1) & 3)): the 16 lanes
//     of a B read then hit distinct banks.
//  4. Epilogue: bias, BN scale/shift, ReLU, branch scale; the tile is staged
//     in LDS and written with 16-byte row-contiguous stores; GAP partials.
// Blocks are mapped so that each XCD (and its L2) gets a contiguous band of
// tiles: neighbouring tiles share their halos through that L2.
//
// Any consistent assignment of k to (lane group, slot) gives the same dot
// product, so A and B only have to agree with each other; the accumulator
// layout (lane -> column lane & 15, rows 4 * (lane >> 4) + i) is the MFMA
// output layout.
#include <mutex>
#include <type_traits>

#include "kad_common.h"

namespace kad {

#ifndef KAD_DCN_WAVES
#define KAD_DCN_WAVES 8
#endif
constexpr int DCN_WAVES = KAD_DCN_WAVES;           // waves per block (8: two per SIMD)
constexpr int DCN_THREADS = 64 * DCN_WAVES;
constexpr int DCN_WM = 8 / DCN_WAVES;              // 16-pixel A fragments per wave
constexpr int DCN_TILE = DCN_WAVES * DCN_WM * 16;  // 128 pixels per block
constexpr int DCN_NPAIR = 9 * DCN_TILE;            // (tap, pixel) samples per block
constexpr int DCN_KSTEP = DCN_THREADS / DCN_TILE;  // sample (tap, pixel) of thread t: pixel t % 128, taps t / 128 + KSTEP u
constexpr int DCN_PPT = (9 + DCN_KSTEP - 1) / DCN_KSTEP;  // samples per thread
constexpr int DCN_NOFF = 18;                       // offset channels (2 x 9 taps)
constexpr int DCN_LDS = 160 * 1024;                // gfx950 LDS per CU
constexpr int DCN_SLOT = DCN_THREADS / 4;          // region pixels staged per round (4 threads per pixel)
constexpr int DCN_FCAP = 704;                      // footprint pixels (enough for stride <= 2)
static_assert(DCN_TILE == 128 && DCN_SLOT % 64 == 0, "tile / staging geometry");
constexpr int DCN_SE_LDS = 48 * 1024;              // fused SE scratch (floats in the region buffer) limit

enum { MODE_EXT = 0, MODE_FUSED = 1, MODE_PLAIN = 2 };

struct DcnGeom {
  int ho, wo, th, tw, tiles_x, tiles, grid_x, nchunk, cout_pad;
  int fh, fw;        // 3x3 footprint of a tile: (th - 1) * stride + 3 rows, likewise columns
  float inv_tw, inv_fw;
};

// Tile shape for an Ho x Wo output: TH x TW <= 128 pixels minimising the
// padded pixel count; ties prefer squarer tiles (smaller halo).
static void pick_tile(int ho, int wo, int* th_out, int* tw_out) {
  long best = -1;
  int bth = 8, btw = 16;
  for (int tw = 4; tw <= 64; ++tw) {
    const int th = DCN_TILE / tw;
    if (th < 1) break;
    const long cost = (long)ceil_div(ho, th) * ceil_div(wo, tw) * DCN_TILE * 64 + (th > tw ? th - tw : tw - th);
    if (best < 0 || cost < best) {
      best = cost;
      bth = th;
      btw = tw;
    }
  }
  *th_out = bth;
  *tw_out = btw;
}

// ---- sample info ----------------------------------------------------------------------------
// Fast-path record per (tap, pixel): byte offsets of the four corners inside the
// staged region and the corner weights (16-bit paths: 16-bit offsets, fp16
// weights; fp32 path: 32-bit offsets, fp32 weights).  Samples that are dead
// (all weights 0) or outside a capped region get zero weights here; the latter
// are accumulated by a separate pass from global memory (s_slow).
struct __align__(16) Info16 { unsigned o01, o23; unsigned w01, w23; };  // weights as 2 x half2
struct __align__(16) Info32 { unsigned o[4]; float w[4]; };

__device__ __forceinline__ unsigned pack_h2(float a, float b) {
  const half2_t h{(half_t)a, (half_t)b};
  return __builtin_bit_cast(unsigned, h);
}

template <typename T> struct InfoOf { typedef Info16 type; };
template <> struct InfoOf<float> { typedef Info32 type; };

template <typename T>
__device__ __forceinline__ typename InfoOf<T>::type make_info(const unsigned* o, const float* w) {
  typename InfoOf<T>::type r;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.o[i] = o[i];
      r.w[i] = w[i];
    }
  } else {
    r.o01 = o[0] | (o[1] << 16);
    r.o23 = o[2] | (o[3] << 16);
    r.w01 = pack_h2(w[0], w[1]);
    r.w23 = pack_h2(w[2], w[3]);
  }
  return r;
}

// byte offset of corner j of a record
__device__ __forceinline__ unsigned corner(const Info16& in, int j) {
  const unsigned v = j < 2 ? in.o01 : in.o23;
  return (j & 1) ? v >> 16 : v & 0xffffu;
}
__device__ __forceinline__ unsigned corner(const Info32& in, int j) { return in.o[j]; }

// ---- A fragment from four corners ------------------------------------------------------------
template <typename T> struct DcnFrag;

template <> struct DcnFrag<half_t> {
  typedef half8_t frag;
  static __device__ __forceinline__ frag blend(const half8_t& v0, const half8_t& v1, const half8_t& v2,
                                               const half8_t& v3, const Info16& in) {
    const half2_t w01 = __builtin_bit_cast(half2_t, in.w01), w23 = __builtin_bit_cast(half2_t, in.w23);
    frag r = v0 * w01[0];
    r += v1 * w01[1];
    r += v2 * w23[0];
    r += v3 * w23[1];
    return r;
  }
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct DcnFrag<bf16_t> {
  typedef bf16x8_t frag;
  static __device__ __forceinline__ frag blend(const bf16x8_t& v0, const bf16x8_t& v1, const bf16x8_t& v2,
                                               const bf16x8_t& v3, const Info16& in) {
    const half2_t w01 = __builtin_bit_cast(half2_t, in.w01), w23 = __builtin_bit_cast(half2_t, in.w23);
    const float a = (float)w01[0], b = (float)w01[1], c = (float)w23[0], d = (float)w23[1];
    frag r;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      r[j] = (bf16_t)(a * (float)v0[j] + b * (float)v1[j] + c * (float)v2[j] + d * (float)v3[j]);
    return r;
  }
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

struct f32x8 { floatx4 lo, hi; };

template <> struct DcnFrag<float> {
  typedef f32x8 frag;
  static __device__ __forceinline__ frag blend(const f32x8& v0, const f32x8& v1, const f32x8& v2,
                                               const f32x8& v3, const Info32& in) {
    frag r;
    r.lo = v0.lo * in.w[0] + v1.lo * in.w[1] + v2.lo * in.w[2] + v3.lo * in.w[3];
    r.hi = v0.hi * in.w[0] + v1.hi * in.w[1] + v2.hi * in.w[2] + v3.hi * in.w[3];
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

template <typename T>
__device__ __forceinline__ typename DcnFrag<T>::frag ld8(const T* p) {
  typedef typename DcnFrag<T>::frag F;
  if constexpr (sizeof(T) == 4) {
    F r;
    r.lo = *(const floatx4*)p;
    r.hi = *(const floatx4*)(p + 4);
    return r;
  } else {
    return *(const F*)p;
  }
}

template <typename T>
__device__ __forceinline__ void st8(T* p, const typename DcnFrag<T>::frag& v) {
  if constexpr (sizeof(T) == 4) {
    *(floatx4*)p = v.lo;
    *(floatx4*)(p + 4) = v.hi;
  } else {
    *(typename DcnFrag<T>::frag*)p = v;
  }
}

template <typename T>
__device__ __forceinline__ typename DcnFrag<T>::frag zero8() {
  typedef typename DcnFrag<T>::frag F;
  if constexpr (sizeof(T) == 4) {
    F r;
    r.lo = floatx4{0.f, 0.f, 0.f, 0.f};
    r.hi = r.lo;
    return r;
  } else {
    return F{};
  }
}

// Bilinear geometry of one sample at (py, px) (torchvision's rule): clamped
// top-left corner, corner steps (0 or 1 per axis) and the four weights times m;
// all weights 0 for a dead sample.
__device__ __forceinline__ void sample_geom(float py, float px, float m, int h, int w, int& cy0, int& cx0, int& sy,
                                            int& sx, float* wt) {
  cy0 = cx0 = sy = sx = 0;
  wt[0] = wt[1] = wt[2] = wt[3] = 0.f;
  if (py > -1.f && py < (float)h && px > -1.f && px < (float)w) {
    const float fy = floorf(py), fx = floorf(px);
    const int y0 = (int)fy, x0 = (int)fx, y1 = y0 + 1, x1 = x0 + 1;
    const float ly = py - fy, lx = px - fx, hy = 1.f - ly, hx = 1.f - lx;
    const bool vy0 = y0 >= 0, vy1 = y1 <= h - 1, vx0 = x0 >= 0, vx1 = x1 <= w - 1;
    cy0 = vy0 ? y0 : 0;
    const int cy1 = vy1 ? y1 : h - 1;
    cx0 = vx0 ? x0 : 0;
    const int cx1 = vx1 ? x1 : w - 1;
    sy = cy1 - cy0;
    sx = cx1 - cx0;
    wt[0] = (vy0 && vx0) ? hy * hx * m : 0.f;
    wt[1] = (vy0 && vx1) ? hy * lx * m : 0.f;
    wt[2] = (vy1 && vx0) ? ly * hx * m : 0.f;
    wt[3] = (vy1 && vx1) ? ly * lx * m : 0.f;
  }
}

// ---- LDS budget per instantiation --------------------------------------------------------------
template <typename T, typename OutT, int NBF, int MODE> struct DcnLds {
  static constexpr bool BLDS = sizeof(T) == 2;     // 16-bit paths stage the weights in LDS
  static constexpr int NB = NBF * 16;
  static constexpr int PXS = sizeof(T) == 2 ? 40 : 36;  // elements per region pixel (32 + pad: conflict-free rows)
  static constexpr int PXB = PXS * (int)sizeof(T);
  // FUSED 16-bit stages the 18 offset filters of up to 3 chunks here first (9 x 18 x 104 elements)
  static constexpr int BCOLS = (MODE == MODE_FUSED && BLDS) ? (NB > 64 ? NB : 64) : (NB > 32 ? NB : 32);
  static constexpr int BSM = BLDS ? 9 * BCOLS * 32 : 8;
  static constexpr int NINFO = MODE == MODE_PLAIN ? 1 : DCN_NPAIR;
  static constexpr int NOFF = MODE == MODE_FUSED ? DCN_TILE * DCN_NOFF : 1;
  static constexpr int SROW = NB + 16 / (int)sizeof(OutT);  // epilogue staging row (elements)
  static constexpr int FIXED = BSM * (int)sizeof(T) + NINFO * ((int)sizeof(typename InfoOf<T>::type) + 1) +
                               NOFF * 4 + 4 * NB * 4 + 256;
  static constexpr int STAGE_BYTES = DCN_TILE * SROW * (int)sizeof(OutT);  // epilogue tile, then GAP rows [waves][NB]
  static constexpr int STAGE_PX = (STAGE_BYTES + DCN_WAVES * NB * 4 + PXB - 1) / PXB;
  // region staging uses RCAP / DCN_SLOT pieces per thread; the epilogue tile reuses the region
  static constexpr int RCAP_MIN = STAGE_PX > 768 ? STAGE_PX : 768;
  static constexpr int RCAP_WANT = (RCAP_MIN + 63) / 64 * 64;
  static constexpr int RCAP_FIT = (DCN_LDS - FIXED) / PXB < RCAP_WANT ? (DCN_LDS - FIXED) / PXB : RCAP_WANT;
  static constexpr int RCAP = RCAP_FIT / 64 * 64;    // a multiple of 64 pixels
  static_assert(RCAP >= DCN_FCAP, "footprint must fit the region buffer");
  static_assert(MODE == MODE_PLAIN || sizeof(T) == 4 || RCAP * PXB <= 65536, "16-bit corner offsets");
  static_assert(RCAP * PXB >= STAGE_BYTES + DCN_WAVES * NB * 4, "epilogue tile must fit the region buffer");
  static_assert(MODE == MODE_PLAIN || RCAP * PXB >= DCN_SE_LDS, "fused SE scratch must fit the region buffer");
};

// ---- buffer loads ------------------------------------------------------------------------------
// A raw buffer load returns 0 for a byte offset at or past the descriptor's
// size, so pieces outside the image (padding ring, channels past Cin, unused
// staging slots) are staged as zeros with no branch; per-thread byte offsets are
// computed once per block and only shifted per channel chunk.
constexpr uint32_t DCN_OOB = KAD_OOB;

template <typename T>
__device__ __forceinline__ typename DcnFrag<T>::frag buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  typedef typename DcnFrag<T>::frag F;
  if constexpr (sizeof(T) == 4) {
    F f;
    f.lo = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
    f.hi = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, 0, 0));
    return f;
  } else {
    return __builtin_bit_cast(F, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
  }
}

// Chunk staging: up to CAP region pixels x 32 channels, 8-channel pieces,
// prefetched in registers; piece u of thread t is pixel t / 4 + DCN_SLOT u,
// channel group t % 4.  The LDS buffer holds CAP pixels (a multiple of 64) and
// every slot below CAP is stored (unused slots receive zeros); only the last
// round can reach past CAP, when CAP is not a multiple of DCN_SLOT.
template <typename T, int CAP> struct RegionTile {
  static_assert(CAP % 64 == 0, "CAP must be a multiple of 64");
  static constexpr int RPT = (CAP + DCN_SLOT - 1) / DCN_SLOT;
  static constexpr bool RAGGED = CAP % DCN_SLOT != 0;
  typename DcnFrag<T>::frag v[RPT];
  uint32_t voff[RPT];  // byte offset of the piece's chunk-0 channels in the image, or DCN_OOB
  // npix = rows x cols pixels starting at (y0, x0); parts outside the image read 0
  __device__ __forceinline__ void setup(int y0, int x0, int cols, int npix, float inv_cols, int h, int w, int x_cs,
                                        int tid) {
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      const int q = (tid >> 2) + u * DCN_SLOT;
      uint32_t o = DCN_OOB;
      if (q < npix) {
        const int qy = (int)(((float)q + 0.5f) * inv_cols);
        const int gy = y0 + qy, gx = x0 + q - qy * cols;
        if (gy >= 0 && gy < h && gx >= 0 && gx < w)
          o = (uint32_t)(((gy * w + gx) * x_cs + (tid & 3) * 8) * (int)sizeof(T));
      }
      voff[u] = o;
    }
  }
  // chunk c; chs_ok = this thread's channel group holds real channels in chunk c
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int c, bool chs_ok) {
    const uint32_t cofs = (uint32_t)(c * 32 * (int)sizeof(T));
#pragma unroll
    for (int u = 0; u < RPT; ++u) v[u] = buf_ld8<T>(r, chs_ok ? voff[u] + cofs : DCN_OOB);
  }
  __device__ __forceinline__ void store(T* region, int pxs, int tid) {
    T* base = region + (tid >> 2) * pxs + (tid & 3) * 8;
#pragma unroll
    for (int u = 0; u < RPT; ++u)
      if (!RAGGED || u + 1 < RPT || (tid >> 2) + u * DCN_SLOT < CAP) st8<T>(base + u * DCN_SLOT * pxs, v[u]);
  }
};

// Chunk weights [9][NBC][32] (16-bit paths), swizzled 16-byte pieces, from the
// packed layout [Cout_pad][nchunk][9][32].
template <typename T, int NBC> struct WeightTile {
  static constexpr int PIECES = 9 * NBC * 4;
  static constexpr int BPT = (PIECES + DCN_THREADS - 1) / DCN_THREADS;
  typename DcnFrag<T>::frag v[BPT];
  uint32_t voff[BPT];
  __device__ __forceinline__ void setup(int co0, int cpad, int nchunk, int tid) {
#pragma unroll
    for (int u = 0; u < BPT; ++u) {
      const int e = tid + u * DCN_THREADS;
      uint32_t o = DCN_OOB;
      if (e < PIECES) {
        const int k = e / (NBC * 4), r = e - k * (NBC * 4), co = co0 + (r >> 2);
        if (co < cpad) o = (uint32_t)((((co * nchunk) * 9 + k) * 32 + (r & 3) * 8) * (int)sizeof(T));
      }
      voff[u] = o;
    }
  }
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int c) {
    const uint32_t cofs = (uint32_t)(c * 9 * 32 * (int)sizeof(T));
#pragma unroll
    for (int u = 0; u < BPT; ++u) v[u] = buf_ld8<T>(r, voff[u] + cofs);
  }
  __device__ __forceinline__ void store(T* bsm, int tid) {
#pragma unroll
    for (int u = 0; u < BPT; ++u) {
      const int e = tid + u * DCN_THREADS;
      if ((u + 1) * DCN_THREADS <= PIECES || e < PIECES) {
        const int k = e / (NBC * 4), r = e - k * (NBC * 4), col = r >> 2;
        st8<T>(bsm + ((k * NBC + col) * 4 + ((r & 3) ^ ((col >> 1) & 3))) * 8, v[u]);
      }
    }
  }
};

template <typename T, int NBC>
__device__ __forceinline__ typename DcnFrag<T>::frag b_read(const T* bsm, int k, int col, int grp) {
  return ld8<T>(bsm + ((k * NBC + col) * 4 + (grp ^ ((col >> 1) & 3))) * 8);
}

// ---- plain 3x3 convolution of one tile (footprint staged per chunk) -------------------------------
// acc[m][b] += sum over taps/chunks of x[footprint] * W[co0 + 16 b + row]; the
// footprint origin is (fy0, fx0) (may be negative: zero padding).  rx covers
// the image, rw the packed weights [cpad][nchunk][9][32].
template <typename T, int NBP, int PXS>
__device__ __forceinline__ void plain_conv(floatx4 (&acc)[DCN_WM][NBP], __amdgpu_buffer_rsrc_t rx,
                                           __amdgpu_buffer_rsrc_t rw, const T* wpk, int co0, int cpad, int nchunk,
                                           int cin8, int h, int w, int x_cs, int stride, int fy0, int fx0,
                                           const DcnGeom& g, T* region, T* bsm) {
  typedef DcnFrag<T> Ops;
  typedef typename Ops::frag frag;
  constexpr bool BLDS = sizeof(T) == 2;
  constexpr int NBC = NBP * 16;
  constexpr int PXB = PXS * (int)sizeof(T);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = lane & 15, grp = lane >> 4;
  const int fpix = g.fh * g.fw;
  // this lane's A rows: output pixel pl -> footprint byte offset of its (0, 0) tap
  int abase[DCN_WM];
#pragma unroll
  for (int m = 0; m < DCN_WM; ++m) {
    int pl = wave * (16 * DCN_WM) + m * 16 + row;
    if (pl >= g.th * g.tw) pl = 0;  // padding lane: any in-bounds address, result discarded
    const int py = (int)(((float)pl + 0.5f) * g.inv_tw), px = pl - py * g.tw;
    abase[m] = ((py * stride) * g.fw + px * stride) * PXB + grp * 8 * (int)sizeof(T);
  }
  const T* wrow[NBP];
#pragma unroll
  for (int b = 0; b < NBP; ++b) {
    const int co = co0 + b * 16 + row;
    wrow[b] = wpk + (int64_t)(co < cpad ? co : 0) * nchunk * 9 * 32 + grp * 8;
  }
  RegionTile<T, DCN_FCAP> rt;
  WeightTile<T, BLDS ? NBC : 1> wt;
  const int gq8 = (tid & 3) * 8;
  rt.setup(fy0, fx0, g.fw, fpix, g.inv_fw, h, w, x_cs, tid);
  rt.load(rx, 0, gq8 < cin8);
  if constexpr (BLDS) {
    wt.setup(co0, cpad, nchunk, tid);
    wt.load(rw, 0);
  }
  rt.store(region, PXS, tid);
  if constexpr (BLDS) wt.store(bsm, tid);
  for (int c = 0; c < nchunk; ++c) {
    __syncthreads();
    if (c + 1 < nchunk) {
      rt.load(rx, c + 1, (c + 1) * 32 + gq8 < cin8);
      if constexpr (BLDS) wt.load(rw, c + 1);
    }
    frag bn[NBP];
    if constexpr (!BLDS) {
#pragma unroll
      for (int b = 0; b < NBP; ++b) bn[b] = ld8<T>(wrow[b] + (c * 9) * 32);
    }
    int ky = 0, kx = 0;
#pragma unroll 1
    for (int k = 0; k < 9; ++k) {
      frag bf[NBP];
      if constexpr (BLDS) {
#pragma unroll
        for (int b = 0; b < NBP; ++b) bf[b] = b_read<T, NBC>(bsm, k, b * 16 + row, grp);
      } else {
#pragma unroll
        for (int b = 0; b < NBP; ++b) bf[b] = bn[b];
        if (k < 8) {
#pragma unroll
          for (int b = 0; b < NBP; ++b) bn[b] = ld8<T>(wrow[b] + (c * 9 + k + 1) * 32);
        }
      }
      const int toff = (ky * g.fw + kx) * PXB;
      frag af[DCN_WM];
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m) af[m] = ld8<T>((const T*)((const char*)region + abase[m] + toff));
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
        for (int b = 0; b < NBP; ++b) acc[m][b] = Ops::mma(af[m], bf[b], acc[m][b]);
      if (++kx == 3) {
        kx = 0;
        ++ky;
      }
    }
    if (c + 1 < nchunk) {
      __syncthreads();
      rt.store(region, PXS, tid);
      if constexpr (BLDS) wt.store(bsm, tid);
    }
  }
}

// ---- conv_offset of one tile, 16-bit input ------------------------------------------------------------
// Up to 3 channel chunks per round trip: the footprint [fpix][GS] goes to
// `region` and the 18 offset filters [9 taps][18][GS] to `bsm` (GS = 32 G + 8
// elements: rows 16 bytes apart in bank space, conflict-free for consecutive
// pixels / filters), all loads of a group issued at once; then 9 G k-steps of
// 2 x 2 MFMA with no barrier in between.  oacc[m][b]: offset channel 16 b + row.
template <typename T, int REGION_BYTES, int BSM_BYTES>
__device__ __forceinline__ void offset_conv16(floatx4 (&oacc)[DCN_WM][2], __amdgpu_buffer_rsrc_t rx,
                                              __amdgpu_buffer_rsrc_t rw, int nchunk, int cin8, int h, int w,
                                              int x_cs, int stride, int fy0, int fx0, const DcnGeom& g, T* region,
                                              T* bsm) {
  typedef DcnFrag<T> Ops;
  typedef typename Ops::frag frag;
  constexpr int NTF = 12, NTW = 8;           // footprint / filter pieces per thread per round
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = lane & 15, grp = lane >> 4;
  const int fpix = g.fh * g.fw;
  int apix[DCN_WM];
#pragma unroll
  for (int m = 0; m < DCN_WM; ++m) {
    int pl = wave * (16 * DCN_WM) + m * 16 + row;
    if (pl >= g.th * g.tw) pl = 0;
    const int py = (int)(((float)pl + 0.5f) * g.inv_tw), px = pl - py * g.tw;
    apix[m] = (py * stride) * g.fw + px * stride;
  }
  for (int c0 = 0; c0 < nchunk;) {
    int G = nchunk - c0 < 3 ? nchunk - c0 : 3;
    while (G > 1 && (fpix * (32 * G + 8) * (int)sizeof(T) > REGION_BYTES ||
                     9 * DCN_NOFF * (32 * G + 8) * (int)sizeof(T) > BSM_BYTES))
      --G;
    const int GS = 32 * G + 8, P4 = 4 * G;
    const float inv_p4 = 1.f / (float)P4;
    const int np = fpix * P4, nw = 9 * DCN_NOFF * P4;
    // one descriptor per pass (a buffer descriptor must be wave-uniform)
    for (int fb = 0, wb = 0; fb < np || wb < nw; fb += NTF * DCN_THREADS, wb += NTW * DCN_THREADS) {
      frag vf[NTF], vw[NTW];
      // pieces past np / nw are skipped by block-uniform branches (no address work, no load)
#pragma unroll
      for (int t = 0; t < NTF; ++t) {  // footprint piece: pixel q, 8 channels r of the group
        vf[t] = zero8<T>();
        if (fb + t * DCN_THREADS >= np) continue;
        const int e = fb + tid + t * DCN_THREADS;
        uint32_t o = DCN_OOB;
        if (e < np) {
          const int q = (int)(((float)e + 0.5f) * inv_p4), r = e - q * P4;
          const int qy = (int)(((float)q + 0.5f) * g.inv_fw), qx = q - qy * g.fw;
          const int gy = fy0 + qy, gx = fx0 + qx, ch = c0 * 32 + r * 8;
          if (gy >= 0 && gy < h && gx >= 0 && gx < w && ch < cin8)
            o = (uint32_t)(((gy * w + gx) * x_cs + ch) * (int)sizeof(T));
        }
        vf[t] = buf_ld8<T>(rx, o);
      }
#pragma unroll
      for (int t = 0; t < NTW; ++t) {  // filter piece: tap k, filter col, 8 channels r
        vw[t] = zero8<T>();
        if (wb + t * DCN_THREADS >= nw) continue;
        const int f = wb + tid + t * DCN_THREADS;
        uint32_t o = DCN_OOB;
        if (f < nw) {
          const int kc = (int)(((float)f + 0.5f) * inv_p4), r = f - kc * P4;
          const int k = kc / DCN_NOFF, col = kc - k * DCN_NOFF;
          o = (uint32_t)((((col * nchunk + c0 + (r >> 2)) * 9 + k) * 32 + (r & 3) * 8) * (int)sizeof(T));
        }
        vw[t] = buf_ld8<T>(rw, o);
      }
#pragma unroll
      for (int t = 0; t < NTF; ++t) {
        const int e = fb + tid + t * DCN_THREADS;
        if (e < np) {
          const int q = (int)(((float)e + 0.5f) * inv_p4), r = e - q * P4;
          st8<T>(region + q * GS + r * 8, vf[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < NTW; ++t) {
        const int f = wb + tid + t * DCN_THREADS;
        if (f < nw) {
          const int kc = (int)(((float)f + 0.5f) * inv_p4), r = f - kc * P4;
          st8<T>(bsm + kc * GS + r * 8, vw[t]);
        }
      }
    }
    __syncthreads();
    for (int gi = 0; gi < G; ++gi) {
      const int cofs = gi * 32 + grp * 8;
#pragma unroll
      for (int k = 0; k < 9; ++k) {  // unrolled: the scheduler runs LDS reads ahead of the MFMAs
        const frag b0 = ld8<T>(bsm + (k * DCN_NOFF + row) * GS + cofs);
        frag b1 = zero8<T>();
        if (row < DCN_NOFF - 16) b1 = ld8<T>(bsm + (k * DCN_NOFF + 16 + row) * GS + cofs);
        const int toff = (k / 3) * g.fw + k % 3;
#pragma unroll
        for (int m = 0; m < DCN_WM; ++m) {
          const frag af = ld8<T>(region + (apix[m] + toff) * GS + cofs);
          oacc[m][0] = Ops::mma(af, b0, oacc[m][0]);
          oacc[m][1] = Ops::mma(af, b1, oacc[m][1]);
        }
      }
    }
    __syncthreads();  // footprint / filters consumed before the next group (or the caller) reuses them
    c0 += G;
  }
}

// ---- fused squeeze-excitation of one image ------------------------------------------------------
// Cross-block exchange without fences.  A device-scope release fence writes
// back the whole L2 of the XCD (8 XCDs, each with its own L2), which costs
// microseconds per block; atomic read-modify-writes, by contrast, are
// performed at the memory-side coherence point for every XCD.  So every step
// of the exchange is a relaxed device-scope RMW whose returned value the
// thread waits for (the RMW has then been performed):
//  - each block stores its GAP partials with atomic exchanges and waits;
//  - after a barrier, thread 0 increments the image's arrival counter;
//  - the block that completes the count resets it (exchange with 0) and reads
//    every partial of the image with device-scope atomic loads (coherent across
//    XCDs: they do not return a stale line of the reader's L2).
// se_tail then forms g = se_inv_count * column sums of the [tiles][Cout]
// partials in a fixed order (thread (slice s, channel c) takes tiles s,
// s + nsl, ...; the slices are then added in order), so the result does not
// depend on which block came last; then att = sigmoid(W2 relu(W1 g + b1) + b2)
// with 4 lanes per output and a shuffle reduction.  lds: Cout + hid + THREADS floats.
// (dev_load / rmw_store: kad_common.h)

template <int THREADS>
__device__ __forceinline__ void se_tail(const float* __restrict__ partial, const float* __restrict__ w1,
                                        const float* __restrict__ b1, const float* __restrict__ w2,
                                        const float* __restrict__ b2, float* __restrict__ att, float inv_count, int C,
                                        int hid, int n, int tiles, float* lds) {
  constexpr int PB = 16;   // loads in flight per thread per batch
  constexpr int LPO = 4;   // lanes per MLP output (shuffle-reduced)
  constexpr int OPP = THREADS / LPO;  // outputs per pass
  const int tid = threadIdx.x;
  float* g = lds;          // [C]
  float* hb = g + C;       // [hid]
  float* red = hb + hid;   // [nsl][C]
  const float* pn = partial + (int64_t)n * tiles * C;
  const int nsl = C < THREADS ? THREADS / C : 1;
  for (int e = tid; e < nsl * C; e += THREADS) {
    const int s = e / C, ch = e - s * C;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int t0 = s; t0 < tiles; t0 += PB * nsl) {
      float v[PB];
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        const int t = t0 + u * nsl;
        v[u] = t < tiles ? dev_load(pn + (int64_t)t * C + ch) : 0.f;
      }
#pragma unroll
      for (int u = 0; u < PB; ++u) acc[u & 3] += v[u];
    }
    red[e] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
  __syncthreads();
  for (int ch = tid; ch < C; ch += THREADS) {
    float v = 0.f;
    for (int s = 0; s < nsl; ++s) v += red[s * C + ch];
    g[ch] = v * inv_count;
  }
  __syncthreads();
  const int part = tid & (LPO - 1);
  // out[o] = act(sum_k w[o][k] in[k] + b[o]): LPO lanes per output, each taking k = part, part + LPO, ...
  auto layer = [&](const float* __restrict__ w, const float* __restrict__ b, const float* in, int nin, int nout,
                   bool relu, float* dst) {
    for (int o0 = 0; o0 < nout; o0 += OPP) {
      const int o = o0 + tid / LPO;
      const float* wr = w + (int64_t)(o < nout ? o : 0) * nin;
      float acc = 0.f;
      for (int k0 = part; k0 < nin; k0 += PB * LPO) {
        float wv[PB];
#pragma unroll
        for (int u = 0; u < PB; ++u) {
          const int k = k0 + u * LPO;
          wv[u] = (o < nout && k < nin) ? wr[k] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < PB; ++u) {
          const int k = k0 + u * LPO;
          acc += wv[u] * in[k < nin ? k : 0];
        }
      }
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      if (o < nout && part == 0) {
        const float v = acc + (b ? b[o] : 0.f);
        dst[o] = relu ? fmaxf(v, 0.f) : sigmoidf_(v);
      }
    }
  };
  layer(w1, b1, g, C, hid, true, hb);
  __syncthreads();
  layer(w2, b2, hb, hid, C, false, att + (int64_t)n * C);
}

// ---- kernel ------------------------------------------------------------------------------------
// The block's work: tile-order index bx (XCD-aware, see below) and column block by of ny, of the
// problem (a, g).  dcn_fwd_kernel runs one problem per launch, dcn_group_kernel several.
template <typename T, typename OutT, int NBF, int MODE>
__device__ __forceinline__ void dcn_block(const kad_dcn_args& a, const DcnGeom& g, const int bx, const int by,
                                          const int ny) {
  typedef DcnFrag<T> Ops;
  typedef typename Ops::frag frag;
  typedef typename InfoOf<T>::type Info;
  typedef DcnLds<T, OutT, NBF, MODE> L;
  constexpr int NB = L::NB, PXS = L::PXS, PXB = L::PXB, RCAP = L::RCAP;
  constexpr bool BLDS = L::BLDS;
  __shared__ __align__(16) T region[RCAP * PXS];     // input region / footprint; epilogue tile at the end
  __shared__ __align__(16) T bsm[L::BSM];            // chunk weights [9][cols][32] (16-bit paths)
  __shared__ Info s_info[L::NINFO];                  // [9][128] corner offsets + weights
  __shared__ unsigned char s_slow[L::NINFO];         // [9][128] 1 = sample outside the capped region
  __shared__ float s_off[L::NOFF];                   // FUSED: [128][18] offsets of the tile
  __shared__ float s_par[4][NB];                     // bias, post_mul, post_add, post_scale
  __shared__ int s_box[4];       // ymin, ymax, xmin, xmax (clamped corners of live samples)
  __shared__ int s_reg[5];       // region y0, x0, rows, cols, capped flag

  // XCD-aware tile order over (image, tile) flattened: block b runs on XCD b % 8, which takes a
  // contiguous run of it (8 images: one image per XCD), so neighbouring tiles share their halos
  // through one L2; the column blocks of a tile (blockIdx.y) land on the same XCD.
  const int q = (bx & 7) * (g.grid_x >> 3) + (bx >> 3);
  if (q >= a.n * g.tiles) return;  // whole block, before any barrier
  const int n = q / g.tiles, tile = q - n * g.tiles;
  const int co0 = by * NB;
  const int tyi = tile / g.tiles_x;
  const int ty0 = tyi * g.th, tx0 = (tile - tyi * g.tiles_x) * g.tw;
  const int P = g.ho * g.wo;
  const int npx = g.th * g.tw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = lane & 15, grp = lane >> 4;
  const T* xb = (const T*)a.x + (int64_t)n * a.h * a.w * a.x_cs;
  const int cin8 = round_up(a.cin, 8);
  const T* wp = (const T*)a.wpack;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xb, (uint32_t)(a.h * a.w * a.x_cs * (int)sizeof(T)));
  const __amdgpu_buffer_rsrc_t rwp = make_rsrc(wp, (uint32_t)(g.cout_pad * g.nchunk * 9 * 32 * (int)sizeof(T)));
  const int fy0 = ty0 * a.stride - a.pad, fx0 = tx0 * a.stride - a.pad;

  // ---- 0. independent loads ------------------------------------------------------------------------
  float par[4] = {0.f, 1.f, 0.f, 1.f};
  if (tid < NB) {
    const int co = co0 + tid;
    if (co < a.cout) {
      if (a.bias) par[0] = a.bias[co];
      if (a.post_mul) par[1] = a.post_mul[co];
      if (a.post_add) par[2] = a.post_add[co];
      if (a.post_scale) par[3] = a.post_scale[co];
    }
  }
  // this thread's prologue pixel (taps tid / 128 + KSTEP u)
  const int ppl = tid & (DCN_TILE - 1);
  const int ppy = (int)(((float)ppl + 0.5f) * g.inv_tw), ppx = ppl - ppy * g.tw;
  const int poy = ty0 + ppy, pox = tx0 + ppx;
  const bool plive = ppl < npx && poy < g.ho && pox < g.wo;
  const int64_t pp = (int64_t)poy * g.wo + pox;
  float pre_dy[DCN_PPT], pre_dx[DCN_PPT], pre_m[DCN_PPT];
  if constexpr (MODE != MODE_PLAIN) {
#pragma unroll
    for (int u = 0; u < DCN_PPT; ++u) {
      const int k = tid / DCN_TILE + DCN_KSTEP * u;
      pre_dy[u] = pre_dx[u] = 0.f;
      pre_m[u] = 1.f;
      if (k < 9 && plive) {
        if constexpr (MODE == MODE_EXT) {
          pre_dy[u] = a.offset[n * a.off_sn + pp * a.off_sp + (2 * k) * a.off_sc];
          pre_dx[u] = a.offset[n * a.off_sn + pp * a.off_sp + (2 * k + 1) * a.off_sc];
        }
        if (a.mask) pre_m[u] = a.mask[n * a.mask_sn + pp * a.mask_sp + k * a.mask_sc];
      }
    }
  }
  if (tid == 0) {
    s_box[0] = 0x7fffffff;
    s_box[1] = -1;
    s_box[2] = 0x7fffffff;
    s_box[3] = -1;
  }

  floatx4 acc[DCN_WM][NBF];
#pragma unroll
  for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
    for (int b = 0; b < NBF; ++b) acc[m][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  if constexpr (MODE == MODE_PLAIN) {
    // ---- 1. plain 3x3 convolution -----------------------------------------------------------------
    plain_conv<T, NBF, PXS>(acc, rx, rwp, wp, co0, g.cout_pad, g.nchunk, cin8, a.h, a.w, a.x_cs, a.stride, fy0, fx0,
                            g, region, bsm);
  } else {
    if constexpr (MODE == MODE_FUSED) {
      // ---- 1. offsets = conv_offset(x) over the tile ----------------------------------------------------
      floatx4 oacc[DCN_WM][2];
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m) oacc[m][0] = oacc[m][1] = floatx4{0.f, 0.f, 0.f, 0.f};
      const __amdgpu_buffer_rsrc_t rwo = make_rsrc(a.off_wpack, (uint32_t)(32 * g.nchunk * 9 * 32 * (int)sizeof(T)));
      if constexpr (BLDS)
        offset_conv16<T, RCAP * PXB, L::BSM * (int)sizeof(T)>(oacc, rx, rwo, g.nchunk, cin8, a.h, a.w, a.x_cs,
                                                               a.stride, fy0, fx0, g, region, bsm);
      else
        plain_conv<T, 2, PXS>(oacc, rx, rwo, (const T*)a.off_wpack, 0, 32, g.nchunk, cin8, a.h, a.w, a.x_cs,
                              a.stride, fy0, fx0, g, region, bsm);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int ch = b * 16 + row;
        if (ch < DCN_NOFF) {
          const float ob = a.off_bias ? a.off_bias[ch] : 0.f;
#pragma unroll
          for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              s_off[(wave * (16 * DCN_WM) + m * 16 + grp * 4 + i) * DCN_NOFF + ch] = oacc[m][b][i] + ob;
        }
      }
      __syncthreads();  // offsets visible; footprint buffers free
    }
    // ---- 2. samples: clamped corners, weights, bounding box (registers) --------------------------------
    int bymin = 0x7fffffff, bymax = -1, bxmin = 0x7fffffff, bxmax = -1;
    int smp_yx[DCN_PPT], smp_st[DCN_PPT];
    float smp_w[DCN_PPT][4];
#pragma unroll
    for (int u = 0; u < DCN_PPT; ++u) {
      const int k = tid / DCN_TILE + DCN_KSTEP * u;
      float* w = smp_w[u];
      w[0] = w[1] = w[2] = w[3] = 0.f;
      int cy0 = 0, cx0 = 0, sy = 0, sx = 0;
      if (k < 9 && plive) {
        const int ky = k / 3, kx = k - (k / 3) * 3;
        float dy = pre_dy[u], dx = pre_dx[u];
        if constexpr (MODE == MODE_FUSED) {
          dy = s_off[ppl * DCN_NOFF + 2 * k];
          dx = s_off[ppl * DCN_NOFF + 2 * k + 1];
        }
        const float py = (float)(poy * a.stride - a.pad + ky) + dy;
        const float px = (float)(pox * a.stride - a.pad + kx) + dx;
        sample_geom(py, px, pre_m[u], a.h, a.w, cy0, cx0, sy, sx, w);
      }
      const bool live = w[0] != 0.f || w[1] != 0.f || w[2] != 0.f || w[3] != 0.f;
      if (live) {
        bymin = min(bymin, cy0);
        bymax = max(bymax, cy0 + sy);
        bxmin = min(bxmin, cx0);
        bxmax = max(bxmax, cx0 + sx);
      }
      smp_yx[u] = (cy0 << 15) | cx0;
      smp_st[u] = (sy << 1) | sx;
    }
    // wave-level then block-level bounding box (integer min / max: order-independent)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      bymin = min(bymin, __shfl_xor(bymin, o));
      bymax = max(bymax, __shfl_xor(bymax, o));
      bxmin = min(bxmin, __shfl_xor(bxmin, o));
      bxmax = max(bxmax, __shfl_xor(bxmax, o));
    }
    __syncthreads();  // s_box initialised
    if (lane == 0) {
      atomicMin(&s_box[0], bymin);
      atomicMax(&s_box[1], bymax);
      atomicMin(&s_box[2], bxmin);
      atomicMax(&s_box[3], bxmax);
    }
    __syncthreads();
    if (tid == 0) {
      int ry0 = s_box[0], ry1 = s_box[1], rx0 = s_box[2], rx1 = s_box[3];
      int capped = 0;
      if (ry1 < ry0 || rx1 < rx0) {  // no live sample at all
        ry0 = ry1 = rx0 = rx1 = 0;
      } else if ((ry1 - ry0 + 1) * (rx1 - rx0 + 1) > RCAP) {
        // keep the tile's own footprint plus the widest halo m that fits
        const int fy0c = max(fy0, 0), fy1 = min(fy0 + g.fh - 1, a.h - 1);
        const int fx0c = max(fx0, 0), fx1 = min(fx0 + g.fw - 1, a.w - 1);
        int m = 0;
        while (m < 4096) {
          const int y0n = max(ry0, fy0c - m - 1), y1n = min(ry1, fy1 + m + 1);
          const int x0n = max(rx0, fx0c - m - 1), x1n = min(rx1, fx1 + m + 1);
          if ((y1n - y0n + 1) * (x1n - x0n + 1) > RCAP) break;
          ++m;
        }
        const int y0n = max(ry0, fy0c - m), y1n = min(ry1, fy1 + m);
        const int x0n = max(rx0, fx0c - m), x1n = min(rx1, fx1 + m);
        if ((y1n - y0n + 1) * (x1n - x0n + 1) <= RCAP && y1n >= y0n && x1n >= x0n) {
          ry0 = y0n;
          ry1 = y1n;
          rx0 = x0n;
          rx1 = x1n;
        } else {  // degenerate (very wide tile footprint): a 1 x 1 region, everything global
          ry1 = ry0;
          rx1 = rx0;
        }
        capped = 1;
      }
      s_reg[0] = ry0;
      s_reg[1] = rx0;
      s_reg[2] = ry1 - ry0 + 1;
      s_reg[3] = rx1 - rx0 + 1;
      s_reg[4] = capped;
    }
    __syncthreads();
    const int ry0 = s_reg[0], rx0 = s_reg[1], rh = s_reg[2], rw = s_reg[3];
    const bool block_may_slow = s_reg[4] != 0;
    const int rpix = rh * rw;
    const float inv_rw = 1.f / (float)rw;
    const int gq8 = (tid & 3) * 8;

    // ---- 3. chunk 0 in flight while the sample records are written ------------------------------------
    RegionTile<T, RCAP> rt;
    WeightTile<T, BLDS ? NB : 1> wt;
    rt.setup(ry0, rx0, rw, rpix, inv_rw, a.h, a.w, a.x_cs, tid);
    rt.load(rx, 0, gq8 < cin8);
    if constexpr (BLDS) {
      wt.setup(co0, g.cout_pad, g.nchunk, tid);
      wt.load(rwp, 0);
    }
#pragma unroll
    for (int u = 0; u < DCN_PPT; ++u) {
      const int k = tid / DCN_TILE + DCN_KSTEP * u;
      if (k >= 9) break;
      const int q = k * DCN_TILE + ppl;
      float* w = smp_w[u];
      const int cy0 = smp_yx[u] >> 15, cx0 = smp_yx[u] & 0x7fff;
      const int sy = smp_st[u] >> 1, sx = smp_st[u] & 1;
      const int ly = cy0 - ry0, lx = cx0 - rx0;
      const bool dead = w[0] == 0.f && w[1] == 0.f && w[2] == 0.f && w[3] == 0.f;
      unsigned o[4] = {0u, 0u, 0u, 0u};
      unsigned char slow = 0;
      if (!dead && ly >= 0 && ly + sy < rh && lx >= 0 && lx + sx < rw) {
        const unsigned b0 = (unsigned)((ly * rw + lx) * PXB);
        const unsigned bxs = (unsigned)(sx * PXB), bys = (unsigned)(sy * rw * PXB);
        o[0] = b0;
        o[1] = b0 + bxs;
        o[2] = b0 + bys;
        o[3] = b0 + bys + bxs;
      } else {
        slow = dead ? 0 : 1;            // the fast path skips it; the slow pass adds it
        w[0] = w[1] = w[2] = w[3] = 0.f;
      }
      s_info[q] = make_info<T>(o, w);
      s_slow[q] = slow;
    }
    rt.store(region, PXS, tid);
    if constexpr (BLDS) wt.store(bsm, tid);

    const int ibase = wave * (16 * DCN_WM) + row;      // this lane's pixel slot within a tap row of s_info
    const T* wrow[NBF];                                // this lane's weight row (output channel) per fragment
#pragma unroll
    for (int b = 0; b < NBF; ++b) {
      const int co = co0 + b * 16 + row;
      wrow[b] = wp + (int64_t)(co < g.cout_pad ? co : 0) * g.nchunk * 9 * 32 + grp * 8;
    }
    for (int c = 0; c < g.nchunk; ++c) {
      __syncthreads();
      if (c + 1 < g.nchunk) {  // in flight during this chunk's taps
        rt.load(rx, c + 1, (c + 1) * 32 + gq8 < cin8);
        if constexpr (BLDS) wt.load(rwp, c + 1);
      }
      // lanes whose channel group lies past Cin read staged zeros: no masking needed
      frag bn[NBF];
      if constexpr (!BLDS) {
#pragma unroll
        for (int b = 0; b < NBF; ++b) bn[b] = ld8<T>(wrow[b] + (c * 9) * 32);
      }
      if constexpr (BLDS) {
        // Software-pipelined taps (fully unrolled, so the buffers rotate without
        // moves): the LDS reads of tap k + 1 (weights, corners) and the sample
        // records of tap k + 2 are in flight while tap k blends and multiplies.
        const char* rb = (const char*)region + grp * 8 * (int)sizeof(T);
        Info inf[3][DCN_WM];
        frag bq[2][NBF], cq[2][DCN_WM][4];
        auto rd_info = [&](int k, Info (&d)[DCN_WM]) {
#pragma unroll
          for (int m = 0; m < DCN_WM; ++m) d[m] = s_info[k * DCN_TILE + m * 16 + ibase];
        };
        auto rd_tap = [&](int k, const Info (&in)[DCN_WM], frag (&bd)[NBF], frag (&cd)[DCN_WM][4]) {
#pragma unroll
          for (int b = 0; b < NBF; ++b) bd[b] = b_read<T, NB>(bsm, k, b * 16 + row, grp);
#pragma unroll
          for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j) cd[m][j] = ld8<T>((const T*)(rb + corner(in[m], j)));
        };
        rd_info(0, inf[0]);
        rd_info(1, inf[1]);
        rd_tap(0, inf[0], bq[0], cq[0]);
#pragma unroll
        for (int k = 0; k < 9; ++k) {
          const int cur = k & 1, nxt = cur ^ 1;
          if (k + 2 < 9) rd_info(k + 2, inf[(k + 2) % 3]);
          if (k + 1 < 9) rd_tap(k + 1, inf[(k + 1) % 3], bq[nxt], cq[nxt]);
          frag af[DCN_WM];
#pragma unroll
          for (int m = 0; m < DCN_WM; ++m)
            af[m] = Ops::blend(cq[cur][m][0], cq[cur][m][1], cq[cur][m][2], cq[cur][m][3], inf[k % 3][m]);
#pragma unroll
          for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
            for (int b = 0; b < NBF; ++b) acc[m][b] = Ops::mma(af[m], bq[cur][b], acc[m][b]);
        }
      } else {
      Info ic[DCN_WM], inx[DCN_WM];
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m) inx[m] = s_info[m * 16 + ibase];
#pragma unroll 1
      for (int k = 0; k < 9; ++k) {
#pragma unroll
        for (int m = 0; m < DCN_WM; ++m) ic[m] = inx[m];
        if (k < 8) {
#pragma unroll
          for (int m = 0; m < DCN_WM; ++m) inx[m] = s_info[(k + 1) * DCN_TILE + m * 16 + ibase];
        }
        frag bf[NBF];
        {
#pragma unroll
          for (int b = 0; b < NBF; ++b) bf[b] = bn[b];
          if (k < 8) {
#pragma unroll
            for (int b = 0; b < NBF; ++b) bn[b] = ld8<T>(wrow[b] + (c * 9 + k + 1) * 32);
          }
        }
        frag af[DCN_WM];
#pragma unroll
        for (int m = 0; m < DCN_WM; ++m) {
          const char* rb = (const char*)region + grp * 8 * (int)sizeof(T);
          const frag v0 = ld8<T>((const T*)(rb + corner(ic[m], 0)));
          const frag v1 = ld8<T>((const T*)(rb + corner(ic[m], 1)));
          const frag v2 = ld8<T>((const T*)(rb + corner(ic[m], 2)));
          const frag v3 = ld8<T>((const T*)(rb + corner(ic[m], 3)));
          af[m] = Ops::blend(v0, v1, v2, v3, ic[m]);
        }
#pragma unroll
        for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
          for (int b = 0; b < NBF; ++b) acc[m][b] = Ops::mma(af[m], bf[b], acc[m][b]);
      }
      }
      if (c + 1 < g.nchunk) {
        __syncthreads();  // every wave is done with this chunk's region and weights
        rt.store(region, PXS, tid);
        if constexpr (BLDS) wt.store(bsm, tid);
      }
    }

    // ---- 3c. samples outside a capped region: straight from global memory (rare) ----------------------
    if (block_may_slow) {
      // The wave stays converged up to every MFMA (MFMA needs all 64 lanes):
      // lanes past Cin contribute zero fragments instead of branching away.
      for (int c = 0; c < g.nchunk; ++c) {
        const int ch = c * 32 + grp * 8;
        const bool ch_ok = ch < cin8;
#pragma unroll 1
        for (int k = 0; k < 9; ++k) {
          frag af[DCN_WM];
          bool any = false;
#pragma unroll
          for (int m = 0; m < DCN_WM; ++m) {
            const int q = k * DCN_TILE + m * 16 + ibase;
            af[m] = zero8<T>();
            if (ch_ok && s_slow[q]) {
              // recompute the sample's geometry (rare path)
              const int pl = m * 16 + ibase;
              const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
              const int oy = ty0 + oyl, ox = tx0 + pl - oyl * g.tw;
              const int64_t p = (int64_t)oy * g.wo + ox;
              float dy, dx;
              if constexpr (MODE == MODE_FUSED) {
                dy = s_off[pl * DCN_NOFF + 2 * k];
                dx = s_off[pl * DCN_NOFF + 2 * k + 1];
              } else {
                dy = a.offset[n * a.off_sn + p * a.off_sp + (2 * k) * a.off_sc];
                dx = a.offset[n * a.off_sn + p * a.off_sp + (2 * k + 1) * a.off_sc];
              }
              const float mk = a.mask ? a.mask[n * a.mask_sn + p * a.mask_sp + k * a.mask_sc] : 1.f;
              int cy0, cx0, sy, sx;
              float w[4];
              sample_geom((float)(oy * a.stride - a.pad + k / 3) + dy, (float)(ox * a.stride - a.pad + k % 3) + dx,
                          mk, a.h, a.w, cy0, cx0, sy, sx, w);
              const unsigned o0[4] = {0u, 0u, 0u, 0u};
              const Info in = make_info<T>(o0, w);
              const T* g0 = xb + ((int64_t)cy0 * a.w + cx0) * a.x_cs + ch;
              af[m] = Ops::blend(ld8<T>(g0), ld8<T>(g0 + sx * a.x_cs), ld8<T>(g0 + (int64_t)sy * a.w * a.x_cs),
                                 ld8<T>(g0 + ((int64_t)sy * a.w + sx) * a.x_cs), in);
              any = true;
            }
          }
          if (__builtin_amdgcn_ballot_w64(any) == 0) continue;
#pragma unroll
          for (int b = 0; b < NBF; ++b) {
            const frag bw = ld8<T>(wrow[b] + (c * 9 + k) * 32);
#pragma unroll
            for (int m = 0; m < DCN_WM; ++m) acc[m][b] = Ops::mma(af[m], bw, acc[m][b]);
          }
        }
      }
    }
  }

  // ---- 4. epilogue: values -> LDS tile -> row-contiguous stores; GAP partials ------------------------
  constexpr int SROW = L::SROW;
  OutT* ost = (OutT*)region;
  float(*gap_red)[NB] = (float(*)[NB])((char*)region + L::STAGE_BYTES);
  // the epilogue parameters, loaded at the start, are staged only now: storing them
  // there would have held waves 0-1 for a global round trip before the offset conv
  if (tid < NB) {  // v = acc * mul + (bias * mul + add)
    s_par[0][tid] = par[0] * par[1] + par[2];
    s_par[1][tid] = par[1];
    s_par[3][tid] = par[3];
  }
  __syncthreads();  // every wave is done reading the region; s_par staged
  bool pix_ok[DCN_WM][4];
#pragma unroll
  for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pl = wave * (16 * DCN_WM) + m * 16 + grp * 4 + i;
      const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
      pix_ok[m][i] = pl < npx && ty0 + oyl < g.ho && tx0 + pl - oyl * g.tw < g.wo;
    }
  float gsum[NBF];
  // the activation as a template argument: a per-value branch would put every value's chain in a
  // basic block of its own, and the scheduler could not interleave the independent chains
  auto epilogue = [&](auto act) {
    constexpr int ACT = decltype(act)::value;
#pragma unroll
    for (int b = 0; b < NBF; ++b) {
      gsum[b] = 0.f;
      const int col = b * 16 + row;
      const bool co_ok = co0 + col < a.cout;
      const float shift = s_par[0][col], mul = s_par[1][col], scl = s_par[3][col];
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int pl = wave * (16 * DCN_WM) + m * 16 + grp * 4 + i;
          float v = fmaf(acc[m][b][i], mul, shift);
          if constexpr (ACT == KAD_ACT_SILU) v = v * sigmoidf_(v);
          else if constexpr (ACT == KAD_ACT_RELU) v = fmaxf(v, 0.f);
          v *= scl;
          const OutT o = from_f32<OutT>(v);
          ost[pl * SROW + col] = o;
          if (co_ok && pix_ok[m][i]) gsum[b] += to_f32(o);
        }
      }
    }
  };
  if (a.relu == KAD_ACT_SILU) epilogue(std::integral_constant<int, KAD_ACT_SILU>{});
  else if (a.relu) epilogue(std::integral_constant<int, KAD_ACT_RELU>{});
  else epilogue(std::integral_constant<int, KAD_ACT_NONE>{});
  if (a.gap_partial) {
#pragma unroll
    for (int b = 0; b < NBF; ++b) {
      float v = gsum[b];
      v = sum_xor32(sum_xor16(v));
      if (grp == 0) gap_red[wave][b * 16 + row] = v;
    }
  }
  __syncthreads();
  OutT* out = (OutT*)a.out;
  constexpr int VEC = 16 / (int)sizeof(OutT);
  const bool vec_ok = a.out_layout == KAD_NHWC && (a.out_cs * (int)sizeof(OutT)) % 16 == 0 &&
                      ((uintptr_t)a.out & 15) == 0;
  if (vec_ok) {
    constexpr int VPP = NB / VEC;  // 16-byte vectors per pixel
    for (int j = tid; j < DCN_TILE * VPP; j += DCN_THREADS) {
      const int pl = j / VPP, v = j - pl * VPP;
      const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
      const int oy = ty0 + oyl, ox = tx0 + pl - oyl * g.tw;
      const int co = co0 + v * VEC;
      if (pl >= npx || oy >= g.ho || ox >= g.wo || co >= a.cout) continue;
      const OutT* src = ost + pl * SROW + v * VEC;
      OutT* dst = out + ((int64_t)n * P + (int64_t)oy * g.wo + ox) * a.out_cs + co;
      if (co + VEC <= a.cout) {
        *(intx4*)dst = *(const intx4*)src;
      } else {
        for (int e = 0; e < a.cout - co; ++e) dst[e] = src[e];
      }
    }
  } else if (a.out_layout == KAD_NHWC) {
    for (int j = tid; j < DCN_TILE * NB; j += DCN_THREADS) {
      const int pl = j / NB, col = j - pl * NB;
      const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
      const int oy = ty0 + oyl, ox = tx0 + pl - oyl * g.tw;
      const int co = co0 + col;
      if (pl >= npx || oy >= g.ho || ox >= g.wo || co >= a.cout) continue;
      out[((int64_t)n * P + (int64_t)oy * g.wo + ox) * a.out_cs + co] = ost[pl * SROW + col];
    }
  } else {  // NCHW: consecutive lanes along the tile's pixels; a thread keeps its pixel for every channel
    static_assert(DCN_THREADS % DCN_TILE == 0, "one pixel per thread across channel steps");
    constexpr int CSTEP = DCN_THREADS / DCN_TILE;
    const int pl = tid % DCN_TILE, col0 = tid / DCN_TILE;
    const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
    const int oy = ty0 + oyl, ox = tx0 + pl - oyl * g.tw;
    if (pl < npx && oy < g.ho && ox < g.wo) {
      OutT* dst = out + ((int64_t)n * a.out_cs + co0 + col0) * P + (int64_t)oy * g.wo + ox;
      const OutT* src = ost + pl * SROW + col0;
      const int ncol = a.cout - co0 < NB ? a.cout - co0 : NB;
#pragma unroll 4
      for (int col = col0; col < ncol; col += CSTEP) {
        *dst = *src;
        dst += (int64_t)CSTEP * P;
        src += CSTEP;
      }
    }
  }
  if (a.gap_partial && tid < NB) {
    const int co = co0 + tid;
    if (co < a.cout) {
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < DCN_WAVES; ++i) v += gap_red[i][tid];
      float* dst = a.gap_partial + ((int64_t)n * g.tiles + tile) * a.cout + co;
      if (MODE != MODE_PLAIN && a.se_att)
        rmw_store(dst, v);  // read by another block of this launch (fused SE)
      else
        *dst = v;
    }
  }

  // ---- 5. fused squeeze-excitation: the image's last block runs the MLP -------------------------------
  // (exchange protocol at se_tail)
  if constexpr (MODE != MODE_PLAIN) {
    if (a.se_att && a.gap_partial) {
      __shared__ int s_last;
      // This block's partial exchanges are performed (each thread waited for its exchange's
      // return) and the epilogue's LDS tile is free.  The barrier waits for LDS traffic only,
      // not for the acknowledgements of the output stores, which no one here reads.
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (tid == 0) {
        const unsigned total = (unsigned)g.tiles * ny;
        const unsigned prev = __hip_atomic_fetch_add(a.se_count + n, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev + 1u == total;
        if (last) {
          const unsigned z = __hip_atomic_exchange(a.se_count + n, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          asm volatile("" ::"v"(z));
        }
        s_last = last;
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (s_last) {
        se_tail<DCN_THREADS>(a.gap_partial, a.se_w1, a.se_b1, a.se_w2, a.se_b2, a.se_att, a.se_inv_count, a.cout, a.se_hid, n,
                g.tiles, (float*)region);
      }
    }
  }
}

template <typename T, typename OutT, int NBF, int MODE>
__global__ __launch_bounds__(DCN_THREADS, 1) void dcn_fwd_kernel(kad_dcn_args a, DcnGeom g) {
  dcn_block<T, OutT, NBF, MODE>(a, g, blockIdx.x, blockIdx.y, gridDim.y);
}

// Several independent problems of one instantiation (same dtype, mode and column-fragment count)
// in one grid: problem p owns blocks [start[p], start[p + 1]) (its grid_x x ny blocks, start a
// multiple of 8 so a block's XCD, id % 8, is its tile order's).  The three branches of a KAD-Conv
// layer run their DSCs this way, as one launch instead of three concurrent streams.
struct DcnGroup {
  kad_dcn_args a[KAD_DCN_GROUP_MAX];
  DcnGeom g[KAD_DCN_GROUP_MAX];
  int start[KAD_DCN_GROUP_MAX + 1];
  int ny[KAD_DCN_GROUP_MAX];
  int count;
};

template <typename T, typename OutT, int NBF, int MODE>
__global__ __launch_bounds__(DCN_THREADS, 1) void dcn_group_kernel(DcnGroup grp) {
  const int id = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < KAD_DCN_GROUP_MAX; ++i)
    if (i < grp.count && id >= grp.start[i]) p = i;
  if (id >= grp.start[p + 1]) return;
  const int local = id - grp.start[p];
  const int gx = grp.g[p].grid_x;
  // p is uniform over the block: the problem's fields are scalar loads from kernel-argument memory
  dcn_block<T, OutT, NBF, MODE>(grp.a[p], grp.g[p], local % gx, local / gx, grp.ny[p]);
}

// ---- 16-bit DCN / DSC with two blocks per CU ------------------------------------------------------
// The 16-bit FUSED and EXT paths at stride 1 with up to 64 output channels and many tiles (KAD-CNet's
// small DSCs; the dispatch rule and its measurements are at d2_ok).  On gfx950 LDS delivers ~128 B/clk per CU and L1 hits ~64 B/clk; the
// tap loop of the 8-wave kernel above is bound by LDS reads, most of them weight fragments that
// every wave re-reads for its 16 pixels.  Here:
//  * 4 waves x 32 pixels (two 16-pixel A fragments per wave): half the weight-fragment reads per
//    pixel, and they come from global memory (L1 / L2 hits: a column block's packed weights are
//    at most 9 x 64 x 64 x 2 bytes), so LDS carries only the corner reads;
//  * LDS < 80 KB, so two blocks share a CU and one block's latency-bound phases (conv_offset,
//    sample setup, epilogue) overlap the other's taps;
//  * input channels in 16-channel half-chunks: a Cin of 10 .. 16 is padded to 16, not 32;
//  * the input region is staged per 16-channel half-chunk by direct global -> LDS loads
//    (buffer_load_dwordx4 ... lds: lane l's 16 bytes land at base + 16 l, out-of-range pieces as
//    zeros), double-buffered: no registers hold the prefetch.  32 bytes per region pixel
//    (channels 8 h .. 8 h + 7 at byte 16 h);
//  * one MFMA k-step covers two taps of a half-chunk: lane groups 0-1 take tap 2 j, groups 2-3
//    tap 2 j + 1 (tap 9 is zero); five k-steps per half-chunk;
//  * the sample records (corner offset, corner steps, blend weights) are built once and held in
//    registers through all half-chunks (ten per lane).
// Vector-memory loads retire in issue order (one counter), so a weight load issued after a
// region prefetch also waits for the prefetch.  The next half-chunk's region is requested right
// after the current half-chunk's last weight loads (a three-stage weight pipeline) and waited for
// at the half-chunk barrier.
constexpr int D2_THREADS = 256;
constexpr int D2_WAVES = 4;
constexpr int D2_TILE = 128;                   // pixels per block: wave w owns [32 w, 32 w + 32)
constexpr int D2_PPT = 5;                      // samples per thread: pixel tid % 128, taps tid / 128 + 2 u
constexpr int D2_RCAP = 1024;                  // region pixels per half-chunk buffer
constexpr int D2_RBUF = D2_RCAP * 32;          // bytes per region buffer
// shared area (conv_offset staging, offsets, region buffers, epilogue, SE): NRB * D2_RBUF bytes
constexpr int D2_RINST = D2_RCAP * 2 / 64 / D2_WAVES;  // direct loads per wave per half-chunk
constexpr int D2_NBF_MAX = 4;
constexpr unsigned D2_SLOW = 0x80000000u;      // record flag: sample outside the region (read from memory)
static_assert(DCN_TILE == D2_TILE && D2_THREADS / D2_TILE == 2, "sample geometry");

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from buffer r at voff (0 if voff is out of range) to LDS: lane l writes
// lds_base + 16 l; lds_base must be wave-uniform.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, void* lds_base, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds_base, 16, voff, 0, 0, 0);
}

// conv_offset of the tile (stride 1) with 4 waves x two pixel fragments: per round G 32-channel
// chunks of the footprint [fpix][8 R] and of the 18 filters [9 taps x 18][8 R] (R = 4 G + 1
// 16-byte slots per row, the last one zero: rows 16 bytes apart in bank space) are loaded
// straight into LDS, then 9 G k-steps of 2 x 2 MFMA.  oacc[m][b]: offset channel 16 b + row.
template <typename T>
__device__ __forceinline__ void d2_offset_conv(floatx4 (&oacc)[2][2], __amdgpu_buffer_rsrc_t rx, const kad_dcn_args& a,
                                               const DcnGeom& g, int fy0, int fx0, int cin8, unsigned char* su,
                                               int su_bytes) {
  typedef DcnFrag<T> Ops;
  typedef typename Ops::frag frag;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = lane & 15, grp = lane >> 4;
  const int fpix = g.fh * g.fw, npx = g.th * g.tw;
  const __amdgpu_buffer_rsrc_t rwo = make_rsrc(a.off_wpack, (uint32_t)(32 * g.nchunk * 9 * 32 * (int)sizeof(T)));
  int apix[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    int pl = wave * 32 + m * 16 + row;
    if (pl >= npx) pl = 0;  // padding lane: any in-bounds address, result discarded
    const int py = (int)(((float)pl + 0.5f) * g.inv_tw), px = pl - py * g.tw;
    apix[m] = py * g.fw + px;
  }
  for (int c0 = 0; c0 < g.nchunk;) {
    int G = g.nchunk - c0 < 3 ? g.nchunk - c0 : 3;
    while (G > 1 && (ceil_div(fpix * (4 * G + 1), 64) + ceil_div(9 * DCN_NOFF * (4 * G + 1), 64)) * 1024 > su_bytes) --G;
    const int R = 4 * G + 1, GS = 8 * R;
    const float inv_r = 1.f / (float)R;
    const int nif = ceil_div(fpix * R, 64), niw = ceil_div(9 * DCN_NOFF * R, 64);
    const T* foot = (const T*)su;
    const T* filt = (const T*)(su + nif * 1024);
    for (int i = wave; i < nif + niw; i += D2_WAVES) {  // wave-uniform: one direct load per i
      uint32_t o = KAD_OOB;
      if (i < nif) {
        const int s = i * 64 + lane;
        const int q = (int)(((float)s + 0.5f) * inv_r), r = s - q * R;
        if (q < fpix && r < 4 * G) {
          const int qy = (int)(((float)q + 0.5f) * g.inv_fw), qx = q - qy * g.fw;
          const int gy = fy0 + qy, gx = fx0 + qx, ch = c0 * 32 + r * 8;
          if (gy >= 0 && gy < a.h && gx >= 0 && gx < a.w && ch < cin8)
            o = (uint32_t)(((gy * a.w + gx) * a.x_cs + ch) * (int)sizeof(T));
        }
        lds_load16(rx, su + i * 1024, o);
      } else {
        const int s = (i - nif) * 64 + lane;
        const int kc = (int)(((float)s + 0.5f) * inv_r), r = s - kc * R;
        if (kc < 9 * DCN_NOFF && r < 4 * G) {
          const int k = kc / DCN_NOFF, col = kc - k * DCN_NOFF;
          o = (uint32_t)((((col * g.nchunk + c0 + (r >> 2)) * 9 + k) * 32 + (r & 3) * 8) * (int)sizeof(T));
        }
        lds_load16(rwo, su + i * 1024, o);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int gi = 0; gi < G; ++gi) {
      const int cofs = gi * 32 + grp * 8;
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        const frag b0 = ld8<T>(filt + (k * DCN_NOFF + row) * GS + cofs);
        frag b1 = zero8<T>();
        if (row < DCN_NOFF - 16) b1 = ld8<T>(filt + (k * DCN_NOFF + 16 + row) * GS + cofs);
        const int toff = (k / 3) * g.fw + k % 3;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const frag af = ld8<T>(foot + (apix[m] + toff) * GS + cofs);
          oacc[m][0] = Ops::mma(af, b0, oacc[m][0]);
          oacc[m][1] = Ops::mma(af, b1, oacc[m][1]);
        }
      }
    }
    __syncthreads();  // staging consumed before the next round (or the caller) reuses it
    c0 += G;
  }
}

// NRB: region buffers.  One suffices when Cin <= 16 (a single half-chunk, nothing to prefetch): the
// block then needs ~46 KB of LDS instead of ~78 KB, three blocks per CU instead of two (the host
// checks that the conv_offset staging and the SE scratch fit the smaller shared area).
template <typename T, int NBF, int MODE, int NRB>
__device__ __forceinline__ void dsc2_block(const kad_dcn_args& a, const DcnGeom& g, const int bx, const int by,
                                           const int ny) {
  static_assert(sizeof(T) == 2 && NBF <= D2_NBF_MAX && MODE != MODE_PLAIN, "16-bit DCN / DSC only");
  static_assert(NRB == 1 || NRB == 2, "one or two region buffers");
  typedef DcnFrag<T> Ops;
  typedef typename Ops::frag frag;
  constexpr int NB = NBF * 16;
  constexpr int SU = NRB * D2_RBUF;
  __shared__ __align__(16) unsigned char s_u[SU];  // staging / offsets / region buffers / epilogue / SE
  __shared__ unsigned s_ia[9 * D2_TILE];            // [tap][pixel] record: region offset + steps, or D2_SLOW
  __shared__ uint2 s_iw[9 * D2_TILE];               // [tap][pixel] corner weights (2 x half2)
  __shared__ float s_par[3][NB];                    // shift, mul, scale
  __shared__ int s_box[4];
  __shared__ int s_reg[5];

  // XCD-aware tile order, as dcn_block
  const int q = (bx & 7) * (g.grid_x >> 3) + (bx >> 3);
  if (q >= a.n * g.tiles) return;  // whole block, before any barrier
  const int n = q / g.tiles, tile = q - n * g.tiles;
  const int co0 = by * NB;
  const int tyi = tile / g.tiles_x;
  const int ty0 = tyi * g.th, tx0 = (tile - tyi * g.tiles_x) * g.tw;
  const int P = g.ho * g.wo, npx = g.th * g.tw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = lane & 15, grp = lane >> 4;
  const T* xb = (const T*)a.x + (int64_t)n * a.h * a.w * a.x_cs;
  const int cin8 = round_up(a.cin, 8);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xb, (uint32_t)(a.h * a.w * a.x_cs * (int)sizeof(T)));
  const __amdgpu_buffer_rsrc_t rwp =
      make_rsrc(a.wpack, (uint32_t)(g.cout_pad * g.nchunk * 9 * 32 * (int)sizeof(T)));
  const int fy0 = ty0 - a.pad, fx0 = tx0 - a.pad;

  // ---- 0. independent loads ------------------------------------------------------------------------
  float par[4] = {0.f, 1.f, 0.f, 1.f};
  if (tid < NB) {
    const int co = co0 + tid;
    if (co < a.cout) {
      if (a.bias) par[0] = a.bias[co];
      if (a.post_mul) par[1] = a.post_mul[co];
      if (a.post_add) par[2] = a.post_add[co];
      if (a.post_scale) par[3] = a.post_scale[co];
    }
  }
  const int ppl = tid & (D2_TILE - 1);
  const int ppy = (int)(((float)ppl + 0.5f) * g.inv_tw), ppx = ppl - ppy * g.tw;
  const int poy = ty0 + ppy, pox = tx0 + ppx;
  const bool plive = ppl < npx && poy < g.ho && pox < g.wo;
  const int64_t pp = (int64_t)poy * g.wo + pox;
  float pre_dy[D2_PPT], pre_dx[D2_PPT], pre_m[D2_PPT];
#pragma unroll
  for (int u = 0; u < D2_PPT; ++u) {
    const int k = (tid >> 7) + 2 * u;
    pre_dy[u] = pre_dx[u] = 0.f;
    pre_m[u] = 1.f;
    if (k < 9 && plive) {
      if constexpr (MODE == MODE_EXT) {
        pre_dy[u] = a.offset[n * a.off_sn + pp * a.off_sp + (2 * k) * a.off_sc];
        pre_dx[u] = a.offset[n * a.off_sn + pp * a.off_sp + (2 * k + 1) * a.off_sc];
      }
      if (a.mask) pre_m[u] = a.mask[n * a.mask_sn + pp * a.mask_sp + k * a.mask_sc];
    }
  }
  if (tid == 0) {
    s_box[0] = 0x7fffffff;
    s_box[1] = -1;
    s_box[2] = 0x7fffffff;
    s_box[3] = -1;
  }

  // ---- 1. FUSED: offsets = conv_offset(x) over the tile -> s_off [128][18] (fp32, in s_u) ---------
  const float* s_off = (const float*)s_u;
  if constexpr (MODE == MODE_FUSED) {
    floatx4 oacc[2][2];
#pragma unroll
    for (int m = 0; m < 2; ++m) oacc[m][0] = oacc[m][1] = floatx4{0.f, 0.f, 0.f, 0.f};
    d2_offset_conv<T>(oacc, rx, a, g, fy0, fx0, cin8, s_u, SU);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int ch = b * 16 + row;
      if (ch < DCN_NOFF) {
        const float ob = a.off_bias ? a.off_bias[ch] : 0.f;
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            ((float*)s_u)[(wave * 32 + m * 16 + grp * 4 + i) * DCN_NOFF + ch] = oacc[m][b][i] + ob;
      }
    }
    __syncthreads();
  }

  // ---- 2. samples: clamped corners, weights, bounding box ----------------------------------------------
  int bymin = 0x7fffffff, bymax = -1, bxmin = 0x7fffffff, bxmax = -1;
  int smp_yx[D2_PPT], smp_st[D2_PPT];
  float smp_w[D2_PPT][4];
#pragma unroll
  for (int u = 0; u < D2_PPT; ++u) {
    const int k = (tid >> 7) + 2 * u;
    float* w = smp_w[u];
    w[0] = w[1] = w[2] = w[3] = 0.f;
    int cy0 = 0, cx0 = 0, sy = 0, sx = 0;
    if (k < 9 && plive) {
      const int ky = k / 3, kx = k - (k / 3) * 3;
      float dy = pre_dy[u], dx = pre_dx[u];
      if constexpr (MODE == MODE_FUSED) {
        dy = s_off[ppl * DCN_NOFF + 2 * k];
        dx = s_off[ppl * DCN_NOFF + 2 * k + 1];
      }
      const float py = (float)(poy - a.pad + ky) + dy;
      const float px = (float)(pox - a.pad + kx) + dx;
      sample_geom(py, px, pre_m[u], a.h, a.w, cy0, cx0, sy, sx, w);
    }
    const bool live = w[0] != 0.f || w[1] != 0.f || w[2] != 0.f || w[3] != 0.f;
    if (live) {
      bymin = min(bymin, cy0);
      bymax = max(bymax, cy0 + sy);
      bxmin = min(bxmin, cx0);
      bxmax = max(bxmax, cx0 + sx);
    }
    smp_yx[u] = (cy0 << 15) | cx0;
    smp_st[u] = (sy << 1) | sx;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    bymin = min(bymin, __shfl_xor(bymin, o));
    bymax = max(bymax, __shfl_xor(bymax, o));
    bxmin = min(bxmin, __shfl_xor(bxmin, o));
    bxmax = max(bxmax, __shfl_xor(bxmax, o));
  }
  __syncthreads();  // s_box initialised; every s_off read done (s_u is free from here)
  if (lane == 0) {
    atomicMin(&s_box[0], bymin);
    atomicMax(&s_box[1], bymax);
    atomicMin(&s_box[2], bxmin);
    atomicMax(&s_box[3], bxmax);
  }
  __syncthreads();
  if (tid == 0) {
    int ry0 = s_box[0], ry1 = s_box[1], rx0 = s_box[2], rx1 = s_box[3];
    int capped = 0;
    if (ry1 < ry0 || rx1 < rx0) {  // no live sample at all
      ry0 = ry1 = rx0 = rx1 = 0;
    } else if ((ry1 - ry0 + 1) * (rx1 - rx0 + 1) > D2_RCAP) {
      // keep the tile's own footprint plus the widest halo m that fits
      const int fy0c = max(fy0, 0), fy1 = min(fy0 + g.fh - 1, a.h - 1);
      const int fx0c = max(fx0, 0), fx1 = min(fx0 + g.fw - 1, a.w - 1);
      int m = 0;
      while (m < 4096) {
        const int y0n = max(ry0, fy0c - m - 1), y1n = min(ry1, fy1 + m + 1);
        const int x0n = max(rx0, fx0c - m - 1), x1n = min(rx1, fx1 + m + 1);
        if ((y1n - y0n + 1) * (x1n - x0n + 1) > D2_RCAP) break;
        ++m;
      }
      const int y0n = max(ry0, fy0c - m), y1n = min(ry1, fy1 + m);
      const int x0n = max(rx0, fx0c - m), x1n = min(rx1, fx1 + m);
      if ((y1n - y0n + 1) * (x1n - x0n + 1) <= D2_RCAP && y1n >= y0n && x1n >= x0n) {
        ry0 = y0n;
        ry1 = y1n;
        rx0 = x0n;
        rx1 = x1n;
      } else {  // degenerate: a 1 x 1 region, everything from memory
        ry1 = ry0;
        rx1 = rx0;
      }
      capped = 1;
    }
    s_reg[0] = ry0;
    s_reg[1] = rx0;
    s_reg[2] = ry1 - ry0 + 1;
    s_reg[3] = rx1 - rx0 + 1;
    s_reg[4] = capped;
  }
  __syncthreads();
  const int ry0 = s_reg[0], rx0 = s_reg[1], rh = s_reg[2], rw = s_reg[3];
  const bool block_may_slow = s_reg[4] != 0;
  const int rpix = rh * rw;

  // ---- 3. region staging: slot s = 64 (wave + 4 u) + lane holds region pixel s / 2, half s % 2 -----
  uint32_t rpx[D2_RINST];
  {
    const float inv_rw = 1.f / (float)rw;
#pragma unroll
    for (int u = 0; u < D2_RINST; ++u) {
      const int s = 64 * (wave + D2_WAVES * u) + lane, rq = s >> 1;
      uint32_t o = KAD_OOB;
      if (rq < rpix) {
        const int qy = (int)(((float)rq + 0.5f) * inv_rw);
        o = (uint32_t)((((ry0 + qy) * a.w + rx0 + rq - qy * rw) * a.x_cs + 8 * (s & 1)) * (int)sizeof(T));
      }
      rpx[u] = o;
    }
  }
  // Every wave issues all D2_RINST loads (slots past the region read out of range and store
  // zeros, inside the buffer): a fixed count lets the compiler's waits on later weight loads
  // count past them instead of waiting for them.
  auto stage = [&](int h) {  // half-chunk h (channels 16 h .. 16 h + 15) into buffer h % 2
    const bool ch_ok = 16 * h + 8 * (lane & 1) < cin8;
    unsigned char* dst = s_u + (h & 1) * D2_RBUF + 1024 * wave;
#pragma unroll
    for (int u = 0; u < D2_RINST; ++u)
      lds_load16(rx, dst + 1024 * D2_WAVES * u, (ch_ok && rpx[u] != KAD_OOB) ? rpx[u] + 32 * h : KAD_OOB);
  };
  stage(0);

  // sample records (region byte offset | sx << 16 | sy << 17, or D2_SLOW with the image corner)
#pragma unroll
  for (int u = 0; u < D2_PPT; ++u) {
    const int k = (tid >> 7) + 2 * u;
    if (k >= 9) break;
    const float* w = smp_w[u];
    const int cy0 = smp_yx[u] >> 15, cx0 = smp_yx[u] & 0x7fff;
    const int sy = smp_st[u] >> 1, sx = smp_st[u] & 1;
    const int ly = cy0 - ry0, lx = cx0 - rx0;
    const bool dead = w[0] == 0.f && w[1] == 0.f && w[2] == 0.f && w[3] == 0.f;
    unsigned ia = 0u;
    if (!dead) {
      if (ly >= 0 && ly + sy < rh && lx >= 0 && lx + sx < rw)
        ia = (unsigned)((ly * rw + lx) * 32) | ((unsigned)sx << 16) | ((unsigned)sy << 17);
      else
        ia = D2_SLOW | ((unsigned)sy << 30) | ((unsigned)sx << 29) | ((unsigned)cy0 << 14) | (unsigned)cx0;
    }
    s_ia[k * D2_TILE + ppl] = ia;
    s_iw[k * D2_TILE + ppl] = make_uint2(pack_h2(w[0], w[1]), pack_h2(w[2], w[3]));
  }
  __syncthreads();  // records visible

  // this lane's records: k-step j, fragment m -> tap 2 j + (grp >> 1), pixel 32 wave + 16 m + row
  unsigned r_a[5][2], r_w01[5][2], r_w23[5][2];
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const int kt = 2 * j + (grp >> 1);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      unsigned ia = 0u;
      uint2 wv = make_uint2(0u, 0u);
      if (kt < 9) {
        const int qi = kt * D2_TILE + wave * 32 + m * 16 + row;
        ia = s_ia[qi];
        wv = s_iw[qi];
        if (ia & D2_SLOW) {  // added by the pass from memory
          ia = 0u;
          wv = make_uint2(0u, 0u);
        }
      }
      r_a[j][m] = ia;
      r_w01[j][m] = wv.x;
      r_w23[j][m] = wv.y;
    }
  }

  // weight fragment (column fragment f, half-chunk h, k-step j): lane (row, grp) reads column
  // co0 + 16 f + row, tap 2 j + (grp >> 1), channels 16 h + 8 (grp & 1) .. + 7 of the packed
  // [cout_pad][nchunk][9][32] weights; tap 9 reads nothing (zero)
  uint32_t wcol[NBF];
#pragma unroll
  for (int f = 0; f < NBF; ++f) {
    const int co = co0 + f * 16 + row;
    wcol[f] = (uint32_t)(((co < g.cout_pad ? co : 0) * g.nchunk * 288 + (grp >> 1) * 32 + (grp & 1) * 8) *
                         (int)sizeof(T));
  }
  auto ld_w = [&](int h, int j, frag (&d)[NBF]) {
    const bool pad = j == 4 && (grp >> 1) != 0;
    const uint32_t so = (uint32_t)((((h >> 1) * 9 + 2 * j) * 32 + (h & 1) * 16) * (int)sizeof(T));
#pragma unroll
    for (int f = 0; f < NBF; ++f) d[f] = buf_ld8<T>(rwp, pad ? KAD_OOB : wcol[f] + so);
  };

  floatx4 acc[2][NBF];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int f = 0; f < NBF; ++f) acc[m][f] = floatx4{0.f, 0.f, 0.f, 0.f};

  // ---- 4. taps: nh half-chunks x 5 k-steps -----------------------------------------------------------
  // Per k-step: the weights of the next k-step and the corners of the next k-step are requested
  // before this k-step's MFMAs; the corners are blended as soon as they arrive (A fragments of one
  // k-step ahead).  Weights alternate between two register sets; the next half-chunk's region is
  // requested after the last weight load of this half-chunk (k-step 4's, issued at k-step 3).
  const int nh = ceil_div(a.cin, 16);
  const int rw32 = rw * 32;
  const unsigned lds_base = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)s_u;
  frag bwa[NBF], bwb[NBF];
  ld_w(0, 0, bwa);
  for (int h = 0; h < nh; ++h) {
    // the records are loop-invariant: keep the compiler from hoisting values derived from them
    // (splat weights, corner addresses) for all ten records out of the loop
#pragma unroll
    for (int j = 0; j < 5; ++j)
#pragma unroll
      for (int m = 0; m < 2; ++m) asm volatile("" : "+v"(r_a[j][m]), "+v"(r_w01[j][m]), "+v"(r_w23[j][m]));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's share of region h has landed
    __syncthreads();  // everyone's share landed; everyone is done with region h - 1 (buffer of h + 1)
    // Corner reads are issued as inline ds_read_b128 with an explicit lgkmcnt wait tied to their
    // registers (wait_c).  Plain loads would make the compiler wait for the region prefetch in
    // flight (it cannot tell that those LDS writes go to the other buffer); the barrier above
    // orders them after this buffer's writes.
    const unsigned rb = lds_base + (unsigned)((h & 1) * D2_RBUF + 16 * (grp & 1));
    auto ld_c = [&](int j, frag (&c)[2][4]) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const unsigned ia = r_a[j][m];
        const unsigned p0 = rb + (ia & 0xffffu), dx = (ia >> 11) & 32u;
        const unsigned p2 = p0 + ((ia & (1u << 17)) ? (unsigned)rw32 : 0u);
        asm volatile("ds_read_b128 %0, %1" : "=v"(c[m][0]) : "v"(p0));
        asm volatile("ds_read_b128 %0, %1" : "=v"(c[m][1]) : "v"(p0 + dx));
        asm volatile("ds_read_b128 %0, %1" : "=v"(c[m][2]) : "v"(p2));
        asm volatile("ds_read_b128 %0, %1" : "=v"(c[m][3]) : "v"(p2 + dx));
      }
    };
    auto wait_c = [&](frag (&c)[2][4]) {
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(c[0][0]), "+v"(c[0][1]), "+v"(c[0][2]), "+v"(c[0][3]), "+v"(c[1][0]), "+v"(c[1][1]),
                     "+v"(c[1][2]), "+v"(c[1][3]));
    };
    auto blend = [&](int j, const frag (&c)[2][4], frag (&af)[2]) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        Info16 in;
        in.o01 = in.o23 = 0u;
        in.w01 = r_w01[j][m];
        in.w23 = r_w23[j][m];
        af[m] = Ops::blend(c[m][0], c[m][1], c[m][2], c[m][3], in);
      }
    };
    auto mma = [&](const frag (&af)[2], const frag (&bw)[NBF]) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int f = 0; f < NBF; ++f) acc[m][f] = Ops::mma(af[m], bw[f], acc[m][f]);
    };
    const bool more = h + 1 < nh;
    frag raw[2][4], af0[2], af1[2];
    ld_c(0, raw);
    wait_c(raw);
    blend(0, raw, af0);
    ld_w(h, 1, bwb);
    ld_c(1, raw);
    mma(af0, bwa);  // k-step 0
    wait_c(raw);
    blend(1, raw, af1);
    ld_w(h, 2, bwa);
    ld_c(2, raw);
    mma(af1, bwb);  // k-step 1
    wait_c(raw);
    blend(2, raw, af0);
    ld_w(h, 3, bwb);
    ld_c(3, raw);
    mma(af0, bwa);  // k-step 2
    wait_c(raw);
    blend(3, raw, af1);
    ld_w(h, 4, bwa);
    if (more) stage(h + 1);  // after the half-chunk's last weight load
    ld_c(4, raw);
    mma(af1, bwb);  // k-step 3
    wait_c(raw);
    blend(4, raw, af0);
    if (more) ld_w(h + 1, 0, bwb);
    mma(af0, bwa);  // k-step 4
#pragma unroll
    for (int f = 0; f < NBF; ++f) bwa[f] = bwb[f];
  }

  // ---- 4b. samples outside a capped region: straight from memory (rare) -------------------------------
  if (block_may_slow) {
    for (int h = 0; h < nh; ++h) {
      const int ch = 16 * h + 8 * (grp & 1);
      const bool ch_ok = ch < cin8;
#pragma unroll 1
      for (int j = 0; j < 5; ++j) {
        const int kt = 2 * j + (grp >> 1);
        frag af[2];
        bool any = false;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          af[m] = zero8<T>();
          if (kt < 9 && ch_ok) {
            const int qi = kt * D2_TILE + wave * 32 + m * 16 + row;
            const unsigned ia = s_ia[qi];
            if (ia & D2_SLOW) {
              const int cy0 = (int)((ia >> 14) & 0x7fffu), cx0 = (int)(ia & 0x3fffu);
              const int sx = (int)((ia >> 29) & 1u), sy = (int)((ia >> 30) & 1u);
              const uint2 wv = s_iw[qi];
              Info16 in;
              in.o01 = in.o23 = 0u;
              in.w01 = wv.x;
              in.w23 = wv.y;
              const T* g0 = xb + ((int64_t)cy0 * a.w + cx0) * a.x_cs + ch;
              af[m] = Ops::blend(ld8<T>(g0), ld8<T>(g0 + sx * a.x_cs), ld8<T>(g0 + (int64_t)sy * a.w * a.x_cs),
                                 ld8<T>(g0 + ((int64_t)sy * a.w + sx) * a.x_cs), in);
              any = true;
            }
          }
        }
        if (__builtin_amdgcn_ballot_w64(any) == 0) continue;
        frag bw[NBF];
        ld_w(h, j, bw);
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int f = 0; f < NBF; ++f) acc[m][f] = Ops::mma(af[m], bw[f], acc[m][f]);
      }
    }
  }

  // ---- 5. epilogue: values -> LDS tile -> row-contiguous stores; GAP partials ------------------------
  typedef T OutT;
  constexpr int SROW = NB + 16 / (int)sizeof(OutT);
  constexpr int STAGE_BYTES = D2_TILE * SROW * (int)sizeof(OutT);
  static_assert(STAGE_BYTES + D2_WAVES * NB * 4 <= SU, "epilogue tile must fit the shared area");
  OutT* ost = (OutT*)s_u;
  float(*gap_red)[NB] = (float(*)[NB])(s_u + STAGE_BYTES);
  if (tid < NB) {  // v = acc * mul + (bias * mul + add)
    s_par[0][tid] = par[0] * par[1] + par[2];
    s_par[1][tid] = par[1];
    s_par[2][tid] = par[3];
  }
  __syncthreads();  // every wave is done reading the region; s_par staged
  bool pix_ok[2][4];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pl = wave * 32 + m * 16 + grp * 4 + i;
      const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
      pix_ok[m][i] = pl < npx && ty0 + oyl < g.ho && tx0 + pl - oyl * g.tw < g.wo;
    }
  float gsum[NBF];
  auto epilogue = [&](auto act) {  // activation as a template argument, as in dcn_block
    constexpr int ACT = decltype(act)::value;
#pragma unroll
    for (int f = 0; f < NBF; ++f) {
      gsum[f] = 0.f;
      const int col = f * 16 + row;
      const bool co_ok = co0 + col < a.cout;
      const float shift = s_par[0][col], mul = s_par[1][col], scl = s_par[2][col];
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int pl = wave * 32 + m * 16 + grp * 4 + i;
          float v = fmaf(acc[m][f][i], mul, shift);
          if constexpr (ACT == KAD_ACT_SILU) v = v * sigmoidf_(v);
          else if constexpr (ACT == KAD_ACT_RELU) v = fmaxf(v, 0.f);
          v *= scl;
          const OutT o = from_f32<OutT>(v);
          ost[pl * SROW + col] = o;
          if (co_ok && pix_ok[m][i]) gsum[f] += to_f32(o);
        }
    }
  };
  if (a.relu == KAD_ACT_SILU) epilogue(std::integral_constant<int, KAD_ACT_SILU>{});
  else if (a.relu) epilogue(std::integral_constant<int, KAD_ACT_RELU>{});
  else epilogue(std::integral_constant<int, KAD_ACT_NONE>{});
  if (a.gap_partial) {
#pragma unroll
    for (int f = 0; f < NBF; ++f) {
      const float v = sum_xor32(sum_xor16(gsum[f]));
      if (grp == 0) gap_red[wave][f * 16 + row] = v;
    }
  }
  __syncthreads();
  OutT* out = (OutT*)a.out;
  constexpr int VEC = 16 / (int)sizeof(OutT);
  const bool vec_ok = a.out_layout == KAD_NHWC && (a.out_cs * (int)sizeof(OutT)) % 16 == 0 &&
                      ((uintptr_t)a.out & 15) == 0;
  if (vec_ok) {
    constexpr int VPP = NB / VEC;
    for (int j = tid; j < D2_TILE * VPP; j += D2_THREADS) {
      const int pl = j / VPP, v = j - pl * VPP;
      const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
      const int oy = ty0 + oyl, ox = tx0 + pl - oyl * g.tw;
      const int co = co0 + v * VEC;
      if (pl >= npx || oy >= g.ho || ox >= g.wo || co >= a.cout) continue;
      const OutT* src = ost + pl * SROW + v * VEC;
      OutT* dst = out + ((int64_t)n * P + (int64_t)oy * g.wo + ox) * a.out_cs + co;
      if (co + VEC <= a.cout) {
        *(intx4*)dst = *(const intx4*)src;
      } else {
        for (int e = 0; e < a.cout - co; ++e) dst[e] = src[e];
      }
    }
  } else if (a.out_layout == KAD_NHWC) {
    for (int j = tid; j < D2_TILE * NB; j += D2_THREADS) {
      const int pl = j / NB, col = j - pl * NB;
      const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
      const int oy = ty0 + oyl, ox = tx0 + pl - oyl * g.tw;
      const int co = co0 + col;
      if (pl >= npx || oy >= g.ho || ox >= g.wo || co >= a.cout) continue;
      out[((int64_t)n * P + (int64_t)oy * g.wo + ox) * a.out_cs + co] = ost[pl * SROW + col];
    }
  } else {  // NCHW: consecutive lanes along the tile's pixels; a thread keeps its pixel
    constexpr int CSTEP = D2_THREADS / D2_TILE;
    const int pl = tid % D2_TILE, col0 = tid / D2_TILE;
    const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
    const int oy = ty0 + oyl, ox = tx0 + pl - oyl * g.tw;
    if (pl < npx && oy < g.ho && ox < g.wo) {
      OutT* dst = out + ((int64_t)n * a.out_cs + co0 + col0) * P + (int64_t)oy * g.wo + ox;
      const OutT* src = ost + pl * SROW + col0;
      const int ncol = a.cout - co0 < NB ? a.cout - co0 : NB;
#pragma unroll 4
      for (int col = col0; col < ncol; col += CSTEP) {
        *dst = *src;
        dst += (int64_t)CSTEP * P;
        src += CSTEP;
      }
    }
  }
  if (a.gap_partial && tid < NB) {
    const int co = co0 + tid;
    if (co < a.cout) {
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < D2_WAVES; ++i) v += gap_red[i][tid];
      float* dst = a.gap_partial + ((int64_t)n * g.tiles + tile) * a.cout + co;
      if (a.se_att)
        rmw_store(dst, v);  // read by another block of this launch (fused SE)
      else
        *dst = v;
    }
  }

  // ---- 6. fused squeeze-excitation: the image's last block runs the MLP (protocol at se_tail) ----------
  if (a.se_att && a.gap_partial) {
    __shared__ int s_last;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (tid == 0) {
      const unsigned total = (unsigned)g.tiles * ny;
      const unsigned prev = __hip_atomic_fetch_add(a.se_count + n, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev + 1u == total;
      if (last) {
        const unsigned z = __hip_atomic_exchange(a.se_count + n, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(z));
      }
      s_last = last;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (s_last)
      se_tail<D2_THREADS>(a.gap_partial, a.se_w1, a.se_b1, a.se_w2, a.se_b2, a.se_att, a.se_inv_count, a.cout,
                          a.se_hid, n, g.tiles, (float*)s_u);
  }
}

template <typename T, int NBF, int MODE, int NRB>
__global__ __launch_bounds__(D2_THREADS, 2) void dsc2_kernel(kad_dcn_args a, DcnGeom g) {
  dsc2_block<T, NBF, MODE, NRB>(a, g, blockIdx.x, blockIdx.y, gridDim.y);
}

template <typename T, int NBF, int NRB>
__global__ __launch_bounds__(D2_THREADS, 2) void dsc2_group_kernel(DcnGroup grp) {
  const int id = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < KAD_DCN_GROUP_MAX; ++i)
    if (i < grp.count && id >= grp.start[i]) p = i;
  if (id >= grp.start[p + 1]) return;
  const int local = id - grp.start[p];
  const int gx = grp.g[p].grid_x;
  dsc2_block<T, NBF, MODE_FUSED, NRB>(grp.a[p], grp.g[p], local % gx, local / gx, grp.ny[p]);
}

// ---- weight packing ------------------------------------------------------------------------------
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

static DcnGeom make_geom(const kad_dcn_args& a, int ho, int wo) {
  DcnGeom g;
  g.ho = ho;
  g.wo = wo;
  pick_tile(ho, wo, &g.th, &g.tw);
  g.tiles_x = ceil_div(wo, g.tw);
  g.tiles = ceil_div(ho, g.th) * g.tiles_x;
  g.grid_x = round_up(a.n * g.tiles, 8);  // flattened (image, tile), padded to whole XCD rounds
  g.nchunk = ceil_div(a.cin, 32);
  g.cout_pad = round_up(a.cout, 16);
  g.fh = (g.th - 1) * a.stride + 3;
  g.fw = (g.tw - 1) * a.stride + 3;
  g.inv_tw = 1.f / (float)g.tw;
  g.inv_fw = 1.f / (float)g.fw;
  return g;
}

template <typename T, typename OutT, int NBF, int MODE>
static int launch_dcn(const kad_dcn_args& a, hipStream_t st, const DcnGeom& g) {
  dim3 grid(g.grid_x, ceil_div(a.cout, NBF * 16), 1);
  hipLaunchKernelGGL((dcn_fwd_kernel<T, OutT, NBF, MODE>), grid, dim3(DCN_THREADS), 0, st, a, g);
  return check_launch(MODE == MODE_PLAIN ? "kad_conv3x3_fwd" : MODE == MODE_FUSED ? "kad_dsc_fwd" : "kad_dcn_fwd");
}

template <typename T, typename OutT, int MODE>
static int dispatch_dcn(const kad_dcn_args& a, hipStream_t st, const DcnGeom& g) {
  const int nbf = ceil_div(a.cout, 16);
  switch (nbf < 8 ? nbf : 8) {
    case 1: return launch_dcn<T, OutT, 1, MODE>(a, st, g);
    case 2: return launch_dcn<T, OutT, 2, MODE>(a, st, g);
    case 3: return launch_dcn<T, OutT, 3, MODE>(a, st, g);
    case 4: return launch_dcn<T, OutT, 4, MODE>(a, st, g);
    case 5: return launch_dcn<T, OutT, 5, MODE>(a, st, g);
    case 6: return launch_dcn<T, OutT, 6, MODE>(a, st, g);
    case 7: return launch_dcn<T, OutT, 7, MODE>(a, st, g);
    default: return launch_dcn<T, OutT, 8, MODE>(a, st, g);
  }
}

static int validate_dcn(const kad_dcn_args* a, int mode, DcnGeom* g_out) {
  KAD_CHECK_ARG(a, "null args");
  KAD_CHECK_ARG(a->x && a->wpack && a->out, "null tensor pointer");
  KAD_CHECK_ARG(mode != MODE_EXT || a->offset, "null offset pointer");
  KAD_CHECK_ARG(mode != MODE_FUSED || a->off_wpack, "null off_wpack pointer");
  KAD_CHECK_ARG(a->n > 0 && a->cin > 0 && a->cout > 0 && a->h > 0 && a->w > 0,
                "bad shape n=%d cin=%d cout=%d h=%d w=%d", a->n, a->cin, a->cout, a->h, a->w);
  KAD_CHECK_ARG(a->h < 32768 && a->w < 16384, "image %dx%d too large (H < 32768, W < 16384)", a->h, a->w);
  KAD_CHECK_ARG((int64_t)a->h * a->w * a->x_cs * dtype_size(a->dtype) < ((int64_t)1 << 31) &&
                    (int64_t)round_up(a->cout, 16) * ceil_div(a->cin, 32) * 288 * dtype_size(a->dtype) < ((int64_t)1 << 31),
                "one image (or the packed weights) exceeds 2 GB");
  KAD_CHECK_ARG(a->stride >= 1 && a->pad >= 0, "bad stride=%d pad=%d", a->stride, a->pad);
  KAD_CHECK_ARG(a->x_cs % 8 == 0 && a->x_cs >= round_up(a->cin, 8),
                "x channel stride %d must be a multiple of 8 and >= roundup(cin=%d, 8)", a->x_cs, a->cin);
  KAD_CHECK_ARG((a->out_layout == KAD_NCHW || a->out_layout == KAD_NHWC) && a->out_cs >= a->cout,
                "bad output layout %d / channel stride %d", a->out_layout, a->out_cs);
  const int ho = (a->h + 2 * a->pad - 3) / a->stride + 1;
  const int wo = (a->w + 2 * a->pad - 3) / a->stride + 1;
  KAD_CHECK_ARG(ho > 0 && wo > 0, "empty output");
  if (a->se_att) {
    KAD_CHECK_ARG(mode != MODE_PLAIN, "the fused squeeze-excitation needs a DCN / DSC output");
    KAD_CHECK_ARG(a->gap_partial && a->se_w1 && a->se_w2 && a->se_count && a->se_hid > 0,
                  "fused squeeze-excitation: gap_partial, se_w1, se_w2, se_count and se_hid > 0 are required");
    KAD_CHECK_ARG((a->cout + a->se_hid + DCN_THREADS) * 4 <= DCN_SE_LDS,
                  "fused squeeze-excitation: Cout + hidden = %d exceeds %d", a->cout + a->se_hid,
                  DCN_SE_LDS / 4 - DCN_THREADS);
  }
  const uintptr_t align = (uintptr_t)a->x | (uintptr_t)a->wpack | (uintptr_t)a->off_wpack;
  KAD_CHECK_ARG(align % 16 == 0, "x and packed weights must be 16-byte aligned");
  KAD_CHECK_ARG((int64_t)a->n * ceil_div(ho, 1) * wo < (1ll << 30), "kad_dcn: N x output pixels too large");
  *g_out = make_geom(*a, ho, wo);
  if (mode != MODE_EXT)
    KAD_CHECK_ARG(g_out->fh * g_out->fw <= DCN_FCAP, "stride %d not supported here (3x3 footprint of a tile %dx%d > %d px)",
                  a->stride, g_out->fh, g_out->fw, DCN_FCAP);
  return KAD_OK;
}

}  // namespace kad

using namespace kad;

namespace kad {
// The two-blocks-per-CU kernel: 16-bit, stride 1, at most D2_COUT_MAX output channels (one column
// block), and enough blocks (>= D2_MIN_BLOCKS over all problems of a launch) for two to share a
// CU.  Measured per launch on KAD-CNet-S (bs16, 800^2, fp16): 1680 blocks of Cout <= 16: 90 ->
// 59 us; 432 blocks: 33 -> 22 us; but 128 blocks of Cout 32: 19.8 -> 21.7 us (one 4-wave block
// per CU), and the KAD-Conv(256) branches (Cout 86 at 100^2 / 50^2 / 25^2: 640 / 160 / 40
// blocks) 87 / 32 / 31 -> 89 / 44 / 44 us.  Everything else runs on dcn_fwd_kernel.
constexpr int D2_COUT_MAX = 16 * D2_NBF_MAX;
constexpr int64_t D2_MIN_BLOCKS = 384;
static bool d2_shape_ok(const kad_dcn_args& a) {
  return (a.dtype == KAD_F16 || a.dtype == KAD_BF16) && a.stride == 1 && a.cout <= D2_COUT_MAX;
}
static bool d2_ok(const kad_dcn_args& a, const DcnGeom& g) {
  return d2_shape_ok(a) && (int64_t)a.n * g.tiles >= D2_MIN_BLOCKS;
}
// One region buffer (NRB = 1): a single 16-channel half-chunk, and the conv_offset staging of one
// 32-channel chunk (footprint and filters, 5 slots per row) and the SE scratch within D2_RBUF.
static bool d2_single(const kad_dcn_args& a, const DcnGeom& g) {
  const int fpix = g.fh * g.fw;
  return a.cin <= 16 && (ceil_div(fpix * 5, 64) + ceil_div(9 * DCN_NOFF * 5, 64)) * 1024 <= D2_RBUF &&
         (a.cout + a.se_hid + D2_THREADS) * 4 <= D2_RBUF;
}

template <typename T, int NBF, int MODE>
static int launch_d2(const kad_dcn_args& a, hipStream_t st, const DcnGeom& g) {
  if (d2_single(a, g))
    hipLaunchKernelGGL((dsc2_kernel<T, NBF, MODE, 1>), dim3(g.grid_x, 1, 1), dim3(D2_THREADS), 0, st, a, g);
  else
    hipLaunchKernelGGL((dsc2_kernel<T, NBF, MODE, 2>), dim3(g.grid_x, 1, 1), dim3(D2_THREADS), 0, st, a, g);
  return check_launch(MODE == MODE_FUSED ? "kad_dsc_fwd" : "kad_dcn_fwd");
}

template <typename T, int MODE>
static int dispatch_d2(const kad_dcn_args& a, hipStream_t st, const DcnGeom& g) {
  switch (ceil_div(a.cout, 16)) {
    case 1: return launch_d2<T, 1, MODE>(a, st, g);
    case 2: return launch_d2<T, 2, MODE>(a, st, g);
    case 3: return launch_d2<T, 3, MODE>(a, st, g);
    default: return launch_d2<T, 4, MODE>(a, st, g);
  }
}

template <int MODE>
static int dispatch_d2_dtype(const kad_dcn_args& a, hipStream_t st, const DcnGeom& g) {
  return a.dtype == KAD_F16 ? dispatch_d2<half_t, MODE>(a, st, g) : dispatch_d2<bf16_t, MODE>(a, st, g);
}

template <typename T, int NBF>
static int launch_group_d2(const DcnGroup& grp, hipStream_t st) {
  bool single = true;
  for (int p = 0; p < grp.count; ++p) single = single && d2_single(grp.a[p], grp.g[p]);
  if (single)
    hipLaunchKernelGGL((dsc2_group_kernel<T, NBF, 1>), dim3(grp.start[grp.count]), dim3(D2_THREADS), 0, st, grp);
  else
    hipLaunchKernelGGL((dsc2_group_kernel<T, NBF, 2>), dim3(grp.start[grp.count]), dim3(D2_THREADS), 0, st, grp);
  return check_launch("kad_dsc_fwd_group");
}

template <typename T>
static int dispatch_group_d2(const DcnGroup& grp, int nbf, hipStream_t st) {
  switch (nbf) {
    case 1: return launch_group_d2<T, 1>(grp, st);
    case 2: return launch_group_d2<T, 2>(grp, st);
    case 3: return launch_group_d2<T, 3>(grp, st);
    default: return launch_group_d2<T, 4>(grp, st);
  }
}
}  // namespace kad

extern "C" int64_t kad_dcn_wpack_elems(int cin, int cout) {
  if (cin <= 0 || cout <= 0) return 0;
  return (int64_t)round_up(cout, 16) * ceil_div(cin, 32) * 9 * 32;
}

extern "C" int kad_dcn_tiles(int ho, int wo) {
  if (ho <= 0 || wo <= 0) return 0;
  int th, tw;
  pick_tile(ho, wo, &th, &tw);
  return ceil_div(ho, th) * ceil_div(wo, tw);
}

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

extern "C" int kad_conv3x3_fwd(const kad_dcn_args* a, void* stream) {
  DcnGeom g;
  int rc = validate_dcn(a, MODE_PLAIN, &g);
  if (rc) return fail(rc, "kad_conv3x3_fwd: %s", kad_last_error());
  hipStream_t st = (hipStream_t)stream;
  switch (a->dtype) {
    case KAD_F32: return dispatch_dcn<float, float, MODE_PLAIN>(*a, st, g);
    case KAD_F16: return dispatch_dcn<half_t, float, MODE_PLAIN>(*a, st, g);
    case KAD_BF16: return dispatch_dcn<bf16_t, float, MODE_PLAIN>(*a, st, g);
    default: return fail(KAD_EINVAL, "kad_conv3x3_fwd: unknown dtype %d", a->dtype);
  }
}

extern "C" int kad_conv_fwd(const kad_dcn_args* a, void* stream) {
  DcnGeom g;
  int rc = validate_dcn(a, MODE_PLAIN, &g);
  if (rc) return fail(rc, "kad_conv_fwd: %s", kad_last_error());
  KAD_CHECK_ARG(a->relu >= KAD_ACT_NONE && a->relu <= KAD_ACT_SILU, "kad_conv_fwd: unknown activation %d", a->relu);
  hipStream_t st = (hipStream_t)stream;
  rc = convolution_igemm(*a, g.ho, g.wo, st);  // 16-bit, NHWC output: implicit-GEMM kernel
  if (rc != 1) return rc;
  switch (a->dtype) {
    case KAD_F32: return dispatch_dcn<float, float, MODE_PLAIN>(*a, st, g);
    case KAD_F16: return dispatch_dcn<half_t, half_t, MODE_PLAIN>(*a, st, g);
    case KAD_BF16: return dispatch_dcn<bf16_t, bf16_t, MODE_PLAIN>(*a, st, g);
    default: return fail(KAD_EINVAL, "kad_conv_fwd: unknown dtype %d", a->dtype);
  }
}

extern "C" int kad_dcn_fwd(const kad_dcn_args* a, void* stream) {
  DcnGeom g;
  int rc = validate_dcn(a, MODE_EXT, &g);
  if (rc) return fail(rc, "kad_dcn_fwd: %s", kad_last_error());
  hipStream_t st = (hipStream_t)stream;
  if (d2_ok(*a, g)) return dispatch_d2_dtype<MODE_EXT>(*a, st, g);
  switch (a->dtype) {
    case KAD_F32: return dispatch_dcn<float, float, MODE_EXT>(*a, st, g);
    case KAD_F16: return dispatch_dcn<half_t, half_t, MODE_EXT>(*a, st, g);
    case KAD_BF16: return dispatch_dcn<bf16_t, bf16_t, MODE_EXT>(*a, st, g);
    default: return fail(KAD_EINVAL, "kad_dcn_fwd: unknown dtype %d", a->dtype);
  }
}

extern "C" int kad_dsc_fwd(const kad_dcn_args* a, void* stream) {
  DcnGeom g;
  int rc = validate_dcn(a, MODE_FUSED, &g);
  if (rc) return fail(rc, "kad_dsc_fwd: %s", kad_last_error());
  hipStream_t st = (hipStream_t)stream;
  if (d2_ok(*a, g)) return dispatch_d2_dtype<MODE_FUSED>(*a, st, g);
  switch (a->dtype) {
    case KAD_F32: return dispatch_dcn<float, float, MODE_FUSED>(*a, st, g);
    case KAD_F16: return dispatch_dcn<half_t, half_t, MODE_FUSED>(*a, st, g);
    case KAD_BF16: return dispatch_dcn<bf16_t, bf16_t, MODE_FUSED>(*a, st, g);
    default: return fail(KAD_EINVAL, "kad_dsc_fwd: unknown dtype %d", a->dtype);
  }
}

namespace kad {
template <typename T, typename OutT, int NBF>
static int launch_group(const DcnGroup& grp, hipStream_t st) {
  hipLaunchKernelGGL((dcn_group_kernel<T, OutT, NBF, MODE_FUSED>), dim3(grp.start[grp.count]), dim3(DCN_THREADS), 0,
                     st, grp);
  return check_launch("kad_dsc_fwd_group");
}

template <typename T, typename OutT>
static int dispatch_group(const DcnGroup& grp, int nbf, hipStream_t st) {
  switch (nbf) {
    case 1: return launch_group<T, OutT, 1>(grp, st);
    case 2: return launch_group<T, OutT, 2>(grp, st);
    case 3: return launch_group<T, OutT, 3>(grp, st);
    case 4: return launch_group<T, OutT, 4>(grp, st);
    case 5: return launch_group<T, OutT, 5>(grp, st);
    case 6: return launch_group<T, OutT, 6>(grp, st);
    case 7: return launch_group<T, OutT, 7>(grp, st);
    default: return launch_group<T, OutT, 8>(grp, st);
  }
}
}  // namespace kad

extern "C" int kad_dsc_fwd_group(const kad_dcn_args* a, int count, void* stream) {
  KAD_CHECK_ARG(a && count >= 1 && count <= KAD_DCN_GROUP_MAX, "kad_dsc_fwd_group: count %d outside [1, %d]", count,
                KAD_DCN_GROUP_MAX);
  DcnGroup grp;
  grp.count = count;
  int nbf = 0;
  int64_t blocks = 0;
  for (int p = 0; p < count; ++p) {
    int rc = validate_dcn(&a[p], MODE_FUSED, &grp.g[p]);
    if (rc) return fail(rc, "kad_dsc_fwd_group: problem %d: %s", p, kad_last_error());
    const int nb = ceil_div(a[p].cout, 16) < 8 ? ceil_div(a[p].cout, 16) : 8;
    KAD_CHECK_ARG(a[p].dtype == a[0].dtype && (p == 0 || nb == nbf),
                  "kad_dsc_fwd_group: problem %d differs in dtype or ceil(Cout / 16) from problem 0", p);
    nbf = nb;
    grp.a[p] = a[p];
    grp.ny[p] = ceil_div(a[p].cout, nb * 16);
    grp.start[p] = (int)blocks;
    blocks += (int64_t)grp.g[p].grid_x * grp.ny[p];  // grid_x is a multiple of 8
  }
  KAD_CHECK_ARG(blocks < (1ll << 31), "kad_dsc_fwd_group: too many blocks");
  grp.start[count] = (int)blocks;
  for (int p = count + 1; p <= KAD_DCN_GROUP_MAX; ++p) grp.start[p] = (int)blocks;
  hipStream_t st = (hipStream_t)stream;
  bool all_d2 = blocks >= D2_MIN_BLOCKS;
  for (int p = 0; p < count; ++p) all_d2 = all_d2 && d2_shape_ok(a[p]);
  if (all_d2) {
    if (a[0].dtype == KAD_F16) return dispatch_group_d2<half_t>(grp, nbf, st);
    return dispatch_group_d2<bf16_t>(grp, nbf, st);
  }
  switch (a[0].dtype) {
    case KAD_F32: return dispatch_group<float, float>(grp, nbf, st);
    case KAD_F16: return dispatch_group<half_t, half_t>(grp, nbf, st);
    case KAD_BF16: return dispatch_group<bf16_t, bf16_t>(grp, nbf, st);
    default: return fail(KAD_EINVAL, "kad_dsc_fwd_group: unknown dtype %d", a[0].dtype);
  }
}

// ---- kad_dsc_fwd without caller-owned scratch -------------------------------------------------------
// The fused squeeze-excitation needs two buffers beyond the inputs and outputs: the per-tile GAP
// partials and the per-image arrival counters.  kad_dsc_fwd_noalloc takes both from `scratch`, a
// file-scope device array of fixed size, so a caller that cannot allocate passes only inputs and
// outputs.  Layout: [0, 16 KB) counters (unsigned, one per image; zero when the code object is
// loaded, as static storage is, and left zero by every call that completes), then the partials.
// The host-side name `scratch` is not a device address: each device's copy is found once with
// hipGetSymbolAddress and only that pointer is handed to kernels.  Every call on a device shares
// that device's array, so calls that overlap on one GPU race.
namespace kad {
constexpr int NOALLOC_MAX_IMAGES = 4096;
constexpr int64_t NOALLOC_MAX_PARTIALS = (int64_t)1 << 20;  // floats: N * tiles * Cout
constexpr size_t NOALLOC_COUNT_BYTES = (size_t)NOALLOC_MAX_IMAGES * 4;
static __device__ __align__(256) unsigned char scratch[NOALLOC_COUNT_BYTES + NOALLOC_MAX_PARTIALS * 4];

constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// This device's address of `scratch`, looked up on the first call per device (current device).
static int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(KAD_ELAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return fail(KAD_EUNSUPPORTED, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(KAD_ELAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KAD_OK;
}
}  // namespace kad

extern "C" int kad_dsc_fwd_noalloc(const kad_dcn_args* a_in, void* stream) {
  KAD_CHECK_ARG(a_in, "kad_dsc_fwd_noalloc: null args");
  KAD_CHECK_ARG(!a_in->gap_partial && !a_in->se_count,
                "kad_dsc_fwd_noalloc: gap_partial and se_count come from the library's scratch; pass NULL");
  kad_dcn_args a = *a_in;
  if (a.se_att) {
    KAD_CHECK_ARG(a.n > 0 && a.h > 0 && a.w > 0 && a.cout > 0 && a.stride >= 1 && a.pad >= 0,
                  "kad_dsc_fwd_noalloc: bad shape n=%d h=%d w=%d cout=%d stride=%d pad=%d", a.n, a.h, a.w, a.cout,
                  a.stride, a.pad);
    const int ho = (a.h + 2 * a.pad - 3) / a.stride + 1, wo = (a.w + 2 * a.pad - 3) / a.stride + 1;
    KAD_CHECK_ARG(ho > 0 && wo > 0, "kad_dsc_fwd_noalloc: empty output");
    const int64_t need = (int64_t)a.n * kad_dcn_tiles(ho, wo) * a.cout;
    KAD_CHECK_ARG(a.n <= NOALLOC_MAX_IMAGES && need <= NOALLOC_MAX_PARTIALS,
                  "kad_dsc_fwd_noalloc: N=%d images and %lld GAP partials exceed the scratch limits (%d images, "
                  "%lld partials = N x tiles x Cout)", a.n, (long long)need, NOALLOC_MAX_IMAGES,
                  (long long)NOALLOC_MAX_PARTIALS);
    void* p = nullptr;
    const int rc = scratch_ptr(&p);
    if (rc) return rc;
    a.se_count = (unsigned*)p;
    a.gap_partial = (float*)((char*)p + NOALLOC_COUNT_BYTES);
  }
  return kad_dsc_fwd(&a, stream);
}
