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
//
// Block = 256 threads (4 waves) x one output tile of up to 128 pixels (TH x TW,
// chosen per image size to waste few lanes) x 16 * NBF output channels.
//  1. Prologue: every (pixel, tap) sample position is computed once; its
//     clamped top-left corner, corner steps and weights (bilinear x mask, 0 for
//     out-of-image corners) go to LDS, and the block reduces the bounding box
//     of all live corners.
//  2. The input region = that bounding box (capped at RCAP pixels around the
//     tile; typical offsets fit).  Each sample's region-relative corner address
//     and weights (fp16 except on the fp32 path) are stored in LDS once.
//     Samples whose corners fall outside a capped region are flagged and read
//     straight from global memory by a rarely taken branch.
//  3. Per 32-channel chunk: the region slice [pixels][32 ch] is staged in LDS
//     (16-byte loads along channels of the NHWC input); then for each of the 9
//     taps, each lane builds its MFMA A fragment (8 channels of one (pixel, tap))
//     from four 16-byte LDS corner reads blended with packed fp16 FMAs, and the
//     wave issues 2 x NBF v_mfma_f32_16x16x32 against B fragments (packed
//     weights, 16 bytes per lane from global/L2, prefetched one tap ahead).
//  4. Epilogue: bias, BN scale/shift, ReLU, branch scale, store, GAP partials.
// Blocks are mapped so that each XCD (and its L2) gets a contiguous band of
// tiles: neighbouring tiles share their halos through that L2.
//
// Any consistent assignment of k to (lane group, slot) gives the same dot
// product, so A and B only have to agree with each other; the accumulator
// layout (lane -> column lane & 15, rows 4 * (lane >> 4) + i) is the MFMA
// output layout.
#include "kad_common.h"

namespace kad {

constexpr int DCN_THREADS = 256;
constexpr int DCN_WM = 2;                          // 16-pixel A fragments per wave
constexpr int DCN_TILE = 4 * DCN_WM * 16;          // 128 pixels per block
constexpr int DCN_NPAIR = 9 * DCN_TILE;            // (tap, pixel) samples per block

template <typename T> struct DcnCfg {              // fp16 / bf16
  static constexpr int pxs = 40;                   // halves per region pixel (32 + 8 pad)
  static constexpr int rcap = 736;                 // region pixels (57.5 KB; + 13.5 KB sample info)
};
template <> struct DcnCfg<float> {
  static constexpr int pxs = 36;                   // floats per region pixel (32 + 4 pad)
  static constexpr int rcap = 320;                 // (45 KB; + 22.5 KB sample info)
};

struct DcnGeom {
  int ho, wo, th, tw, tiles_x, tiles, grid_x, nchunk, cout_pad;
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
// staged region (16 bits each) and the corner weights.  Samples that are dead
// (all weights 0) or outside a capped region get zero weights here; the latter
// are accumulated by a separate pass from global memory (s_slow).
struct __align__(16) Info16 { unsigned o01, o23; unsigned w01, w23; };  // weights as 2 x half2
struct __align__(16) Info32 { unsigned o01, o23, pad0, pad1; float w[4]; };

__device__ __forceinline__ unsigned pack_h2(float a, float b) {
  const half2_t h{(half_t)a, (half_t)b};
  return __builtin_bit_cast(unsigned, h);
}

template <typename T> struct InfoOf { typedef Info16 type; };
template <> struct InfoOf<float> { typedef Info32 type; };

template <typename T>
__device__ __forceinline__ typename InfoOf<T>::type make_info(unsigned o01, unsigned o23, const float* w) {
  typename InfoOf<T>::type r;
  r.o01 = o01;
  r.o23 = o23;
  if constexpr (sizeof(T) == 4) {
    r.pad0 = r.pad1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.w[i] = w[i];
  } else {
    r.w01 = pack_h2(w[0], w[1]);
    r.w23 = pack_h2(w[2], w[3]);
  }
  return r;
}

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

// ---- kernel ------------------------------------------------------------------------------------
// PLAIN = true computes an ordinary 3x3 convolution (integer taps, no offsets or
// mask): DSC's offset branch, conv_offset (kad_conv.py:55-56).
template <typename T, typename OutT, int NBF, bool PLAIN>
__global__ __launch_bounds__(DCN_THREADS, 2) void dcn_fwd_kernel(kad_dcn_args a, DcnGeom g) {
  typedef DcnFrag<T> Ops;
  typedef typename Ops::frag frag;
  typedef typename InfoOf<T>::type Info;
  constexpr int PXS = DcnCfg<T>::pxs;
  constexpr int RCAP = DcnCfg<T>::rcap;
  static_assert(RCAP * PXS * sizeof(T) >= DCN_NPAIR * 24, "prologue scratch must fit in the region buffer");
  // region [RCAP][PXS] T; during the prologue it holds the raw samples instead
  __shared__ __align__(16) T region[RCAP * PXS];
  __shared__ Info s_info[DCN_NPAIR];                 // [9][128] per-sample corner offsets + weights
  __shared__ unsigned char s_slow[DCN_NPAIR];        // [9][128] 1 = sample outside the capped region
  __shared__ int s_box[4];       // ymin, ymax, xmin, xmax (clamped corners of live samples)
  __shared__ int s_reg[5];       // region y0, x0, rows, cols, capped flag
  __shared__ float gap_red[4][NBF * 16];
  float4* raw_w = (float4*)region;                   // [9][128] corner weights
  int* raw_yx = (int*)(raw_w + DCN_NPAIR);           // [9][128] clamped top-left corner (y << 15 | x)
  int* raw_st = raw_yx + DCN_NPAIR;                  // [9][128] corner steps (dy << 1 | dx)

  // XCD-aware tile order: block b runs on XCD b % 8; give each XCD a contiguous band.
  const int bx = blockIdx.x;
  const int tile = (bx & 7) * (g.grid_x >> 3) + (bx >> 3);
  if (tile >= g.tiles) return;  // whole block, before any barrier
  const int co0 = blockIdx.y * NBF * 16;
  const int n = blockIdx.z;
  const int tyi = tile / g.tiles_x;
  const int ty0 = tyi * g.th, tx0 = (tile - tyi * g.tiles_x) * g.tw;
  const int P = g.ho * g.wo;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = lane & 15, grp = lane >> 4;

  if (tid == 0) {
    s_box[0] = 0x7fffffff;
    s_box[1] = -1;
    s_box[2] = 0x7fffffff;
    s_box[3] = -1;
  }
  __syncthreads();
  // ---- 1. samples: clamped corners, weights, bounding box ------------------------------------------
  int bymin = 0x7fffffff, bymax = -1, bxmin = 0x7fffffff, bxmax = -1;
  // offsets and mask of this thread's samples, all loads issued before any use
  constexpr int PPT = (DCN_NPAIR + DCN_THREADS - 1) / DCN_THREADS;
  float pre_dy[PPT], pre_dx[PPT], pre_m[PPT];
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int q = tid + u * DCN_THREADS;
    pre_dy[u] = pre_dx[u] = 0.f;
    pre_m[u] = 1.f;
    if (!PLAIN && q < DCN_NPAIR) {
      const int k = q / DCN_TILE, pl = q - k * DCN_TILE;
      const int oy = ty0 + pl / g.tw, ox = tx0 + pl - (pl / g.tw) * g.tw;
      if (pl < g.th * g.tw && oy < g.ho && ox < g.wo) {
        const int64_t p = oy * g.wo + ox;
        pre_dy[u] = a.offset[n * a.off_sn + p * a.off_sp + (2 * k) * a.off_sc];
        pre_dx[u] = a.offset[n * a.off_sn + p * a.off_sp + (2 * k + 1) * a.off_sc];
        if (a.mask) pre_m[u] = a.mask[n * a.mask_sn + p * a.mask_sp + k * a.mask_sc];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int q = tid + u * DCN_THREADS;
    if (q >= DCN_NPAIR) break;
    const int k = q / DCN_TILE, pl = q - k * DCN_TILE;
    const int oy = ty0 + pl / g.tw, ox = tx0 + pl - (pl / g.tw) * g.tw;
    float w[4] = {0.f, 0.f, 0.f, 0.f};
    int cy0 = 0, cx0 = 0, sy = 0, sx = 0;
    const bool live_px = pl < g.th * g.tw && oy < g.ho && ox < g.wo;
    const int ky = k / 3, kx = k - (k / 3) * 3;
    if (live_px && PLAIN) {
      const int iy = oy * a.stride - a.pad + ky, ix = ox * a.stride - a.pad + kx;
      if (iy >= 0 && iy < a.h && ix >= 0 && ix < a.w) {
        cy0 = iy;
        cx0 = ix;
        w[0] = 1.f;
      }
    } else if (live_px) {
      const float py = (float)(oy * a.stride - a.pad + ky) + pre_dy[u];
      const float px = (float)(ox * a.stride - a.pad + kx) + pre_dx[u];
      sample_geom(py, px, pre_m[u], a.h, a.w, cy0, cx0, sy, sx, w);
    }
    const bool live = w[0] != 0.f || w[1] != 0.f || w[2] != 0.f || w[3] != 0.f;
    if (live) {
      bymin = min(bymin, cy0);
      bymax = max(bymax, cy0 + sy);
      bxmin = min(bxmin, cx0);
      bxmax = max(bxmax, cx0 + sx);
    }
    raw_yx[q] = (cy0 << 15) | cx0;
    raw_w[q] = float4{w[0], w[1], w[2], w[3]};
    raw_st[q] = (sy << 1) | sx;
  }
  // wave-level then block-level bounding box (integer min / max: order-independent)
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    bymin = min(bymin, __shfl_xor(bymin, o));
    bymax = max(bymax, __shfl_xor(bymax, o));
    bxmin = min(bxmin, __shfl_xor(bxmin, o));
    bxmax = max(bxmax, __shfl_xor(bxmax, o));
  }
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
      const int fy0 = max(ty0 * a.stride - a.pad, 0), fy1 = min((ty0 + g.th - 1) * a.stride - a.pad + 2, a.h - 1);
      const int fx0 = max(tx0 * a.stride - a.pad, 0), fx1 = min((tx0 + g.tw - 1) * a.stride - a.pad + 2, a.w - 1);
      int m = 0;
      while (m < 4096) {
        const int y0n = max(ry0, fy0 - m - 1), y1n = min(ry1, fy1 + m + 1);
        const int x0n = max(rx0, fx0 - m - 1), x1n = min(rx1, fx1 + m + 1);
        if ((y1n - y0n + 1) * (x1n - x0n + 1) > RCAP) break;
        ++m;
      }
      const int y0n = max(ry0, fy0 - m), y1n = min(ry1, fy1 + m);
      const int x0n = max(rx0, fx0 - m), x1n = min(rx1, fx1 + m);
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
  // ---- 2. sample info: corner byte offsets in the region + weights; slow samples listed apart -------
  constexpr int PXB = PXS * (int)sizeof(T);          // bytes per region pixel
  for (int q = tid; q < DCN_NPAIR; q += DCN_THREADS) {
    const int yx = raw_yx[q], st = raw_st[q];
    const float4 wv = raw_w[q];
    float w[4] = {wv.x, wv.y, wv.z, wv.w};
    const int cy0 = yx >> 15, cx0 = yx & 0x7fff;
    const int sy = st >> 1, sx = st & 1;
    const int ly = cy0 - ry0, lx = cx0 - rx0;
    const bool dead = w[0] == 0.f && w[1] == 0.f && w[2] == 0.f && w[3] == 0.f;
    unsigned o01 = 0, o23 = 0;
    unsigned char slow = 0;
    if (!dead && ly >= 0 && ly + sy < rh && lx >= 0 && lx + sx < rw) {
      const unsigned b0 = (unsigned)((ly * rw + lx) * PXB);
      const unsigned bx = (unsigned)(sx * PXB), by = (unsigned)(sy * rw * PXB);
      o01 = b0 | ((b0 + bx) << 16);
      o23 = (b0 + by) | ((b0 + by + bx) << 16);
    } else if (!dead) {
      slow = 1;                         // the fast path skips it; the slow pass adds it
      w[0] = w[1] = w[2] = w[3] = 0.f;
    } else {
      w[0] = w[1] = w[2] = w[3] = 0.f;
    }
    s_info[q] = make_info<T>(o01, o23, w);
    s_slow[q] = slow;
  }

  const T* xb = (const T*)a.x + (int64_t)n * a.h * a.w * a.x_cs;
  const T* wp = (const T*)a.wpack;
  const int cin8 = round_up(a.cin, 8);

  floatx4 acc[DCN_WM][NBF];
#pragma unroll
  for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
    for (int b = 0; b < NBF; ++b) acc[m][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int rpix = rh * rw;
  const int step = DCN_THREADS / 4;
  const int ibase = wave * (16 * DCN_WM) + row;      // this lane's pixel slot within a tap row of s_info
  const T* wrow[NBF];                                // this lane's weight row (output channel) per fragment
#pragma unroll
  for (int b = 0; b < NBF; ++b) {
    const int co = co0 + b * 16 + row;
    wrow[b] = wp + (int64_t)(co < g.cout_pad ? co : 0) * g.nchunk * 9 * 32 + grp * 8;
  }
  for (int c = 0; c < g.nchunk; ++c) {
    __syncthreads();  // previous chunk (or the prologue's raw samples) fully consumed
    // ---- 3a. stage the region slice [rpix][32 ch], four 16-byte loads in flight per thread -------------
    {
      const int gq = tid & 3;
      const int chs = c * 32 + gq * 8;
      const bool chs_ok = chs < cin8;
      const float inv_rw = 1.f / (float)rw;
      for (int base = tid >> 2; base < rpix; base += 4 * step) {
        frag v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int q = base + u * step;
          v[u] = zero8<T>();
          if (q < rpix && chs_ok) {
            const int qy = (int)(((float)q + 0.5f) * inv_rw);
            const int qx = q - qy * rw;
            v[u] = ld8<T>(xb + ((int64_t)(ry0 + qy) * a.w + rx0 + qx) * a.x_cs + chs);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int q = base + u * step;
          if (q < rpix) {
            T* d = region + q * PXS + gq * 8;
            if constexpr (sizeof(T) == 4) {
              *(floatx4*)d = v[u].lo;
              *(floatx4*)(d + 4) = v[u].hi;
            } else {
              *(frag*)d = v[u];
            }
          }
        }
      }
    }
    __syncthreads();
    // ---- 3b. nine taps of this chunk: weights and sample records prefetched one tap ahead -----------
    const bool ch_ok = c * 32 + grp * 8 < cin8;
    frag bf[NBF], bn[NBF];
    Info ic[DCN_WM], inx[DCN_WM];
#pragma unroll
    for (int b = 0; b < NBF; ++b) bn[b] = ld8<T>(wrow[b] + (c * 9) * 32);
#pragma unroll
    for (int m = 0; m < DCN_WM; ++m) inx[m] = s_info[m * 16 + ibase];
#pragma unroll 1
    for (int k = 0; k < 9; ++k) {
#pragma unroll
      for (int b = 0; b < NBF; ++b) bf[b] = bn[b];
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m) ic[m] = inx[m];
      if (k < 8) {
#pragma unroll
        for (int b = 0; b < NBF; ++b) bn[b] = ld8<T>(wrow[b] + (c * 9 + k + 1) * 32);
#pragma unroll
        for (int m = 0; m < DCN_WM; ++m) inx[m] = s_info[(k + 1) * DCN_TILE + m * 16 + ibase];
      }
      frag af[DCN_WM];
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m) {
        const char* rb = (const char*)region + grp * 8 * (int)sizeof(T);
        if (PLAIN) {
          af[m] = Ops::blend(ld8<T>((const T*)(rb + (ic[m].o01 & 0xffffu))), zero8<T>(), zero8<T>(), zero8<T>(),
                             ic[m]);
        } else {
          const frag v0 = ld8<T>((const T*)(rb + (ic[m].o01 & 0xffffu)));
          const frag v1 = ld8<T>((const T*)(rb + (ic[m].o01 >> 16)));
          const frag v2 = ld8<T>((const T*)(rb + (ic[m].o23 & 0xffffu)));
          const frag v3 = ld8<T>((const T*)(rb + (ic[m].o23 >> 16)));
          af[m] = Ops::blend(v0, v1, v2, v3, ic[m]);
        }
        if (!ch_ok) af[m] = zero8<T>();
      }
#pragma unroll
      for (int m = 0; m < DCN_WM; ++m)
#pragma unroll
        for (int b = 0; b < NBF; ++b) acc[m][b] = Ops::mma(af[m], bf[b], acc[m][b]);
    }
  }

  // ---- 3c. samples outside a capped region: straight from global memory (rare) -----------------------
  if (block_may_slow) {
    for (int c = 0; c < g.nchunk; ++c) {
      const int ch = c * 32 + grp * 8;
      if (ch >= cin8) continue;  // uniform per lane group; no barrier inside
#pragma unroll 1
      for (int k = 0; k < 9; ++k) {
        frag af[DCN_WM];
        bool any = false;
#pragma unroll
        for (int m = 0; m < DCN_WM; ++m) {
          const int q = k * DCN_TILE + m * 16 + ibase;
          af[m] = zero8<T>();
          if (s_slow[q]) {
            // recompute the sample's geometry from the offsets (rare path)
            const int pl = m * 16 + ibase;
            const int oy = ty0 + pl / g.tw, ox = tx0 + pl - (pl / g.tw) * g.tw;
            const int64_t p = oy * g.wo + ox;
            const float dy = a.offset[n * a.off_sn + p * a.off_sp + (2 * k) * a.off_sc];
            const float dx = a.offset[n * a.off_sn + p * a.off_sp + (2 * k + 1) * a.off_sc];
            const float mk = a.mask ? a.mask[n * a.mask_sn + p * a.mask_sp + k * a.mask_sc] : 1.f;
            int cy0, cx0, sy, sx;
            float w[4];
            sample_geom((float)(oy * a.stride - a.pad + k / 3) + dy, (float)(ox * a.stride - a.pad + k % 3) + dx, mk,
                        a.h, a.w, cy0, cx0, sy, sx, w);
            const typename InfoOf<T>::type in = make_info<T>(0u, 0u, w);
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

  // ---- 4. epilogue ---------------------------------------------------------------------------------
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
        const int pl = wave * (16 * DCN_WM) + m * 16 + grp * 4 + i;
        const int oy = ty0 + pl / g.tw, ox = tx0 + pl - (pl / g.tw) * g.tw;
        float v = (acc[m][b][i] + bias) * mul + add;
        if (a.relu) v = fmaxf(v, 0.f);
        v *= scl;
        if (co_ok && pl < g.th * g.tw && oy < g.ho && ox < g.wo) {
          const int p = oy * g.wo + ox;
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
        a.gap_partial[((int64_t)n * g.tiles + tile) * a.cout + co] = v;
      }
    }
  }
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
  g.grid_x = round_up(g.tiles, 8);
  g.nchunk = ceil_div(a.cin, 32);
  g.cout_pad = round_up(a.cout, 16);
  return g;
}

template <typename T, typename OutT, int NBF, bool PLAIN>
static int launch_dcn(const kad_dcn_args& a, hipStream_t st, int ho, int wo) {
  const DcnGeom g = make_geom(a, ho, wo);
  dim3 grid(g.grid_x, ceil_div(a.cout, NBF * 16), a.n);
  hipLaunchKernelGGL((dcn_fwd_kernel<T, OutT, NBF, PLAIN>), grid, dim3(DCN_THREADS), 0, st, a, g);
  return check_launch(PLAIN ? "kad_conv3x3_fwd" : "kad_dcn_fwd");
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

static int validate_dcn(const kad_dcn_args* a, bool need_offset, int* ho_out, int* wo_out) {
  KAD_CHECK_ARG(a, "null args");
  KAD_CHECK_ARG(a->x && a->wpack && a->out && (a->offset || !need_offset), "null tensor pointer");
  KAD_CHECK_ARG(a->n > 0 && a->cin > 0 && a->cout > 0 && a->h > 0 && a->w > 0,
                "bad shape n=%d cin=%d cout=%d h=%d w=%d", a->n, a->cin, a->cout, a->h, a->w);
  KAD_CHECK_ARG(a->h < 32768 && a->w < 16384, "image %dx%d too large (H < 32768, W < 16384)", a->h, a->w);
  KAD_CHECK_ARG(a->stride >= 1 && a->pad >= 0, "bad stride=%d pad=%d", a->stride, a->pad);
  KAD_CHECK_ARG(a->x_cs % 8 == 0 && a->x_cs >= round_up(a->cin, 8),
                "x channel stride %d must be a multiple of 8 and >= roundup(cin=%d, 8)", a->x_cs, a->cin);
  KAD_CHECK_ARG(a->out_layout == KAD_NCHW || (a->out_layout == KAD_NHWC && a->out_cs >= a->cout),
                "bad output layout %d / channel stride %d", a->out_layout, a->out_cs);
  const int ho = (a->h + 2 * a->pad - 3) / a->stride + 1;
  const int wo = (a->w + 2 * a->pad - 3) / a->stride + 1;
  KAD_CHECK_ARG(ho > 0 && wo > 0, "empty output");
  const uintptr_t align = (uintptr_t)a->x | (uintptr_t)a->wpack;
  KAD_CHECK_ARG(align % 16 == 0, "x and wpack must be 16-byte aligned");
  *ho_out = ho;
  *wo_out = wo;
  return KAD_OK;
}

}  // namespace kad

using namespace kad;

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
