// LCSA (Low-Cost Spatial Attention), the mask generator of DSC:
//   mask = sigmoid( conv1x1_{C->9}( dwconv_{11x1}( relu(bn( dwconv_{1x11}( mean_w(x)[h] + mean_h(x)[w] ))))))
// (KAD-Conv/kadconv/kad_conv.py:18-39, 65; twin RCA in KAD-CNet/models/module/ops.py:12-37).
//
// Algebra used here (all exact rewrites of the module):
//  * The 1x11 depthwise conv of the broadcast sum a[h] + b[w] is separable
//    (the reference's Triton path uses the same identity,
//    acceleration/kadc_fused_sm75.py:861-878):
//      t[c,h,w] = a[c,h] * S_c(w) + B_c(w) + b1[c],  S_c(w) = sum of in-row taps,
//      B_c(w) = sum_k w1[c,k] b[c, w+k-5].
//    With eval BN folded (bn_a, bn_b):  u[c,h,w] = relu(alpha[c,w] * a[c,h] + beta[c,w]),
//      alpha = bn_a * S,  beta = bn_a * (B + b1) + bn_b.
//  * The 11x1 depthwise conv followed by the 1x1 projection is one matrix product
//      m[j, (h,w)] = b4'[j] + sum_{k,c} E[j,k,c] * u[c, h+k-5, w],
//      E[j,k,c] = w4[j,c] * w3[c,k],  b4' = b4 + w4 . b3,
//    i.e. a GEMM with M = 9 (padded to 16), K = 11 * C, N = pixels, run on MFMA
//    with u staged in LDS per 16 x 16 pixel tile (+5 rows above and below).
//
// Kernels: kad_axial_sums (row/column sums of an NHWC map, used when the sums
// do not come from kad_pyramid_proj), kad_lcsa_pack (E, b4' from the module
// weights), kad_lcsa_prep (row and column means from partial sums),
// kad_lcsa_mask (alpha/beta for its columns, u in LDS, the GEMM + sigmoid ->
// mask [N, H, W, 9] fp32, pixel-major).
#include "kad_common.h"

namespace kad {

constexpr int BAND = 11;
constexpr int HALF_BAND = 5;

// ---- axial sums of an NHWC map ---------------------------------------------------------------
// grid.x = H + W lines, grid.y = N.  Line l < H is row l (sum over w);
// otherwise column l - H (sum over h).  Threads stride over channels.
// Each sum is multiplied by rsc (rows) / csc (columns) before it is stored: 1 for sums, 1 / W and
// 1 / H for the means kad_lcsa_mask reads (the same product kad_lcsa_prep forms from one slice).
template <typename T>
__global__ __launch_bounds__(256) void axial_sums_kernel(const T* x, float* rows, float* cols, int c, int h, int w,
                                                        int cs, float rsc, float csc) {
  const int n = blockIdx.y;
  const int l = blockIdx.x;
  const T* base = x + (int64_t)n * h * w * cs;
  if (l < h) {
    for (int ch = threadIdx.x; ch < c; ch += 256) {
      float acc = 0.f;
      const T* p = base + (int64_t)l * w * cs + ch;
      for (int j = 0; j < w; ++j) acc += to_f32(p[(int64_t)j * cs]);
      rows[((int64_t)n * h + l) * c + ch] = acc * rsc;
    }
  } else {
    const int col = l - h;
    for (int ch = threadIdx.x; ch < c; ch += 256) {
      float acc = 0.f;
      const T* p = base + (int64_t)col * cs + ch;
      for (int i = 0; i < h; ++i) acc += to_f32(p[(int64_t)i * w * cs]);
      cols[((int64_t)n * w + col) * c + ch] = acc * csc;
    }
  }
}

// ---- axial sums of an NCHW map ---------------------------------------------------------------
// One block per (image, channel) plane: the plane is read once (8-byte pieces
// when its size is a multiple of 4 elements) into LDS as fp32 (rows padded by
// one float), then thread y sums row y and thread x sums column x, each in
// index order (deterministic).  Plane of at most AX_MAX_PX pixels.
constexpr int AX_MAX_PX = 12288;

template <typename T>
__global__ __launch_bounds__(256) void axial_sums_nchw_kernel(const T* x, float* rows, float* cols, int c, int h,
                                                             int w, float rsc, float csc) {
  extern __shared__ float pl[];  // [h][w + 1]
  const int plane = blockIdx.x, n = plane / c, ch = plane - n * c;
  const int P = h * w, ws = w + 1;
  const T* xp = x + (int64_t)plane * P;
  const float inv_w = 1.f / (float)w;
  if (P % 4 == 0) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    for (int e = threadIdx.x; e < P / 4; e += 256) {
      const t4 v = *(const t4*)(xp + 4 * e);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int f = 4 * e + j, y = (int)(((float)f + 0.5f) * inv_w), xx = f - y * w;
        pl[y * ws + xx] = to_f32(v[j]);
      }
    }
  } else {
    for (int f = threadIdx.x; f < P; f += 256) {
      const int y = (int)(((float)f + 0.5f) * inv_w), xx = f - y * w;
      pl[y * ws + xx] = to_f32(xp[f]);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < h + w; i += 256) {
    float a0 = 0.f, a1 = 0.f;
    if (i < h) {
      const float* r = pl + i * ws;
      int j = 0;
      for (; j + 1 < w; j += 2) {
        a0 += r[j];
        a1 += r[j + 1];
      }
      if (j < w) a0 += r[j];
      rows[((int64_t)n * h + i) * c + ch] = (a0 + a1) * rsc;
    } else {
      const int xx = i - h;
      int j = 0;
      for (; j + 1 < h; j += 2) {
        a0 += pl[j * ws + xx];
        a1 += pl[(j + 1) * ws + xx];
      }
      if (j < h) a0 += pl[j * ws + xx];
      cols[((int64_t)n * w + xx) * c + ch] = (a0 + a1) * csc;
    }
  }
}

// ---- E and b4' from the module weights -----------------------------------------------------------
// params (fp32): w1[C][11] | b1[C] | bn_a[C] | bn_b[C] | w3[C][11] | b3[C] | w4[9][C] | b4[9]
template <typename ET>
__global__ void lcsa_pack_kernel(const float* params, ET* emat, float* ebias, int c, int cp) {
  const float* w3 = params + 14 * c;
  const float* b3 = params + 25 * c;
  const float* w4 = params + 26 * c;
  const float* b4 = params + 35 * c;
  const int total = 16 * BAND * cp;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const int ch = i % cp, k = (i / cp) % BAND, j = i / (cp * BAND);
    const float v = (j < 9 && ch < c) ? w4[j * c + ch] * w3[ch * BAND + k] : 0.f;
    emat[i] = from_f32<ET>(v);
  }
  if (blockIdx.x == 0 && threadIdx.x < 16) {
    const int j = threadIdx.x;
    float acc = 0.f;
    if (j < 9) {
      acc = b4[j];
      for (int ch = 0; ch < c; ++ch) acc += w4[j * c + ch] * b3[ch];
    }
    ebias[j] = acc;
  }
}

// ---- axial means from partial slices -----------------------------------------------------------
// grid (H + W, N): block l < H reduces row l's slices, else column l - H's.
__device__ __forceinline__ void lcsa_prep_row(const float* rows, int nrp, const float* cols, int ncp, float* arow,
                                              float* colm, int c, int h, int w, int n, int l) {
  if (l < h) {
    const float inv = 1.f / (float)w;
    for (int ch = threadIdx.x; ch < c; ch += 256) {
      float s = 0.f;
#pragma unroll 8
      for (int p = 0; p < nrp; ++p) s += rows[(((int64_t)n * nrp + p) * h + l) * c + ch];
      arow[((int64_t)n * h + l) * c + ch] = s * inv;
    }
  } else {
    const int x = l - h;
    const float inv = 1.f / (float)h;
    for (int ch = threadIdx.x; ch < c; ch += 256) {
      float s = 0.f;
#pragma unroll 8
      for (int p = 0; p < ncp; ++p) s += cols[(((int64_t)n * ncp + p) * w + x) * c + ch];
      colm[((int64_t)n * w + x) * c + ch] = s * inv;
    }
  }
}

__global__ __launch_bounds__(256) void lcsa_prep_kernel(const float* rows, int nrp, const float* cols, int ncp,
                                                       float* arow, float* colm, int c, int h, int w) {
  lcsa_prep_row(rows, nrp, cols, ncp, arow, colm, c, h, w, blockIdx.y, blockIdx.x);
}

// ---- mask GEMM ------------------------------------------------------------------------------------
// The mask's sigmoid, shared by the single and split paths: v_rcp_f32 (1 ulp)
// instead of the IEEE division sequence (about ten instructions per value).
__device__ __forceinline__ float mask_sigmoid(float v) { return __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

constexpr int LM_TH = 16, LM_TW = 16;                   // output tile
constexpr int LM_UR = LM_TH + 2 * HALF_BAND;            // u rows staged
constexpr int LM_THREADS = 256;

template <typename ET> struct LmCfg { static constexpr int ldu = 40; };  // 32 + 8 halves per (row, col)
template <> struct LmCfg<float> { static constexpr int ldu = 36; };

// E fragment of one lane (8 channels) and the MFMA against 8 channels of u in LDS.
template <typename ET> struct LmFrag;
template <> struct LmFrag<half_t> {
  typedef half8_t frag;
  static __device__ __forceinline__ frag ld(const half_t* p) { return *(const half8_t*)p; }
  static __device__ __forceinline__ floatx4 mma(const frag& a, const half_t* b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, *(const half8_t*)b, c, 0, 0, 0);
  }
};
struct LmF32x8 { floatx4 lo, hi; };
template <> struct LmFrag<float> {
  typedef LmF32x8 frag;
  static __device__ __forceinline__ frag ld(const float* p) { return LmF32x8{*(const floatx4*)p, *(const floatx4*)(p + 4)}; }
  static __device__ __forceinline__ floatx4 mma(const frag& a, const float* b, floatx4 c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[j], b[j], c, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[j], b[4 + j], c, 0, 0, 0);
    return c;
  }
};

constexpr int LM_SC = 96;                              // channels per staged group (3 chunks)
constexpr int LM_SCS = LM_SC + 4;                       // fp32 row stride of the staged group

// grid (ceil(W/16), ceil(H/16), N).  Wave v computes tile rows 4v..4v+3 (4 MFMA
// column fragments of 16 pixels each) for all 16 (9 used) mask logits.
// Per group of up to 96 channels, one round trip brings the block's column
// means (26 columns: 16 + the 11-tap halo), row means (26 rows) and the
// strip-conv / BN parameters into LDS; alpha / beta of the 16 columns are
// formed there once.  Per 32-channel chunk: the lanes' E fragments (11 taps) are
// requested first, u = relu(alpha a + beta) is written to LDS meanwhile, then
// 11 x 4 MFMAs.
// SC: channels per staged group (LM_SC; 32 when every problem has one 32-channel chunk, which cuts
// the block's LDS from ~71 KB to ~46 KB: three blocks per CU instead of two).
template <typename ET, int SC = LM_SC>
__device__ __forceinline__ void lcsa_mask_block(const float* arow, const float* colm, const float* params,
                                                const ET* emat, const float* ebias, float* mask, int c, int h, int w,
                                                int cp, int ksplit, float* part, const int bx, const int by,
                                                const int bz, const int nz) {
  constexpr int LDU = LmCfg<ET>::ldu;
  constexpr int SCS = SC + 4;
  static_assert(SC % 32 == 0 && SC <= LM_SC, "whole 32-channel chunks");
  __shared__ __align__(16) ET us[LM_UR * LM_TW * LDU];
  __shared__ __align__(16) float s_col[LM_UR][SCS];   // column means, columns w0 - 5 .. w0 + 20
  __shared__ __align__(16) float s_a[LM_UR][SCS];     // row means, rows h0 - 5 .. h0 + 20
  __shared__ float s_w1[SC * BAND], s_b1[SC], s_bna[SC], s_bnb[SC];
  __shared__ __align__(16) float s_alpha[LM_TW][SCS], s_beta[LM_TW][SCS];
  __shared__ float s_eb[16];  // logit biases, staged with the first group
  const float* w1 = params;
  const float* b1 = params + 11 * c;
  const float* bna = params + 12 * c;
  const float* bnb = params + 13 * c;
  // grid.z = N x ksplit: split sp takes the chunks [kc0, kc1) of the channel contraction
  const int n = bz / ksplit, sp = bz - n * ksplit;
  const int h0 = by * LM_TH, w0 = bx * LM_TW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, grp = lane >> 4;
  const float* colm_n = colm + (int64_t)n * w * c;
  const float* arow_n = arow + (int64_t)n * h * c;
  floatx4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Flat loop over 32-channel chunks kc; groups of SC / 32 = 3 chunks share the
  // staged means / parameters.  Loads run ahead: the next group's means and
  // parameters are requested as soon as the current group is in LDS, the next
  // chunk's E fragments as soon as the current chunk's MFMAs are issued.  The
  // barriers inside the loop wait for LDS traffic only (a workgroup barrier
  // would also drain those loads).
  constexpr int NW = (LM_UR * SC + LM_THREADS - 1) / LM_THREADS;    // per window
  constexpr int NP = (SC * BAND + LM_THREADS - 1) / LM_THREADS;     // w1
  constexpr int NQ = (3 * SC + LM_THREADS - 1) / LM_THREADS;        // b1 | bn_a | bn_b
  constexpr int CPG = SC / 32;                                      // chunks per group
  const int nk = cp / 32;
  const int kc0 = sp * nk / ksplit, kc1 = (sp + 1) * nk / ksplit;
  float vc_[NW], va_[NW], vw_[NP], vq_[NQ];
  typedef typename LmFrag<ET>::frag EF;
  EF ef[BAND];
  // Index space uses the fixed group width SC (constant divisors); channels past
  // c or past the group read 0.
#define LM_LOAD_GROUP(CS)                                                                                      \
  {                                                                                                            \
    const int cs_ = (CS), nsc_ = cp - cs_ < SC ? cp - cs_ : SC;                                          \
    _Pragma("unroll") for (int u = 0; u < NW; ++u) {                                                           \
      const int e = tid + u * LM_THREADS, r = e / SC, ch = e - r * SC, gc = cs_ + ch;                    \
      const int gx = w0 - HALF_BAND + r, gy = h0 - HALF_BAND + r;                                              \
      const bool ok = r < LM_UR && ch < nsc_ && gc < c;                                                        \
      vc_[u] = (ok && gx >= 0 && gx < w) ? colm_n[(uint32_t)(gx * c + gc)] : 0.f;                              \
      va_[u] = (ok && gy >= 0 && gy < h) ? arow_n[(uint32_t)(gy * c + gc)] : 0.f;                              \
    }                                                                                                          \
    _Pragma("unroll") for (int u = 0; u < NP; ++u) {                                                           \
      const int e = tid + u * LM_THREADS;                                                                      \
      vw_[u] = (e < nsc_ * BAND && cs_ * BAND + e < c * BAND) ? w1[cs_ * BAND + e] : 0.f;                      \
    }                                                                                                          \
    _Pragma("unroll") for (int u = 0; u < NQ; ++u) {                                                           \
      const int e = tid + u * LM_THREADS, which = e / SC, ch = e - which * SC, gc = cs_ + ch;            \
      vq_[u] = (which < 3 && ch < nsc_ && gc < c) ? (which == 0 ? b1 : which == 1 ? bna : bnb)[gc] : 0.f;      \
    }                                                                                                          \
  }
  // this lane's E fragments of chunk KC: logit row l16, taps 0..10, channels 32 KC + grp * 8 .. + 8
#define LM_LOAD_E(KC)                                                                                          \
  _Pragma("unroll") for (int k = 0; k < BAND; ++k) ef[k] =                                                     \
      LmFrag<ET>::ld(emat + (int64_t)(l16 * BAND + k) * cp + (KC) * 32 + grp * 8);
#define LM_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")
  // logit biases, read in the epilogue after many barriers; loaded first, so that their LDS
  // store waits for this load only, not for the group's and the E fragments' loads behind it
  const float ebv = tid < 9 ? ebias[tid] : 0.f;
  LM_LOAD_GROUP((kc0 / CPG) * SC);
  LM_LOAD_E(kc0);
  if (tid < 16) s_eb[tid] = ebv;
  for (int kc = kc0; kc < kc1; ++kc) {
    const int g = kc / CPG, c0 = (kc - g * CPG) * 32, cs = g * SC;
    if (c0 == 0 || kc == kc0) {  // first chunk of a group (or of the split): stage it, request the next one
      const int nsc = cp - cs < SC ? cp - cs : SC;
      LM_LDS_BARRIER();  // the previous group's LDS data is consumed
#pragma unroll
      for (int u = 0; u < NW; ++u) {
        const int e = tid + u * LM_THREADS, r = e / SC, ch = e - r * SC;
        if (r < LM_UR) {
          s_col[r][ch] = vc_[u];
          s_a[r][ch] = va_[u];
        }
      }
#pragma unroll
      for (int u = 0; u < NP; ++u) {
        const int e = tid + u * LM_THREADS;
        if (e < SC * BAND) s_w1[e] = vw_[u];
      }
#pragma unroll
      for (int u = 0; u < NQ; ++u) {
        const int e = tid + u * LM_THREADS, which = e / SC, ch = e - which * SC;
        if (which < 3) (which == 0 ? s_b1 : which == 1 ? s_bna : s_bnb)[ch] = vq_[u];
      }
      LM_LDS_BARRIER();
      // strip-conv coefficients of the 16 columns (separable 1x11 conv + folded BN): task
      // (channel ch, quarter qc of the columns) holds the channel's 11 taps and the 14 column
      // means its 4 columns need in registers and forms the 4 sliding sums.  The staged column
      // means are 0 outside the image, so only S needs the in-image mask.
      static_assert(LM_TW == 16, "four column quarters");
      for (int e = tid; e < 4 * SC; e += LM_THREADS) {
        const int qc = e / SC, ch = e - qc * SC;
        float wk[BAND], cm[4 + BAND - 1];
#pragma unroll
        for (int k = 0; k < BAND; ++k) wk[k] = s_w1[ch * BAND + k];
#pragma unroll
        for (int j = 0; j < 4 + BAND - 1; ++j) cm[j] = s_col[qc * 4 + j][ch];
        const bool chok = ch < nsc && cs + ch < c;
        const float bna = s_bna[ch], bb = s_b1[ch], bnb = s_bnb[ch];
        // 1 / 0: window column j (image column w0 + 4 qc - 5 + j) inside / outside the image.
        // S sums the in-image taps as fma(wk, ind, S): S + wk * 1 and S + wk * 0 round exactly
        // like S + wk and S + 0 (finite weights), with one instruction per tap instead of three.
        float ind[4 + BAND - 1];
#pragma unroll
        for (int j = 0; j < 4 + BAND - 1; ++j) {
          const int xx = w0 + qc * 4 - HALF_BAND + j;
          ind[j] = (xx >= 0 && xx < w) ? 1.f : 0.f;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = qc * 4 + q, gx = w0 + col;
          float S0 = 0.f, S1 = 0.f, B0 = 0.f, B1 = 0.f;  // even / odd taps, added last
#pragma unroll
          for (int k = 0; k < BAND; ++k) {
            if (k & 1) {
              S1 = fmaf(wk[k], ind[q + k], S1);
              B1 += wk[k] * cm[q + k];
            } else {
              S0 = fmaf(wk[k], ind[q + k], S0);
              B0 += wk[k] * cm[q + k];
            }
          }
          const float S = S0 + S1, B = B0 + B1;
          const bool ok = gx < w && chok;
          s_alpha[col][ch] = ok ? bna * S : 0.f;
          s_beta[col][ch] = ok ? bna * (B + bb) + bnb : 0.f;
        }
      }
      if ((g + 1) * CPG < kc1) LM_LOAD_GROUP(cs + SC);  // after the coefficients: fewer live registers there
    }
    LM_LDS_BARRIER();  // alpha / beta ready; the previous chunk's MFMAs are done with us
    // u = relu(alpha * a + beta): thread (column, 8-channel group) fixed, rows r0, r0 + 4, ...;
    // its alpha / beta are read once per chunk, one 16-byte LDS store per row
    {
    const int gq = tid & 3, col = (tid >> 2) & (LM_TW - 1), r0 = tid >> 6;
    const int ch = c0 + gq * 8;
    const floatx4 al0 = *(const floatx4*)&s_alpha[col][ch], al1 = *(const floatx4*)&s_alpha[col][ch + 4];
    const floatx4 be0 = *(const floatx4*)&s_beta[col][ch], be1 = *(const floatx4*)&s_beta[col][ch + 4];
    [[maybe_unused]] const half8_t alh =
        __builtin_convertvector(__builtin_shufflevector(al0, al1, 0, 1, 2, 3, 4, 5, 6, 7), half8_t);
    [[maybe_unused]] const half8_t beh =
        __builtin_convertvector(__builtin_shufflevector(be0, be1, 0, 1, 2, 3, 4, 5, 6, 7), half8_t);
    for (int r = r0; r < LM_UR; r += LM_THREADS / (4 * LM_TW)) {
      const int gy = h0 - HALF_BAND + r;
      const bool rv = gy >= 0 && gy < h;
      const floatx4 a0 = *(const floatx4*)&s_a[r][ch], a1 = *(const floatx4*)&s_a[r][ch + 4];
      ET* dst = us + (r * LM_TW + col) * LDU + gq * 8;
      if constexpr (sizeof(ET) == 2) {
        // packed fp16 (two values per v_pk_fma_f16 / v_pk_max_f16): u is stored in fp16 anyway;
        // alpha, a and beta rounded to fp16 first move it by a few fp16 ulps
        const half8_t ah = __builtin_convertvector(__builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7), half8_t);
        half8_t v = __builtin_elementwise_max(alh * ah + beh, (half8_t)(half_t)0);
        if (!rv) v = (half8_t)(half_t)0;
        *(half8_t*)dst = v;
      } else {
        floatx4 v0, v1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v0[j] = rv ? fmaxf(al0[j] * a0[j] + be0[j], 0.f) : 0.f;
          v1[j] = rv ? fmaxf(al1[j] * a1[j] + be1[j], 0.f) : 0.f;
        }
        ((floatx4*)dst)[0] = v0;
        ((floatx4*)dst)[1] = v1;
      }
    }
    }
    LM_LDS_BARRIER();
#pragma unroll
    for (int k = 0; k < BAND; ++k) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int r = wave * 4 + f;  // tile row of this fragment
        acc[f] = LmFrag<ET>::mma(ef[k], &us[((r + k) * LM_TW + l16) * LDU + grp * 8], acc[f]);
      }
    }
    if (kc + 1 < kc1) LM_LOAD_E(kc + 1);
  }
#undef LM_LOAD_GROUP
#undef LM_LOAD_E
#undef LM_LDS_BARRIER
  float eb[4];  // this lane's logit biases (logits 4 grp .. 4 grp + 3)
#pragma unroll
  for (int i = 0; i < 4; ++i) eb[i] = s_eb[grp * 4 + i];
  // acc[f][i]: logit j = 4 * grp + i of pixel (row 4 * wave + f, col l16)
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int gy = h0 + wave * 4 + f, gx = w0 + l16;
    if (gy >= h || gx >= w) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = grp * 4 + i;
      if (j >= 9) continue;
      if (ksplit == 1)
        mask[(((int64_t)n * h + gy) * w + gx) * 9 + j] = mask_sigmoid(acc[f][i] + eb[i]);
      else  // raw logits of this split; lcsa_mask_reduce_kernel adds the splits up
        part[((((int64_t)sp * nz / ksplit + n) * h + gy) * w + gx) * 9 + j] = acc[f][i];
    }
  }
}

template <typename ET>
__global__ __launch_bounds__(LM_THREADS, 2) void lcsa_mask_kernel(const float* arow, const float* colm,
                                                                 const float* params, const ET* emat,
                                                                 const float* ebias, float* mask, int c, int h,
                                                                 int w, int cp, int ksplit, float* part) {
  lcsa_mask_block<ET>(arow, colm, params, emat, ebias, mask, c, h, w, cp, ksplit, part, blockIdx.x, blockIdx.y,
                      blockIdx.z, gridDim.z);
}

// Several LCSA problems (the branches of a KAD-Conv layer) in one launch: problem p owns blocks
// [start[p], start[p + 1]) = its ceil(W/16) x ceil(H/16) x N tiles, unsplit.
struct LcsaGroup {
  kad_lcsa_args a[KAD_LCSA_GROUP_MAX];
  int start[KAD_LCSA_GROUP_MAX + 1];
  int count;
};

template <typename ET, int SC>
__global__ __launch_bounds__(LM_THREADS, SC == 32 ? 3 : 2) void lcsa_mask_group_kernel(LcsaGroup grp) {
  const int id = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < KAD_LCSA_GROUP_MAX; ++i)
    if (i < grp.count && id >= grp.start[i]) p = i;
  const kad_lcsa_args& a = grp.a[p];
  const int local = id - grp.start[p];
  const int tx = ceil_div(a.w, LM_TW), ty = ceil_div(a.h, LM_TH);
  lcsa_mask_block<ET, SC>(a.arow, a.colm, a.params, (const ET*)a.emat, a.ebias, a.mask, a.c, a.h, a.w,
                          round_up(a.c, 32), 1, nullptr, local % tx, (local / tx) % ty, local / (tx * ty), a.n);
}

// The axial means of several problems in one launch, one thread per (problem, image, row or
// column, channel), consecutive threads on consecutive channels (contiguous in the slices).  A
// block per line left 256 - C threads of every block idle: 9600 blocks of which 5% of the lanes
// worked at KAD-CNet-S's 100^2 layers.  Sums in the same order as lcsa_prep_row (bit-identical).
__global__ __launch_bounds__(256) void lcsa_prep_flat_kernel(LcsaGroup grp) {
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (int q = 0; q < grp.count; ++q) {
    const kad_lcsa_args& a = grp.a[q];
    const int64_t items = (int64_t)a.n * (a.h + a.w) * a.c;
    if (i >= items) {
      i -= items;
      continue;
    }
    const int ch = (int)(i % a.c);
    const int64_t r = i / a.c;
    const int l = (int)(r % (a.h + a.w)), n = (int)(r / (a.h + a.w));
    float s = 0.f;
    if (l < a.h) {
#pragma unroll 8
      for (int p = 0; p < a.nrp; ++p) s += a.rows[(((int64_t)n * a.nrp + p) * a.h + l) * a.c + ch];
      a.arow[((int64_t)n * a.h + l) * a.c + ch] = s * (1.f / (float)a.w);
    } else {
      const int x = l - a.h;
#pragma unroll 8
      for (int p = 0; p < a.ncp; ++p) s += a.cols[(((int64_t)n * a.ncp + p) * a.w + x) * a.c + ch];
      a.colm[((int64_t)n * a.w + x) * a.c + ch] = s * (1.f / (float)a.h);
    }
    return;
  }
}

// mask = sigmoid(sum over the splits, in split order, + ebias): one thread per (pixel, logit).
__global__ __launch_bounds__(256) void lcsa_mask_reduce_kernel(const float* part, const float* ebias, float* mask,
                                                               int64_t total, int ksplit) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  float v = 0.f;
  for (int s = 0; s < ksplit; ++s) v += part[s * total + i];
  mask[i] = mask_sigmoid(v + ebias[i % 9]);
}

}  // namespace kad

using namespace kad;

extern "C" int64_t kad_lcsa_params_elems(int c) { return c > 0 ? 35 * (int64_t)c + 9 : 0; }

extern "C" int64_t kad_lcsa_emat_elems(int c) { return c > 0 ? (int64_t)16 * BAND * round_up(c, 32) : 0; }

namespace kad {
static int launch_axial_nhwc(const void* x, float* rows, float* cols, int n, int c, int h, int w, int x_cs,
                             int dtype, float rsc, float csc, hipStream_t st, const char* who) {
  KAD_CHECK_ARG(x && rows && cols, "%s: null pointer", who);
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0 && x_cs >= c, "%s: bad shape", who);
  dim3 grid(h + w, n);
  switch (dtype) {
    case KAD_F32: hipLaunchKernelGGL(axial_sums_kernel<float>, grid, dim3(256), 0, st, (const float*)x, rows, cols, c, h, w, x_cs, rsc, csc); break;
    case KAD_F16: hipLaunchKernelGGL(axial_sums_kernel<half_t>, grid, dim3(256), 0, st, (const half_t*)x, rows, cols, c, h, w, x_cs, rsc, csc); break;
    case KAD_BF16: hipLaunchKernelGGL(axial_sums_kernel<bf16_t>, grid, dim3(256), 0, st, (const bf16_t*)x, rows, cols, c, h, w, x_cs, rsc, csc); break;
    default: return fail(KAD_EINVAL, "%s: unknown dtype %d", who, dtype);
  }
  return check_launch(who);
}

static int launch_axial_nchw(const void* x, float* rows, float* cols, int n, int c, int h, int w, int dtype,
                             float rsc, float csc, hipStream_t st, const char* who) {
  KAD_CHECK_ARG(x && rows && cols, "%s: null pointer", who);
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0, "%s: bad shape", who);
  KAD_CHECK_ARG((int64_t)h * w <= AX_MAX_PX, "%s: %dx%d plane exceeds %d pixels", who, h, w, AX_MAX_PX);
  KAD_CHECK_ARG((int64_t)n * c < (1ll << 31), "%s: too many planes", who);
  KAD_CHECK_ARG(((uintptr_t)x) % (4 * dtype_size(dtype)) == 0, "%s: x must be aligned to 4 elements", who);
  const size_t lds = (size_t)h * (w + 1) * sizeof(float);
  const dim3 grid(n * c);
  switch (dtype) {
    case KAD_F32: allow_lds(axial_sums_nchw_kernel<float>, lds); hipLaunchKernelGGL(axial_sums_nchw_kernel<float>, grid, dim3(256), lds, st, (const float*)x, rows, cols, c, h, w, rsc, csc); break;
    case KAD_F16: allow_lds(axial_sums_nchw_kernel<half_t>, lds); hipLaunchKernelGGL(axial_sums_nchw_kernel<half_t>, grid, dim3(256), lds, st, (const half_t*)x, rows, cols, c, h, w, rsc, csc); break;
    case KAD_BF16: allow_lds(axial_sums_nchw_kernel<bf16_t>, lds); hipLaunchKernelGGL(axial_sums_nchw_kernel<bf16_t>, grid, dim3(256), lds, st, (const bf16_t*)x, rows, cols, c, h, w, rsc, csc); break;
    default: return fail(KAD_EINVAL, "%s: unknown dtype %d", who, dtype);
  }
  return check_launch(who);
}
}  // namespace kad

extern "C" int kad_axial_sums(const void* x, float* rows, float* cols, int n, int c, int h, int w, int x_cs,
                              int dtype, void* stream) {
  return launch_axial_nhwc(x, rows, cols, n, c, h, w, x_cs, dtype, 1.f, 1.f, (hipStream_t)stream, "kad_axial_sums");
}

extern "C" int kad_axial_sums_nchw(const void* x, float* rows, float* cols, int n, int c, int h, int w, int dtype,
                                   void* stream) {
  return launch_axial_nchw(x, rows, cols, n, c, h, w, dtype, 1.f, 1.f, (hipStream_t)stream, "kad_axial_sums_nchw");
}

extern "C" int kad_axial_means(const void* x, float* arow, float* colm, int n, int c, int h, int w, int x_cs,
                               int dtype, void* stream) {
  if (h <= 0 || w <= 0) return fail(KAD_EINVAL, "kad_axial_means: bad shape");
  return launch_axial_nhwc(x, arow, colm, n, c, h, w, x_cs, dtype, 1.f / (float)w, 1.f / (float)h,
                           (hipStream_t)stream, "kad_axial_means");
}

extern "C" int kad_axial_means_nchw(const void* x, float* arow, float* colm, int n, int c, int h, int w, int dtype,
                                    void* stream) {
  if (h <= 0 || w <= 0) return fail(KAD_EINVAL, "kad_axial_means_nchw: bad shape");
  return launch_axial_nchw(x, arow, colm, n, c, h, w, dtype, 1.f / (float)w, 1.f / (float)h, (hipStream_t)stream,
                           "kad_axial_means_nchw");
}

extern "C" int kad_lcsa_pack(const float* params, void* emat, float* ebias, int c, int emat_dtype, void* stream) {
  KAD_CHECK_ARG(params && emat && ebias && c > 0, "kad_lcsa_pack: bad arguments");
  const int cp = round_up(c, 32);
  hipStream_t st = (hipStream_t)stream;
  if (emat_dtype == KAD_F32)
    hipLaunchKernelGGL(lcsa_pack_kernel<float>, dim3(64), dim3(256), 0, st, params, (float*)emat, ebias, c, cp);
  else if (emat_dtype == KAD_F16)
    hipLaunchKernelGGL(lcsa_pack_kernel<half_t>, dim3(64), dim3(256), 0, st, params, (half_t*)emat, ebias, c, cp);
  else
    return fail(KAD_EINVAL, "kad_lcsa_pack: emat dtype must be KAD_F32 or KAD_F16");
  return check_launch("kad_lcsa_pack");
}

extern "C" int kad_lcsa_prep(const float* rows, int nrp, const float* cols, int ncp, float* arow, float* colm,
                             int n, int c, int h, int w, void* stream) {
  KAD_CHECK_ARG(rows && cols && arow && colm, "kad_lcsa_prep: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0 && nrp > 0 && ncp > 0, "kad_lcsa_prep: bad shape");
  hipLaunchKernelGGL(lcsa_prep_kernel, dim3(h + w, n), dim3(256), 0, (hipStream_t)stream, rows, nrp, cols, ncp,
                     arow, colm, c, h, w);
  return check_launch("kad_lcsa_prep");
}

namespace kad {

static int launch_lcsa_mask(const float* arow, const float* colm, const float* params, const void* emat,
                            const float* ebias, float* mask, int n, int c, int h, int w, int emat_dtype, int ksplit,
                            float* work, hipStream_t st) {
  const int cp = round_up(c, 32);
  dim3 grid(ceil_div(w, LM_TW), ceil_div(h, LM_TH), n * ksplit);
  if (emat_dtype == KAD_F32)
    hipLaunchKernelGGL(lcsa_mask_kernel<float>, grid, dim3(LM_THREADS), 0, st, arow, colm, params,
                       (const float*)emat, ebias, mask, c, h, w, cp, ksplit, work);
  else if (emat_dtype == KAD_F16)
    hipLaunchKernelGGL(lcsa_mask_kernel<half_t>, grid, dim3(LM_THREADS), 0, st, arow, colm, params,
                       (const half_t*)emat, ebias, mask, c, h, w, cp, ksplit, work);
  else
    return fail(KAD_EINVAL, "kad_lcsa_mask: emat dtype must be KAD_F32 or KAD_F16");
  int rc = check_launch("kad_lcsa_mask");
  if (rc || ksplit == 1) return rc;
  const int64_t total = (int64_t)n * h * w * 9;
  hipLaunchKernelGGL(lcsa_mask_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, work, ebias,
                     mask, total, ksplit);
  return check_launch("kad_lcsa_mask (split reduction)");
}

}  // namespace kad

extern "C" int kad_lcsa_mask(const float* arow, const float* colm, const float* params, const void* emat,
                             const float* ebias, float* mask, int n, int c, int h, int w, int emat_dtype,
                             void* stream) {
  KAD_CHECK_ARG(arow && colm && params && emat && ebias && mask, "kad_lcsa_mask: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0, "kad_lcsa_mask: bad shape");
  KAD_CHECK_ARG((int64_t)(h > w ? h : w) * c < (1ll << 31), "kad_lcsa_mask: H or W times C exceeds 2^31 (32-bit mean indices)");
  KAD_CHECK_ARG(((uintptr_t)emat) % 16 == 0, "kad_lcsa_mask: emat must be 16-byte aligned");
  return kad::launch_lcsa_mask(arow, colm, params, emat, ebias, mask, n, c, h, w, emat_dtype, 1, nullptr,
                               (hipStream_t)stream);
}

static int validate_lcsa_group(const kad_lcsa_args* a, int count, const char* what) {
  KAD_CHECK_ARG(a && count >= 1 && count <= KAD_LCSA_GROUP_MAX, "%s: count %d outside [1, %d]", what, count,
                KAD_LCSA_GROUP_MAX);
  for (int p = 0; p < count; ++p) {
    const kad_lcsa_args& b = a[p];
    KAD_CHECK_ARG(b.rows && b.cols && b.arow && b.colm && b.params && b.emat && b.ebias && b.mask,
                  "%s: problem %d: null pointer", what, p);
    KAD_CHECK_ARG(b.n > 0 && b.c > 0 && b.h > 0 && b.w > 0 && b.nrp > 0 && b.ncp > 0, "%s: problem %d: bad shape",
                  what, p);
    KAD_CHECK_ARG((int64_t)(b.h > b.w ? b.h : b.w) * b.c < (1ll << 31), "%s: problem %d: H or W times C too large",
                  what, p);
    KAD_CHECK_ARG(((uintptr_t)b.emat) % 16 == 0, "%s: problem %d: emat must be 16-byte aligned", what, p);
  }
  return KAD_OK;
}

extern "C" int kad_lcsa_prep_group(const kad_lcsa_args* a, int count, void* stream) {
  int rc = validate_lcsa_group(a, count, "kad_lcsa_prep_group");
  if (rc) return rc;
  kad::LcsaGroup grp;
  grp.count = count;
  int64_t items = 0;
  for (int p = 0; p < count; ++p) {
    grp.a[p] = a[p];
    items += (int64_t)a[p].n * (a[p].h + a[p].w) * a[p].c;
  }
  KAD_CHECK_ARG(items < (1ll << 31) - 256, "kad_lcsa_prep_group: too many (image, line, channel) items");
  hipLaunchKernelGGL(kad::lcsa_prep_flat_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, grp);
  return check_launch("kad_lcsa_prep_group");
}

extern "C" int kad_lcsa_mask_group(const kad_lcsa_args* a, int count, int emat_dtype, void* stream) {
  int rc = validate_lcsa_group(a, count, "kad_lcsa_mask_group");
  if (rc) return rc;
  kad::LcsaGroup grp;
  grp.count = count;
  int64_t blocks = 0;
  for (int p = 0; p < count; ++p) {
    grp.a[p] = a[p];
    grp.start[p] = (int)blocks;
    blocks += (int64_t)ceil_div(a[p].w, kad::LM_TW) * ceil_div(a[p].h, kad::LM_TH) * a[p].n;
  }
  KAD_CHECK_ARG(blocks < (1ll << 31), "kad_lcsa_mask_group: too many blocks");
  for (int p = count; p <= KAD_LCSA_GROUP_MAX; ++p) grp.start[p] = (int)blocks;
  hipStream_t st = (hipStream_t)stream;
  bool one_chunk = true;  // every problem's channels in one 32-channel chunk: the narrow staging
  for (int p = 0; p < count; ++p) one_chunk = one_chunk && a[p].c <= 32;
  if (emat_dtype == KAD_F32 && one_chunk)
    hipLaunchKernelGGL((kad::lcsa_mask_group_kernel<float, 32>), dim3((unsigned)blocks), dim3(kad::LM_THREADS), 0, st, grp);
  else if (emat_dtype == KAD_F32)
    hipLaunchKernelGGL((kad::lcsa_mask_group_kernel<float, kad::LM_SC>), dim3((unsigned)blocks), dim3(kad::LM_THREADS), 0, st, grp);
  else if (emat_dtype == KAD_F16 && one_chunk)
    hipLaunchKernelGGL((kad::lcsa_mask_group_kernel<half_t, 32>), dim3((unsigned)blocks), dim3(kad::LM_THREADS), 0, st, grp);
  else if (emat_dtype == KAD_F16)
    hipLaunchKernelGGL((kad::lcsa_mask_group_kernel<half_t, kad::LM_SC>), dim3((unsigned)blocks), dim3(kad::LM_THREADS), 0, st, grp);
  else
    return fail(KAD_EINVAL, "kad_lcsa_mask_group: emat dtype must be KAD_F32 or KAD_F16");
  return check_launch("kad_lcsa_mask_group");
}

extern "C" int kad_lcsa_mask_splits(int n, int c, int h, int w) {
  if (n <= 0 || c <= 0 || h <= 0 || w <= 0) return 0;
  // two blocks fit a CU; split the channel chunks until about 512 blocks are in flight
  const int blocks = ceil_div(w, kad::LM_TW) * ceil_div(h, kad::LM_TH) * n;
  const int nk = round_up(c, 32) / 32;
  const int want = 512 / blocks;
  return want <= 1 ? 1 : (want < nk ? want : nk);
}

extern "C" int64_t kad_lcsa_mask_work_elems(int n, int h, int w, int ksplit) {
  return (n > 0 && h > 0 && w > 0 && ksplit > 1) ? (int64_t)ksplit * n * h * w * 9 : 0;
}

extern "C" int kad_lcsa_mask_split(const float* arow, const float* colm, const float* params, const void* emat,
                                   const float* ebias, float* mask, int n, int c, int h, int w, int emat_dtype,
                                   int ksplit, float* work, void* stream) {
  KAD_CHECK_ARG(arow && colm && params && emat && ebias && mask, "kad_lcsa_mask_split: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0, "kad_lcsa_mask_split: bad shape");
  KAD_CHECK_ARG((int64_t)(h > w ? h : w) * c < (1ll << 31), "kad_lcsa_mask_split: H or W times C exceeds 2^31 (32-bit mean indices)");
  KAD_CHECK_ARG(((uintptr_t)emat) % 16 == 0, "kad_lcsa_mask_split: emat must be 16-byte aligned");
  KAD_CHECK_ARG(ksplit >= 1 && ksplit <= round_up(c, 32) / 32, "kad_lcsa_mask_split: ksplit %d outside [1, %d]",
                ksplit, round_up(c, 32) / 32);
  KAD_CHECK_ARG(ksplit == 1 || work, "kad_lcsa_mask_split: ksplit > 1 needs a work buffer");
  KAD_CHECK_ARG((int64_t)n * ksplit < 65536, "kad_lcsa_mask_split: N x ksplit too large");
  return kad::launch_lcsa_mask(arow, colm, params, emat, ebias, mask, n, c, h, w, emat_dtype, ksplit, work,
                               (hipStream_t)stream);
}
