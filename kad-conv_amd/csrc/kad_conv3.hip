// Plain 3x3 convolution, 16-bit NHWC, as an implicit GEMM on MFMA (gfx950).
//
// The hot path of KAD-CNet's ordinary 3x3 Convs (stem, AConv / ELAN / GELAN convs,
// the DDetect heads): out = post_scale * act((conv3x3(x, W) + bias) * post_mul + post_add),
// KAD-CNet/models/common.py:43-58 (Conv = conv + BN + SiLU, BN folded into W and bias
// by the host as KAD-CNet/utils/torch_utils.py:244-265 does).  kad_conv_fwd sends
// 16-bit NHWC-output launches here (convolution_igemm); other cases stay on the DCN
// machinery's plain mode.
//
// Design (one block = a TH x TW output patch of at most 128 pixels x BN = 32 NBW output
// channels; 4 waves):
//  * GEMM view: M = pixels, N = output channels, K = 9 taps x Cin, walked as
//    32-channel chunks x 9 taps.  For each chunk the block stages in LDS
//      - the patch's input footprint [(TH-1)S+3][(TW-1)S+3] pixels x 32 channels
//        (80-byte pixel rows), and
//      - the chunk's weights [9 taps][BN][32] (64-byte rows, 16-byte pieces
//        XOR-swizzled by column so a B read's lanes spread over the banks);
//    the next chunk is loaded into registers while the current one is multiplied.
//  * Waves form a 2 x 2 grid: wave (wm, wn) owns pixels 64 wm .. 64 wm + 63 (four
//    16-pixel A fragments) and columns 16 NBW wn .. (NBW B fragments), so every
//    LDS fragment read feeds 4 or NBW MFMAs (v_mfma_f32_16x16x32): per tap a wave
//    reads 4 + NBW fragments for 4 NBW MFMAs.
//  * The A fragment of tap (ky, kx) for output pixel (py, px) is the footprint
//    pixel (py S + ky, px S + kx): a shifted view of the staged footprint, no im2col.
//    For stride 2 the footprint's even and odd columns are stored as two halves
//    (column fx at fx / 2 or (FW + 1) / 2 + fx / 2), so the 16 lanes of a fragment
//    (consecutive output columns) read consecutive 80-byte rows for every tap, as
//    with stride 1.
//  * Taps are software-pipelined (fully unrolled, fragments of tap k + 1 read while
//    tap k multiplies).  Accumulation is fp32, chunk-major then tap order.  The MFMA
//    takes the weights as its row operand, so a lane's accumulator holds 4 consecutive
//    output channels of one pixel: the epilogue writes them as one 8-byte piece.
//  * Epilogue: parameters applied in registers, the tile staged in LDS (the weight
//    buffer) and written with 16-byte row-contiguous stores.
//  * Blocks over (image, patch) flattened in XCD-aware order: each XCD takes a
//    contiguous run of patches, so neighbouring patches share input rows in one L2.
#include <type_traits>

#include "kad_common.h"

namespace kad {
namespace {

constexpr int CV_THREADS = 256;
constexpr int CV_PX = 128;               // output pixels per block (4 waves x 2 pixel halves of 64)
constexpr int CV_PXS = 40;               // elements per staged footprint pixel (32 + 8 pad: 80-byte rows)
constexpr int CV_PXB = CV_PXS * 2;

template <int S> struct CvCap {
  // largest footprint of a patch of <= 128 pixels chosen by cv_pick_tile (TW in [4, 64])
  static constexpr int FPIX = S == 1 ? 264 : 648;
  // staging pieces per thread (4 per pixel) and the LDS pixels they cover (every slot is stored)
  static constexpr int RPT = (FPIX * 4 + CV_THREADS - 1) / CV_THREADS;
  static constexpr int SLOTS = RPT * CV_THREADS / 4;
};

template <typename T> struct CvFrag;
template <> struct CvFrag<half_t> {
  typedef half8_t frag;
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct CvFrag<bf16_t> {
  typedef bf16x8_t frag;
  static __device__ __forceinline__ floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ typename CvFrag<T>::frag lds8(const char* p) {
  return *(const typename CvFrag<T>::frag*)p;
}
template <typename T>
__device__ __forceinline__ void sts8(char* p, const typename CvFrag<T>::frag& v) {
  *(typename CvFrag<T>::frag*)p = v;
}
template <typename T>
__device__ __forceinline__ typename CvFrag<T>::frag gld8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(typename CvFrag<T>::frag, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}


// Weight tile slot of piece g of column c: g ^ ((c >> 1) & 3).
__device__ __forceinline__ int cv_wunit(int k, int bn, int col, int g) { return (k * bn + col) * 4 + (g ^ ((col >> 1) & 3)); }

struct CvGeom {
  int ho, wo, th, tw, tiles_x, tiles, grid_x, nchunk, cout_pad, fh, fw, hw, fpix;
  float inv_tw, inv_fw;
};

template <typename T, int NBW, int S>
__global__ __launch_bounds__(CV_THREADS, NBW <= 2 ? 2 : 1) void conv3x3_ig_kernel(kad_dcn_args a, CvGeom g) {
  typedef CvFrag<T> Ops;
  typedef typename Ops::frag frag;
  constexpr int BN = 32 * NBW;                                  // block columns
  constexpr int RPT = CvCap<S>::RPT;                            // footprint pieces per thread
  constexpr int WPT = (9 * BN * 4 + CV_THREADS - 1) / CV_THREADS;  // weight pieces per thread
  constexpr int SROW = BN + 8;                                  // epilogue staging row (elements)
  static_assert(CV_PX * SROW * 2 <= 9 * BN * 64, "epilogue tile must fit the weight buffer");
  __shared__ __align__(16) char region[CvCap<S>::SLOTS * CV_PXB];
  __shared__ __align__(16) char wsm[9 * BN * 64];
  __shared__ __align__(16) float s_par[3][BN];  // shift (bias * mul + add), mul, post_scale per column

  // XCD-aware order over (patch, column block), column blocks fastest: XCD b % 8 takes a contiguous
  // run, so a patch's column blocks stage its footprint from one L2, one after another
  const int ncb = ceil_div(a.cout, BN);
  const int qq = (blockIdx.x & 7) * (g.grid_x >> 3) + (blockIdx.x >> 3);
  if (qq >= a.n * g.tiles * ncb) return;  // whole block, before any barrier
  const int q = qq / ncb, cb = qq - q * ncb;
  const int n = q / g.tiles, tile = q - n * g.tiles;
  const int tyi = tile / g.tiles_x;
  const int ty0 = tyi * g.th, tx0 = (tile - tyi * g.tiles_x) * g.tw;
  const int co0 = cb * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = lane & 15, grp = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int fy0 = ty0 * S - a.pad, fx0 = tx0 * S - a.pad;
  const int cin8 = round_up(a.cin, 8);
  const T* xb = (const T*)a.x + (int64_t)n * a.h * a.w * a.x_cs;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xb, (uint32_t)(a.h * a.w * a.x_cs * 2));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.wpack, (uint32_t)(g.cout_pad * g.nchunk * 9 * 32 * 2));

  // epilogue parameters: requested first, staged in LDS with chunk 0
  float par[4] = {0.f, 1.f, 0.f, 1.f};
  if (tid < BN && co0 + tid < a.cout) {
    const int co = co0 + tid;
    if (a.bias) par[0] = a.bias[co];
    if (a.post_mul) par[1] = a.post_mul[co];
    if (a.post_add) par[2] = a.post_add[co];
    if (a.post_scale) par[3] = a.post_scale[co];
  }

  // ---- staging, walked in LDS order so every store is at a fixed offset from the thread's base -------
  // footprint: thread t, piece u -> stored pixel (t / 4 + 64 u), channels 8 (t % 4) of the chunk; stored
  // pixels past the footprint load nothing (zeros) and are never read.
  // weights: thread t, piece u -> 16-byte unit t + 256 u of the tile [9][BN][4 swizzled pieces].
  uint32_t roff[RPT];  // byte offset of the piece's chunk-0 channels in the image, or KAD_OOB
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int sp = (tid >> 2) + u * (CV_THREADS / 4);
    uint32_t o = KAD_OOB;
    if (sp < g.fpix) {
      const int fy = (int)(((float)sp + 0.5f) * g.inv_fw), sc = sp - fy * g.fw;
      const int fx = S == 1 ? sc : (sc < g.hw ? 2 * sc : 2 * (sc - g.hw) + 1);
      const int gy = fy0 + fy, gx = fx0 + fx;
      if (gy >= 0 && gy < a.h && gx >= 0 && gx < a.w) o = (uint32_t)(((gy * a.w + gx) * a.x_cs + (tid & 3) * 8) * 2);
    }
    roff[u] = o;
  }
  uint32_t woff[WPT];
#pragma unroll
  for (int u = 0; u < WPT; ++u) {
    const int e = tid + u * CV_THREADS;
    uint32_t o = KAD_OOB;
    if (e < 9 * BN * 4) {
      const int k = e / (BN * 4), r = e - k * (BN * 4), col = r >> 2, co = co0 + col;
      const int gq = (r & 3) ^ ((col >> 1) & 3);  // the piece stored in this slot
      if (co < g.cout_pad) o = (uint32_t)((((co * g.nchunk) * 9 + k) * 32 + gq * 8) * 2);
    }
    woff[u] = o;
  }
  char* const rst = region + (tid >> 2) * CV_PXB + (tid & 3) * 16;
  char* const wst = wsm + tid * 16;
  frag rv[RPT], wv[WPT];
  // piece p of a chunk's staging (p < RPT: footprint, else weights)
  auto load_piece = [&](int p, int c) {
    if (p < RPT) {
      const bool chs = c * 32 + (tid & 3) * 8 < cin8;  // this thread's channel group holds real channels
      rv[p] = gld8<T>(rx, chs ? roff[p] : KAD_OOB, (uint32_t)(c * 64));
    } else {
      wv[p - RPT] = gld8<T>(rw, woff[p - RPT], (uint32_t)(c * 9 * 64));
    }
  };
  auto stage_load = [&](int c) {
#pragma unroll
    for (int p = 0; p < RPT + WPT; ++p) load_piece(p, c);
  };
  auto stage_store = [&]() {
#pragma unroll
    for (int u = 0; u < RPT; ++u) sts8<T>(rst + u * (CV_THREADS / 4) * CV_PXB, rv[u]);
#pragma unroll
    for (int u = 0; u < WPT; ++u)
      if ((u + 1) * CV_THREADS <= 9 * BN * 4 || tid + u * CV_THREADS < 9 * BN * 4) sts8<T>(wst + u * CV_THREADS * 16, wv[u]);
  };

  // ---- this lane's A rows: output pixel -> footprint byte offset of its (0, 0) tap ---------------------
  int abase[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    int pl = wm * 64 + m * 16 + row;
    if (pl >= g.th * g.tw) pl = 0;  // padding row: any in-bounds address, result discarded
    const int py = (int)(((float)pl + 0.5f) * g.inv_tw), px = pl - py * g.tw;
    abase[m] = (py * S * g.fw + px) * CV_PXB + grp * 16;
  }
  const int rowstep = g.fw * CV_PXB;
  const int kx1 = (S == 1 ? 1 : g.hw) * CV_PXB, kx2 = (S == 1 ? 2 : 1) * CV_PXB;
  const int bcol0 = wn * 16 * NBW + row;

  floatx4 acc[4][NBW];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int b = 0; b < NBW; ++b) acc[m][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  stage_load(0);
  stage_store();
  if (tid < BN) {
    s_par[0][tid] = par[0] * par[1] + par[2];
    s_par[1][tid] = par[1];
    s_par[2][tid] = par[3];
  }
  for (int c = 0; c < g.nchunk; ++c) {
    __syncthreads();  // chunk c staged
    const bool next = c + 1 < g.nchunk;
    frag af[2][4], bf[2][NBW];
    auto rd = [&](int k, frag (&ad)[4], frag (&bd)[NBW]) {
      const int ky = k / 3, kx = k - (k / 3) * 3;
      const int toff = ky * rowstep + (kx == 0 ? 0 : kx == 1 ? kx1 : kx2);
#pragma unroll
      for (int b = 0; b < NBW; ++b) bd[b] = lds8<T>(wsm + cv_wunit(k, BN, bcol0 + b * 16, grp) * 16);
#pragma unroll
      for (int m = 0; m < 4; ++m) ad[m] = lds8<T>(region + abase[m] + toff);
    };
    rd(0, af[0], bf[0]);
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      if (k + 1 < 9) rd(k + 1, af[(k + 1) & 1], bf[(k + 1) & 1]);
      // the next chunk's staging loads, spread over the taps (a burst would stall the MFMA issue)
      if (next) {
#pragma unroll
        for (int p = k * (RPT + WPT) / 9; p < (k + 1) * (RPT + WPT) / 9; ++p) load_piece(p, c + 1);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int b = 0; b < NBW; ++b) acc[m][b] = Ops::mma(bf[k & 1][b], af[k & 1][m], acc[m][b]);
    }
    if (next) {
      __syncthreads();  // every wave is done with chunk c
      stage_store();
    }
  }

  // ---- epilogue: parameters in registers -> LDS tile [128 px][SROW] -> 16-byte row stores --------------
  __syncthreads();  // every wave is done reading the weight buffer
  T* ost = (T*)wsm;
  // the activation is a template argument: with a per-value branch, every value's chain would be a
  // basic block of its own, and the scheduler could not interleave the 4 NBW x 4 independent chains
  auto epilogue = [&](auto act) {
    constexpr int ACT = decltype(act)::value;
#pragma unroll
    for (int b = 0; b < NBW; ++b) {
      const int col = wn * 16 * NBW + b * 16 + grp * 4;  // this lane's 4 channels
      const floatx4 sh = *(const floatx4*)&s_par[0][col], mu = *(const floatx4*)&s_par[1][col],
                    sc = *(const floatx4*)&s_par[2][col];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        T o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = fmaf(acc[m][b][i], mu[i], sh[i]);
          if constexpr (ACT == KAD_ACT_SILU) v = v * sigmoidf_(v);
          else if constexpr (ACT == KAD_ACT_RELU) v = fmaxf(v, 0.f);
          o[i] = from_f32<T>(v * sc[i]);
        }
        *(uint2*)(ost + (wm * 64 + m * 16 + row) * SROW + col) = __builtin_bit_cast(uint2, o);
      }
    }
  };
  if (a.relu == KAD_ACT_SILU) epilogue(std::integral_constant<int, KAD_ACT_SILU>{});
  else if (a.relu) epilogue(std::integral_constant<int, KAD_ACT_RELU>{});
  else epilogue(std::integral_constant<int, KAD_ACT_NONE>{});
  __syncthreads();
  T* out = (T*)a.out;
  const int64_t P = (int64_t)g.ho * g.wo;
  const bool vec_ok = (a.out_cs % 8) == 0 && ((uintptr_t)a.out & 15) == 0;
  constexpr int VPP = BN / 8;  // 16-byte vectors per pixel row of the tile
  constexpr int NIT = CV_PX * VPP / CV_THREADS;
  static_assert(NIT * CV_THREADS == CV_PX * VPP, "whole copy rounds");
  intx4 vv[NIT];
#pragma unroll
  for (int t = 0; t < NIT; ++t) {  // every LDS read first, then the stores
    const int j = tid + t * CV_THREADS, pl = j / VPP, v = j - pl * VPP;
    vv[t] = *(const intx4*)(ost + pl * SROW + v * 8);
  }
#pragma unroll
  for (int t = 0; t < NIT; ++t) {
    const int j = tid + t * CV_THREADS, pl = j / VPP, v = j - pl * VPP;
    const int oyl = (int)(((float)pl + 0.5f) * g.inv_tw);
    const int oy = ty0 + oyl, ox = tx0 + pl - oyl * g.tw;
    const int co = co0 + v * 8;
    if (pl >= g.th * g.tw || oy >= g.ho || ox >= g.wo || co >= a.cout) continue;
    T* dst = out + ((int64_t)n * P + (int64_t)oy * g.wo + ox) * a.out_cs + co;
    if (vec_ok && co + 8 <= a.cout) {
      *(intx4*)dst = vv[t];
    } else {
      const T* src = ost + pl * SROW + v * 8;
      for (int e = 0; e < 8 && co + e < a.cout; ++e) dst[e] = src[e];
    }
  }
}

// Patch shape for an Ho x Wo output: TH x TW <= 128 pixels with TW in [4, 64], minimising the
// padded pixel count; ties prefer squarer patches (smaller footprint).
void cv_pick_tile(int ho, int wo, int* th_out, int* tw_out) {
  long best = -1;
  int bth = 8, btw = 16;
  for (int tw = 4; tw <= 64; ++tw) {
    const int th = CV_PX / tw;
    const long cost = (long)ceil_div(ho, th) * ceil_div(wo, tw) * CV_PX * 64 + (th > tw ? th - tw : tw - th);
    if (best < 0 || cost < best) {
      best = cost;
      bth = th;
      btw = tw;
    }
  }
  *th_out = bth;
  *tw_out = btw;
}

// Output-channel fragments per wave (column blocks of 32 NBW channels).  Measured at batch 16, fp16
// (us for NBW = 1 .. 5):
//  * stride 1: NBW <= 2 keeps two blocks per CU, wider blocks one, so NBW = 2 wins broadly
//    (144 -> 208 at 100^2: 214 162 224 182 218; 216 -> 208 at 50^2: 79 61 80 72 85; 144 -> 144 at
//    25^2: 17.0 13.7 16.7 20.2 23.0).  Exceptions: Cout <= 96 where NBW = 2 pads more columns than
//    NBW = 1 (96 -> 96 at 50^2: 20.5 21.9; 32 -> 32 at 200^2: 41 70); one column block of 3 - 5
//    fragments on a launch of >= 1024 patches (144 -> 144 at 100^2: 163 135 154 180 116); and a small
//    launch that NBW = 3 fits in one block per CU where NBW = 2 would not (288 -> 208 at 25^2:
//    35.7 30.9 24.7 29.4 34.1).
//  * stride 2: every column block re-stages a footprint four times its patch, so the cost counts the
//    padded columns plus 32 per column block, ties to the narrower block, and a launch of fewer than
//    200 blocks narrows its column blocks (144 -> 216 at 100^2: 91 87 80 67.5 79; 216 -> 144 at 50^2:
//    25.0 20.5 22.8 26.8 30.3).
int cv_pick_nbw(int cout, long tiles, int stride) {
  if (stride != 1) {
    int best = 1;
    long best_cost = -1;
    for (int nbw = 1; nbw <= 5; ++nbw) {
      const long cb = ceil_div(cout, 32 * nbw), cost = cb * 32 * nbw + 32 * cb;
      if (best_cost < 0 || cost < best_cost) {
        best_cost = cost;
        best = nbw;
      }
    }
    while (best > 1 && tiles * ceil_div(cout, 32 * best) < 200) --best;
    return best;
  }
  if (cout <= 96 && round_up(cout, 64) > round_up(cout, 32)) return 1;
  const int nb1 = ceil_div(cout, 32);
  if (nb1 >= 3 && nb1 <= 5 && tiles >= 1024) return nb1;
  if (tiles * ceil_div(cout, 64) > 256 && tiles * ceil_div(cout, 96) <= 256) return 3;
  return 2;
}

template <typename T, int S>
int launch_nbw(const kad_dcn_args& a, const CvGeom& g, int nbw, hipStream_t st) {
  const dim3 block(CV_THREADS);
  CvGeom gl = g;  // one grid dimension over (patch, column block)
  gl.grid_x = round_up(a.n * g.tiles * ceil_div(a.cout, 32 * nbw), 8);
  const dim3 grid(gl.grid_x, 1, 1);
  switch (nbw) {
    case 1: hipLaunchKernelGGL((conv3x3_ig_kernel<T, 1, S>), grid, block, 0, st, a, gl); break;
    case 2: hipLaunchKernelGGL((conv3x3_ig_kernel<T, 2, S>), grid, block, 0, st, a, gl); break;
    case 3: hipLaunchKernelGGL((conv3x3_ig_kernel<T, 3, S>), grid, block, 0, st, a, gl); break;
    case 4: hipLaunchKernelGGL((conv3x3_ig_kernel<T, 4, S>), grid, block, 0, st, a, gl); break;
    default: hipLaunchKernelGGL((conv3x3_ig_kernel<T, 5, S>), grid, block, 0, st, a, gl); break;
  }
  return check_launch("kad_conv_fwd");
}

// ---- stem: 3x3 convolution of an NCHW image with at most 3 channels -----------------------------------
// The network's first Conv (3 -> C, stride 2) has K = 9 Cin <= 27: the whole reduction is one
// v_mfma_f32_16x16x32 step with k = 9 c + 3 ky + kx (k >= 9 Cin zero), instead of nine 32-channel taps
// of which 29 / 32 are padding.  The image is read as it comes (NCHW, no channels-last copy): a block
// (8 x 32 output pixels, 4 waves of two rows) stages its footprint as [Cin][FH][FWP] rows of 16-byte
// pieces (W % 8 == 0, so every piece is wholly inside or outside the image), each lane gathers the 8
// taps of its k-group from LDS, and the weights [co][k] form the MFMA's row operand, so a lane ends
// with 4 consecutive output channels of one pixel (one 8-byte NHWC store).
constexpr int ST_TH = 8, ST_TW = 32;

template <int S> struct StGeo {
  static constexpr int FH = (ST_TH - 1) * S + 3;          // footprint rows
  static constexpr int FWP = ((ST_TW - 1) * S + 3 + 7 + 7) / 8 * 8;  // from 8 before the first column
  static constexpr int PIECES = 3 * FH * (FWP / 8);       // at most 3 channels
  static constexpr int PPT = (PIECES + CV_THREADS - 1) / CV_THREADS;
};

template <typename T, int S, int NB>
__global__ __launch_bounds__(CV_THREADS) void stem_conv_kernel(kad_dcn_args a, int ho, int wo, int tiles_x,
                                                             int tiles) {
  typedef CvFrag<T> Ops;
  typedef typename Ops::frag frag;
  typedef StGeo<S> G;
  __shared__ __align__(16) T fp[3 * G::FH * G::FWP];
  const int q = blockIdx.x;
  const int n = q / tiles, tile = q - n * tiles;
  const int tyi = tile / tiles_x;
  const int ty0 = tyi * ST_TH, tx0 = (tile - tyi * tiles_x) * ST_TW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = lane & 15, grp = lane >> 4;
  const int y0 = ty0 * S - a.pad, xa = tx0 * S - 8;  // footprint row 0; column 0 of the staged rows
  const int cin = a.cin;
  const T* xb = (const T*)a.x + (int64_t)n * cin * a.h * a.w;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xb, (uint32_t)(cin * a.h * a.w * 2));

  // footprint pieces: (channel, row, 8 columns); outside the image -> zeros
  frag v[G::PPT];
  const int np = cin * G::FH * (G::FWP / 8);
#pragma unroll
  for (int u = 0; u < G::PPT; ++u) {
    const int e = tid + u * CV_THREADS;
    uint32_t o = KAD_OOB;
    if (e < np) {
      const int c = e / (G::FH * (G::FWP / 8)), r = e - c * (G::FH * (G::FWP / 8));
      const int fy = r / (G::FWP / 8), pc = r - fy * (G::FWP / 8);
      const int gy = y0 + fy, gx = xa + 8 * pc;
      if (gy >= 0 && gy < a.h && gx >= 0 && gx < a.w) o = (uint32_t)(((c * a.h + gy) * a.w + gx) * 2);
    }
    v[u] = gld8<T>(rx, o, 0);
  }
  // weights as the row operand: lane -> output channel 16 b + row, k = 8 grp + j (packed [co][9][32])
  frag wa[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int co = 16 * b + row;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = 8 * grp + j;
      T w = from_f32<T>(0.f);
      if (k < 9 * cin && co < a.cout) w = ((const T*)a.wpack)[co * 288 + (k % 9) * 32 + k / 9];
      wa[b][j] = w;
    }
  }
  float shift[NB][4];  // bias of this lane's output channels
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int co = 16 * b + 4 * grp + i;
      shift[b][i] = (a.bias && co < a.cout) ? a.bias[co] : 0.f;
    }
  // this lane's tap offsets in the footprint (element units), -1: k past 9 Cin
  int koff[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * grp + j;
    const int c = k / 9, t = k - 9 * c, ky = t / 3, kx = t - 3 * ky;
    koff[j] = k < 9 * cin ? (c * G::FH + ky) * G::FWP + kx + 7 : -1;
  }
#pragma unroll
  for (int u = 0; u < G::PPT; ++u) {
    const int e = tid + u * CV_THREADS;
    if (e < np) {
      const int c = e / (G::FH * (G::FWP / 8)), r = e - c * (G::FH * (G::FWP / 8));
      *(frag*)(fp + (c * G::FH) * G::FWP + r * 8) = v[u];
    }
  }
  __syncthreads();

  floatx4 acc[4][NB];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int py = 2 * wave + (m >> 1), px = 16 * (m & 1) + row;  // output pixel of this lane's column
    const T* base = fp + (py * S) * G::FWP + px * S;
    frag bm;
#pragma unroll
    for (int j = 0; j < 8; ++j) bm[j] = koff[j] >= 0 ? base[koff[j]] : from_f32<T>(0.f);
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[m][b] = Ops::mma(wa[b], bm, floatx4{0.f, 0.f, 0.f, 0.f});
  }

  T* out = (T*)a.out;
  const bool vec_ok = (a.out_cs % 4) == 0 && ((uintptr_t)a.out & 7) == 0;
  auto epilogue = [&](auto act) {
    constexpr int ACT = decltype(act)::value;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int oy = ty0 + 2 * wave + (m >> 1), ox = tx0 + 16 * (m & 1) + row;
      if (oy >= ho || ox >= wo) continue;
      T* dst = out + (((int64_t)n * ho + oy) * wo + ox) * a.out_cs;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int co = 16 * b + 4 * grp;
        if (co >= a.cout) continue;
        T o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float val = acc[m][b][i] + shift[b][i];
          if constexpr (ACT == KAD_ACT_SILU) val = val * sigmoidf_(val);
          else if constexpr (ACT == KAD_ACT_RELU) val = fmaxf(val, 0.f);
          o[i] = from_f32<T>(val);
        }
        if (vec_ok && co + 4 <= a.cout) {
          *(uint2*)(dst + co) = __builtin_bit_cast(uint2, o);
        } else {
          for (int i = 0; i < 4 && co + i < a.cout; ++i) dst[co + i] = o[i];
        }
      }
    }
  };
  if (a.relu == KAD_ACT_SILU) epilogue(std::integral_constant<int, KAD_ACT_SILU>{});
  else if (a.relu) epilogue(std::integral_constant<int, KAD_ACT_RELU>{});
  else epilogue(std::integral_constant<int, KAD_ACT_NONE>{});
}

template <typename T, int S>
int launch_stem(const kad_dcn_args& a, int ho, int wo, hipStream_t st) {
  const int tiles_x = ceil_div(wo, ST_TW), tiles = ceil_div(ho, ST_TH) * tiles_x;
  const dim3 grid(a.n * tiles), block(CV_THREADS);
  const int nb = ceil_div(a.cout, 16);
  switch (nb) {
    case 1: hipLaunchKernelGGL((stem_conv_kernel<T, S, 1>), grid, block, 0, st, a, ho, wo, tiles_x, tiles); break;
    case 2: hipLaunchKernelGGL((stem_conv_kernel<T, S, 2>), grid, block, 0, st, a, ho, wo, tiles_x, tiles); break;
    case 3: hipLaunchKernelGGL((stem_conv_kernel<T, S, 3>), grid, block, 0, st, a, ho, wo, tiles_x, tiles); break;
    default: hipLaunchKernelGGL((stem_conv_kernel<T, S, 4>), grid, block, 0, st, a, ho, wo, tiles_x, tiles); break;
  }
  return check_launch("kad_stem_conv_fwd");
}

}  // namespace

// 16-bit NHWC-output 3x3 convolution on the implicit-GEMM kernel; 1 = not handled here
// (the caller runs its general path).  `a` has passed the caller's validation.
int convolution_igemm(const kad_dcn_args& a, int ho, int wo, hipStream_t st) {
  if ((a.dtype != KAD_F16 && a.dtype != KAD_BF16) || a.out_layout != KAD_NHWC || a.gap_partial || a.se_att ||
      (a.stride != 1 && a.stride != 2))
    return 1;
  // stride 2 over fewer than 64 input channels (the stem and the next conv): the footprint is 4x the
  // output patch and at most two thin chunks amortise its staging; the general path is faster there
  if (a.stride == 2 && a.cin < 64) return 1;
  CvGeom g;
  g.ho = ho;
  g.wo = wo;
  cv_pick_tile(ho, wo, &g.th, &g.tw);
  g.tiles_x = ceil_div(wo, g.tw);
  g.tiles = ceil_div(ho, g.th) * g.tiles_x;
  g.grid_x = round_up(a.n * g.tiles, 8);
  g.nchunk = ceil_div(a.cin, 32);
  g.cout_pad = round_up(a.cout, 16);
  g.fh = (g.th - 1) * a.stride + 3;
  g.fw = (g.tw - 1) * a.stride + 3;
  g.hw = (g.fw + 1) / 2;
  g.fpix = g.fh * g.fw;
  g.inv_tw = 1.f / (float)g.tw;
  g.inv_fw = 1.f / (float)g.fw;
  if (g.fpix > (a.stride == 1 ? CvCap<1>::SLOTS : CvCap<2>::SLOTS)) return 1;
  const int nbw = cv_pick_nbw(a.cout, (long)a.n * g.tiles, a.stride);
  if (a.stride == 1) return a.dtype == KAD_F16 ? launch_nbw<half_t, 1>(a, g, nbw, st) : launch_nbw<bf16_t, 1>(a, g, nbw, st);
  return a.dtype == KAD_F16 ? launch_nbw<half_t, 2>(a, g, nbw, st) : launch_nbw<bf16_t, 2>(a, g, nbw, st);
}

}  // namespace kad

extern "C" int kad_stem_conv_fwd(const kad_dcn_args* a, void* stream) {
  using namespace kad;
  KAD_CHECK_ARG(a && a->x && a->wpack && a->out, "kad_stem_conv_fwd: null pointer");
  KAD_CHECK_ARG(a->dtype == KAD_F16 || a->dtype == KAD_BF16, "kad_stem_conv_fwd: 16-bit dtypes only (got %d)", a->dtype);
  KAD_CHECK_ARG(a->n > 0 && a->cin >= 1 && a->cin <= 3 && a->cout >= 1 && a->cout <= 64,
                "kad_stem_conv_fwd: n=%d cin=%d cout=%d (cin in [1, 3], cout in [1, 64])", a->n, a->cin, a->cout);
  KAD_CHECK_ARG((a->stride == 1 || a->stride == 2) && a->pad == 1, "kad_stem_conv_fwd: stride %d pad %d (stride 1 or 2, pad 1)",
                a->stride, a->pad);
  KAD_CHECK_ARG(a->h > 0 && a->w > 0 && a->w % 8 == 0 && (int64_t)a->cin * a->h * a->w * 2 < ((int64_t)1 << 31),
                "kad_stem_conv_fwd: image %dx%d (W a multiple of 8, one image below 2 GB)", a->h, a->w);
  KAD_CHECK_ARG(a->out_layout == KAD_NHWC && a->out_cs >= a->cout, "kad_stem_conv_fwd: NHWC output with out_cs >= cout");
  KAD_CHECK_ARG(!a->post_mul && !a->post_add && !a->post_scale && !a->gap_partial && !a->se_att,
                "kad_stem_conv_fwd: bias and activation only");
  KAD_CHECK_ARG(a->relu >= KAD_ACT_NONE && a->relu <= KAD_ACT_SILU, "kad_stem_conv_fwd: unknown activation %d", a->relu);
  KAD_CHECK_ARG(((uintptr_t)a->x & 15) == 0, "kad_stem_conv_fwd: x must be 16-byte aligned");
  const int ho = (a->h - 1) / a->stride + 1, wo = (a->w - 1) / a->stride + 1;
  KAD_CHECK_ARG((int64_t)a->n * ceil_div(ho, ST_TH) * ceil_div(wo, ST_TW) < (1ll << 31), "kad_stem_conv_fwd: grid too large");
  hipStream_t st = (hipStream_t)stream;
  if (a->stride == 1)
    return a->dtype == KAD_F16 ? launch_stem<half_t, 1>(*a, ho, wo, st) : launch_stem<bf16_t, 1>(*a, ho, wo, st);
  return a->dtype == KAD_F16 ? launch_stem<half_t, 2>(*a, ho, wo, st) : launch_stem<bf16_t, 2>(*a, ho, wo, st);
}
