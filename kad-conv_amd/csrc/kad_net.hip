// Network-level kernels of the KAD-CNet-S forward (everything around the KAD-Conv
// layers that is not a convolution), on NHWC feature maps with explicit channel
// strides so that producers and consumers address channel slices of concat
// buffers in place:
//  * kad_nhwc_resample: average pool (AConv's 2x2 / stride 1,
//    KAD-CNet/models/common.py:65-67), max pool (SPPELAN's SP(5),
//    common.py:187-193,563-577), nearest upsample (nn.Upsample(None, 2,
//    'nearest') of the neck) and plain channel-slice copies (torch.cat);
//  * kad_ddetect_decode: DDetect's inference tail (KAD-CNet/models/yolo.py:102-127):
//    DFL softmax expectation (models/common.py:232-244), anchors and
//    dist2bbox (utils/tal/anchor_generator.py:8-32) times the level stride,
//    and the class sigmoid, for all levels in one launch;
//  * kad_nms: greedy IoU suppression of score-sorted boxes (the
//    torchvision.ops.nms call of utils/general.py:961) as a pairwise bitmask
//    launch plus a one-block sweep.
// All are HBM- or latency-bound elementwise work: one thread per output pixel
// and 16-byte channel vector, consecutive threads along channels then pixels.
#include "kad_common.h"

namespace kad {

// ---- NHWC resample ---------------------------------------------------------------------------
enum { RS_AVG = 0, RS_MAX = 1, RS_NEAREST = 2 };

template <typename T, int VEC>
struct Vec {
  T v[VEC];
};

template <typename T, int VEC, int MODE>
__global__ __launch_bounds__(256) void resample_nhwc_kernel(kad_resample_args a) {
  const int cv = a.c / VEC;
  const int64_t total = (int64_t)a.n * a.ho * a.wo * cv;
  const T* src = (const T*)a.x;
  T* dst = (T*)a.out;
  const float inv_area = 1.f / (float)(a.k * a.k);
  // XCD-aware order (gridDim.x a multiple of 8): XCD b % 8 takes a contiguous eighth of the items,
  // so the input rows that neighbouring output rows share (pool windows, nearest-upsample sources)
  // are fetched into one L2 instead of several
  const int64_t bq = (int64_t)(blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const bool i32 = total < ((int64_t)1 << 32);
  for (int64_t i = bq * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int c, ox, oy, n;
    if (i32) {
      const uint32_t ii = (uint32_t)i, pix = ii / (uint32_t)cv, t = pix / (uint32_t)a.wo;
      c = (int)(ii - pix * (uint32_t)cv) * VEC;
      ox = (int)(pix - t * (uint32_t)a.wo);
      n = (int)(t / (uint32_t)a.ho);
      oy = (int)(t - (uint32_t)n * (uint32_t)a.ho);
    } else {
      c = (int)(i % cv) * VEC;
      const int64_t pix = i / cv;
      ox = (int)(pix % a.wo);
      const int64_t t = pix / a.wo;
      oy = (int)(t % a.ho);
      n = (int)(t / a.ho);
    }
    const T* base = src + (int64_t)n * a.h * a.w * a.x_cs + c;
    float acc[VEC];
    if (MODE == RS_NEAREST) {
      // PyTorch nearest with an integer scale factor: src = floor(dst / s)
      const int sy = oy / a.s, sx = ox / a.s;
      const Vec<T, VEC> v = *(const Vec<T, VEC>*)(base + ((int64_t)sy * a.w + sx) * a.x_cs);
      *(Vec<T, VEC>*)(dst + (((int64_t)n * a.ho + oy) * a.wo + ox) * a.out_cs + c) = v;
      continue;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = MODE == RS_MAX ? -INFINITY : 0.f;
    const int y0 = oy * a.s - a.p, x0 = ox * a.s - a.p;
    for (int dy = 0; dy < a.k; ++dy) {
      const int yy = y0 + dy;
      if (yy < 0 || yy >= a.h) continue;  // padding: 0 for the average (counted), -inf for the max
      for (int dx = 0; dx < a.k; ++dx) {
        const int xx = x0 + dx;
        if (xx < 0 || xx >= a.w) continue;
        const Vec<T, VEC> v = *(const Vec<T, VEC>*)(base + ((int64_t)yy * a.w + xx) * a.x_cs);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float f = to_f32(v.v[e]);
          acc[e] = MODE == RS_MAX ? fmaxf(acc[e], f) : acc[e] + f;
        }
      }
    }
    Vec<T, VEC> o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o.v[e] = from_f32<T>(MODE == RS_AVG ? acc[e] * inv_area : acc[e]);
    *(Vec<T, VEC>*)(dst + (((int64_t)n * a.ho + oy) * a.wo + ox) * a.out_cs + c) = o;
  }
}

template <typename T, int VEC>
static int launch_resample(const kad_resample_args& a, hipStream_t st) {
  const int64_t total = (int64_t)a.n * a.ho * a.wo * (a.c / VEC);
  const int blocks = round_up((int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536), 8);
  switch (a.mode) {
    case KAD_RS_AVG: hipLaunchKernelGGL((resample_nhwc_kernel<T, VEC, RS_AVG>), dim3(blocks), dim3(256), 0, st, a); break;
    case KAD_RS_MAX: hipLaunchKernelGGL((resample_nhwc_kernel<T, VEC, RS_MAX>), dim3(blocks), dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((resample_nhwc_kernel<T, VEC, RS_NEAREST>), dim3(blocks), dim3(256), 0, st, a); break;
  }
  return check_launch("kad_nhwc_resample");
}

// SPPELAN's three chained k x k max pools (stride 1, padding k / 2) of one 8-channel group of one
// image, the map held in LDS: a max pool applied j times is one max pool of radius j r (r = k / 2,
// padding never wins a max), so row maxima of radius r, 2 r, 3 r come from one another (radius
// 2 r at x = the larger of radius r at x - r and at x + r, indices clamped to the row: the clamped
// window stays inside the wanted one), then each output takes its column window over them.  One
// launch and one read of the map instead of three pools that each re-read the previous output.
template <typename T>
__global__ __launch_bounds__(256) void maxpool3_nhwc_kernel(kad_resample_args a) {
  typedef Vec8<T> V;  // 16-byte aligned: one 16-byte LDS / memory access per 8 channels
  extern __shared__ __align__(16) char mp_smem[];
  const int hw = a.h * a.w, r = a.k / 2;
  V* xs = (V*)mp_smem;  // [4][h][w]: the map, then row maxima of radius r, 2 r, 3 r
  const int g = blockIdx.x, n = blockIdx.y;
  const T* src = (const T*)a.x + (int64_t)n * hw * a.x_cs + 8 * g;
  auto vmax = [](const V& p, const V& q) {
    V o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o.v[e] = from_f32<T>(fmaxf(to_f32(p.v[e]), to_f32(q.v[e])));
    return o;
  };
  for (int i = threadIdx.x; i < hw; i += 256) xs[i] = *(const V*)(src + (int64_t)i * a.x_cs);
  __syncthreads();
  for (int i = threadIdx.x; i < hw; i += 256) {
    const int y = i / a.w, x = i - y * a.w;
    const int x0 = x - r < 0 ? 0 : x - r, x1 = x + r >= a.w ? a.w - 1 : x + r;
    V m = xs[y * a.w + x0];
    for (int xx = x0 + 1; xx <= x1; ++xx) m = vmax(m, xs[y * a.w + xx]);
    xs[hw + i] = m;
  }
  for (int j = 2; j <= 3; ++j) {
    __syncthreads();
    const V* prev = xs + (j - 1) * hw;
    for (int i = threadIdx.x; i < hw; i += 256) {
      const int y = i / a.w, x = i - y * a.w;
      const int xl = x - r < 0 ? 0 : x - r, xr = x + r >= a.w ? a.w - 1 : x + r;
      xs[j * hw + i] = vmax(prev[y * a.w + xl], prev[y * a.w + xr]);
    }
  }
  __syncthreads();
  T* dst = (T*)a.out + (int64_t)n * hw * a.out_cs + 8 * g;
  for (int e = threadIdx.x; e < 3 * hw; e += 256) {
    const int j = e / hw, i = e - j * hw;  // output j + 1: column window of radius (j + 1) r
    const int y = i / a.w, x = i - y * a.w, rad = (j + 1) * r;
    const int y0 = y - rad < 0 ? 0 : y - rad, y1 = y + rad >= a.h ? a.h - 1 : y + rad;
    const V* rm = xs + (j + 1) * hw;
    V m = rm[y0 * a.w + x];
    for (int yy = y0 + 1; yy <= y1; ++yy) m = vmax(m, rm[yy * a.w + x]);
    *(V*)(dst + (int64_t)i * a.out_cs + j * a.c) = m;
  }
}

template <typename T>
static int dispatch_resample(const kad_resample_args& a, hipStream_t st) {
  constexpr int V = 16 / (int)sizeof(T);
  const bool vec = a.c % V == 0 && a.x_cs % V == 0 && a.out_cs % V == 0 && ((uintptr_t)a.x & 15) == 0 &&
                   ((uintptr_t)a.out & 15) == 0;
  return vec ? launch_resample<T, V>(a, st) : launch_resample<T, 1>(a, st);
}

// ---- DDetect decode ---------------------------------------------------------------------------
// One thread per (image, anchor).  Anchor a of level l sits at cell (x, y) of
// that level's map, centre (x + 0.5, y + 0.5) in cells; its 16 x 4 box logits
// are channels [0, 64) of the level's head map (side j's bins at 16 j + b) and
// its class logits channels [box_ch, box_ch + nc).
template <typename T>
__global__ __launch_bounds__(256) void ddetect_decode_kernel(kad_decode_args a, int total_anchors) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.n * total_anchors) return;
  const int n = (int)(i / total_anchors);
  int anc = (int)(i - (int64_t)n * total_anchors);
  int l = 0;
  while (l + 1 < a.nl && anc >= a.anchor_off[l + 1]) ++l;
  const int cell = anc - a.anchor_off[l];
  const int cx = cell % a.lw[l], cy = cell / a.lw[l];
  const T* h = (const T*)a.head[l] + ((int64_t)n * a.lh[l] * a.lw[l] + cell) * a.head_cs[l];
  const int reg = a.reg_max;
  float d[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float m = -INFINITY;
    for (int b = 0; b < reg; ++b) m = fmaxf(m, to_f32(h[j * reg + b]));
    float s = 0.f, e = 0.f;
    for (int b = 0; b < reg; ++b) {
      const float p = __expf(to_f32(h[j * reg + b]) - m);
      s += p;
      e += p * (float)b;
    }
    d[j] = e / s;  // expectation of the bin index under the softmax
  }
  const float st = a.stride[l];
  const float ax = (float)cx + 0.5f, ay = (float)cy + 0.5f;
  const float x1 = ax - d[0], y1 = ay - d[1], x2 = ax + d[2], y2 = ay + d[3];
  T* y = (T*)a.out + (int64_t)n * (4 + a.nc) * total_anchors + anc;
  const int64_t A = total_anchors;
  y[0] = from_f32<T>((x1 + x2) * 0.5f * st);
  y[A] = from_f32<T>((y1 + y2) * 0.5f * st);
  y[2 * A] = from_f32<T>((x2 - x1) * st);
  y[3 * A] = from_f32<T>((y2 - y1) * st);
  for (int k = 0; k < a.nc; ++k) y[(4 + k) * A] = from_f32<T>(sigmoidf_(to_f32(h[a.box_ch + k])));
}

// The same decode when reg_max is 16 and every level's anchor records are whole 16-byte pieces
// (head_cs and box_ch multiples of 16 bytes, 16-byte aligned maps): the thread fetches its anchor's
// box logits with 4 * 16 / V 16-byte loads issued together and its class logits up to 4 pieces
// at a time, instead of one element per load (records are head_cs elements apart, so an
// element-wise load touches a different cache line in every lane).  Arithmetic as above, in the
// same order.
template <typename T>
__global__ __launch_bounds__(256) void ddetect_decode_vec_kernel(kad_decode_args a, int total_anchors) {
  constexpr int V = 16 / (int)sizeof(T), REG = 16, NBV = 4 * REG / V, CU = 4;
  typedef T piece[V];
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.n * total_anchors) return;
  const int n = (int)(i / total_anchors);
  int anc = (int)(i - (int64_t)n * total_anchors);
  int l = 0;
  while (l + 1 < a.nl && anc >= a.anchor_off[l + 1]) ++l;
  const int cell = anc - a.anchor_off[l];
  const int cx = cell % a.lw[l], cy = cell / a.lw[l];
  const T* h = (const T*)a.head[l] + ((int64_t)n * a.lh[l] * a.lw[l] + cell) * a.head_cs[l];
  intx4 bv[NBV];
#pragma unroll
  for (int q = 0; q < NBV; ++q) bv[q] = *(const intx4*)(h + q * V);
  float d[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float x[REG];
#pragma unroll
    for (int b = 0; b < REG; ++b) x[b] = to_f32(__builtin_bit_cast(piece, bv[(j * REG + b) / V])[(j * REG + b) % V]);
    float m = -INFINITY;
#pragma unroll
    for (int b = 0; b < REG; ++b) m = fmaxf(m, x[b]);
    float s = 0.f, e = 0.f;
#pragma unroll
    for (int b = 0; b < REG; ++b) {
      const float p = __expf(x[b] - m);
      s += p;
      e += p * (float)b;
    }
    d[j] = e / s;
  }
  const float st = a.stride[l];
  const float ax = (float)cx + 0.5f, ay = (float)cy + 0.5f;
  const float x1 = ax - d[0], y1 = ay - d[1], x2 = ax + d[2], y2 = ay + d[3];
  T* y = (T*)a.out + (int64_t)n * (4 + a.nc) * total_anchors + anc;
  const int64_t A = total_anchors;
  y[0] = from_f32<T>((x1 + x2) * 0.5f * st);
  y[A] = from_f32<T>((y1 + y2) * 0.5f * st);
  y[2 * A] = from_f32<T>((x2 - x1) * st);
  y[3 * A] = from_f32<T>((y2 - y1) * st);
  const T* hc = h + a.box_ch;
  const int ncv = a.nc - a.nc % V;  // classes in whole pieces
  for (int k0 = 0; k0 < ncv; k0 += CU * V) {
    intx4 cv[CU];
#pragma unroll
    for (int u = 0; u < CU; ++u)
      if (k0 + u * V < ncv) cv[u] = *(const intx4*)(hc + k0 + u * V);
#pragma unroll
    for (int u = 0; u < CU; ++u) {
      if (k0 + u * V >= ncv) break;
      const auto pc = __builtin_bit_cast(piece, cv[u]);
#pragma unroll
      for (int e = 0; e < V; ++e) y[(4 + k0 + u * V + e) * A] = from_f32<T>(sigmoidf_(to_f32(pc[e])));
    }
  }
  for (int k = ncv; k < a.nc; ++k) y[(4 + k) * A] = from_f32<T>(sigmoidf_(to_f32(hc[k])));
}

// ---- NMS --------------------------------------------------------------------------------------
// boxes [n][4] fp32 (x1, y1, x2, y2), sorted by descending score.  Block (col block
// cb, row block rb) with cb >= rb: thread t owns row i = 64 rb + t and sets bit j
// of mask[i][cb] when box 64 cb + j comes after i and IoU(i, that box) > thr,
// IoU = inter / (area_i + area_j - inter) in fp32, as torchvision computes it.
__global__ __launch_bounds__(64) void nms_mask_kernel(const float* __restrict__ boxes, unsigned long long* mask,
                                                      int n, int nw, float thr) {
  const int rb = blockIdx.y, cb = blockIdx.x;
  if (cb < rb) return;
  __shared__ float cbox[64][4];
  const int t = threadIdx.x;
  const int j0 = cb * 64;
  if (j0 + t < n) {
#pragma unroll
    for (int e = 0; e < 4; ++e) cbox[t][e] = boxes[(int64_t)(j0 + t) * 4 + e];
  }
  __syncthreads();
  const int i = rb * 64 + t;
  if (i >= n) return;
  const float bx1 = boxes[(int64_t)i * 4 + 0], by1 = boxes[(int64_t)i * 4 + 1];
  const float bx2 = boxes[(int64_t)i * 4 + 2], by2 = boxes[(int64_t)i * 4 + 3];
  // every step rounded on its own (no fused multiply-add), so the IoU is the
  // plain fp32 evaluation of the formula, bit for bit
  const float area = __fmul_rn(__fsub_rn(bx2, bx1), __fsub_rn(by2, by1));
  unsigned long long bits = 0ull;
  const int jn = n - j0 < 64 ? n - j0 : 64;
  for (int jj = 0; jj < jn; ++jj) {
    if (j0 + jj <= i) continue;
    const float iw = fmaxf(__fsub_rn(fminf(bx2, cbox[jj][2]), fmaxf(bx1, cbox[jj][0])), 0.f);
    const float ih = fmaxf(__fsub_rn(fminf(by2, cbox[jj][3]), fmaxf(by1, cbox[jj][1])), 0.f);
    const float inter = __fmul_rn(iw, ih);
    const float other = __fmul_rn(__fsub_rn(cbox[jj][2], cbox[jj][0]), __fsub_rn(cbox[jj][3], cbox[jj][1]));
    const float iou = __fdiv_rn(inter, __fsub_rn(__fadd_rn(area, other), inter));
    if (iou > thr) bits |= 1ull << jj;
  }
  mask[(int64_t)i * nw + cb] = bits;
}

// One block walks the boxes in score order: box i is kept unless an earlier kept
// box suppressed it; a kept box ORs its row of the mask into the removed set.
// Only words >= i / 64 of row i are read (the mask launch writes just those).
// Every thread reads the same removed bit, then a barrier separates those reads
// from the ORs of a kept box (which a second barrier closes), so the decision
// is block-uniform and no LDS word is read while it is written.
constexpr int NMS_SWEEP = 256;
__global__ __launch_bounds__(NMS_SWEEP) void nms_sweep_kernel(const unsigned long long* __restrict__ mask,
                                                              unsigned char* keep, int n, int nw) {
  extern __shared__ unsigned long long removed[];
  const int t = threadIdx.x;
  for (int w = t; w < nw; w += NMS_SWEEP) removed[w] = 0ull;
  __syncthreads();
  for (int i = 0; i < n; ++i) {
    const int wi = i >> 6;
    const bool alive = !((removed[wi] >> (i & 63)) & 1ull);
    if (t == 0) keep[i] = alive ? 1 : 0;
    __syncthreads();
    if (alive) {
      for (int w = wi + t; w < nw; w += NMS_SWEEP) removed[w] |= mask[(int64_t)i * nw + w];
      __syncthreads();
    }
  }
}

}  // namespace kad

using namespace kad;

extern "C" int kad_nhwc_resample(const kad_resample_args* a, void* stream) {
  KAD_CHECK_ARG(a && a->x && a->out, "kad_nhwc_resample: null pointer");
  KAD_CHECK_ARG(a->n > 0 && a->c > 0 && a->h > 0 && a->w > 0 && a->ho > 0 && a->wo > 0,
                "kad_nhwc_resample: bad shape n=%d c=%d %dx%d -> %dx%d", a->n, a->c, a->h, a->w, a->ho, a->wo);
  KAD_CHECK_ARG(a->x_cs >= a->c && a->out_cs >= a->c, "kad_nhwc_resample: channel strides %d / %d < c=%d", a->x_cs,
                a->out_cs, a->c);
  KAD_CHECK_ARG(a->mode == KAD_RS_AVG || a->mode == KAD_RS_MAX || a->mode == KAD_RS_NEAREST ||
                    a->mode == KAD_RS_MAX3,
                "kad_nhwc_resample: unknown mode %d", a->mode);
  if (a->mode == KAD_RS_MAX3) {
    KAD_CHECK_ARG(a->k >= 1 && a->k % 2 == 1 && a->s == 1 && a->p == a->k / 2 && a->ho == a->h && a->wo == a->w,
                  "kad_nhwc_resample: KAD_RS_MAX3 needs an odd k, s = 1, p = k / 2 and ho, wo = h, w");
    KAD_CHECK_ARG(a->out_cs >= 3 * a->c, "kad_nhwc_resample: KAD_RS_MAX3 writes 3 c channels (out_cs %d < %d)",
                  a->out_cs, 3 * a->c);
    hipStream_t st = (hipStream_t)stream;
    const size_t lds = (size_t)4 * a->h * a->w * 16;
    if (a->dtype != KAD_F32 && a->c % 8 == 0 && a->x_cs % 8 == 0 && a->out_cs % 8 == 0 &&
        ((uintptr_t)a->x & 15) == 0 && ((uintptr_t)a->out & 15) == 0 && lds <= 64 * 1024) {
      const dim3 grid(a->c / 8, a->n);
      if (a->dtype == KAD_F16) hipLaunchKernelGGL(maxpool3_nhwc_kernel<half_t>, grid, dim3(256), lds, st, *a);
      else hipLaunchKernelGGL(maxpool3_nhwc_kernel<bf16_t>, grid, dim3(256), lds, st, *a);
      return check_launch("kad_nhwc_resample");
    }
    // otherwise three max pools, each reading the previous output slice
    kad_resample_args b = *a;
    b.mode = KAD_RS_MAX;
    const int esz = a->dtype == KAD_F32 ? 4 : 2;
    for (int j = 0; j < 3; ++j) {
      if (j > 0) {
        b.x = (const char*)a->out + (size_t)(j - 1) * a->c * esz;
        b.x_cs = a->out_cs;
      }
      b.out = (char*)a->out + (size_t)j * a->c * esz;
      int rc;
      switch (a->dtype) {
        case KAD_F32: rc = dispatch_resample<float>(b, st); break;
        case KAD_F16: rc = dispatch_resample<half_t>(b, st); break;
        case KAD_BF16: rc = dispatch_resample<bf16_t>(b, st); break;
        default: return fail(KAD_EINVAL, "kad_nhwc_resample: unknown dtype %d", a->dtype);
      }
      if (rc) return rc;
    }
    return KAD_OK;
  }
  if (a->mode == KAD_RS_NEAREST) {
    KAD_CHECK_ARG(a->s >= 1 && a->ho == a->h * a->s && a->wo == a->w * a->s,
                  "kad_nhwc_resample: nearest upsample needs ho = h * s, wo = w * s (s=%d)", a->s);
  } else {
    KAD_CHECK_ARG(a->k >= 1 && a->s >= 1 && a->p >= 0 && 2 * a->p <= a->k,
                  "kad_nhwc_resample: bad pool k=%d s=%d p=%d", a->k, a->s, a->p);
    KAD_CHECK_ARG(a->ho == (a->h + 2 * a->p - a->k) / a->s + 1 && a->wo == (a->w + 2 * a->p - a->k) / a->s + 1,
                  "kad_nhwc_resample: output %dx%d does not match the pool of %dx%d", a->ho, a->wo, a->h, a->w);
  }
  hipStream_t st = (hipStream_t)stream;
  switch (a->dtype) {
    case KAD_F32: return dispatch_resample<float>(*a, st);
    case KAD_F16: return dispatch_resample<half_t>(*a, st);
    case KAD_BF16: return dispatch_resample<bf16_t>(*a, st);
    default: return fail(KAD_EINVAL, "kad_nhwc_resample: unknown dtype %d", a->dtype);
  }
}

extern "C" int kad_ddetect_decode(const kad_decode_args* a, void* stream) {
  KAD_CHECK_ARG(a && a->out, "kad_ddetect_decode: null pointer");
  KAD_CHECK_ARG(a->n > 0 && a->nl >= 1 && a->nl <= KAD_MAX_LEVELS && a->nc >= 0 && a->reg_max >= 1 &&
                    a->box_ch >= 4 * a->reg_max,
                "kad_ddetect_decode: bad n=%d nl=%d nc=%d reg_max=%d box_ch=%d", a->n, a->nl, a->nc, a->reg_max,
                a->box_ch);
  int total = 0;
  for (int l = 0; l < a->nl; ++l) {
    KAD_CHECK_ARG(a->head[l] && a->lh[l] > 0 && a->lw[l] > 0 && a->head_cs[l] >= a->box_ch + a->nc,
                  "kad_ddetect_decode: level %d: bad map or channel stride", l);
    KAD_CHECK_ARG(a->anchor_off[l] == total, "kad_ddetect_decode: anchor_off[%d] = %d, expected %d", l,
                  a->anchor_off[l], total);
    total += a->lh[l] * a->lw[l];
  }
  const int64_t threads = (int64_t)a->n * total;
  KAD_CHECK_ARG(threads < (1ll << 31), "kad_ddetect_decode: too many anchors");
  hipStream_t st = (hipStream_t)stream;
  const int blocks = (int)((threads + 255) / 256);
  const int V = a->dtype == KAD_F32 ? 4 : 8;  // elements per 16-byte piece
  bool vec = a->reg_max == 16 && a->box_ch % V == 0;
  for (int l = 0; l < a->nl; ++l) vec = vec && a->head_cs[l] % V == 0 && ((uintptr_t)a->head[l] & 15) == 0;
  switch (a->dtype) {
    case KAD_F32:
      if (vec) hipLaunchKernelGGL(ddetect_decode_vec_kernel<float>, dim3(blocks), dim3(256), 0, st, *a, total);
      else hipLaunchKernelGGL(ddetect_decode_kernel<float>, dim3(blocks), dim3(256), 0, st, *a, total);
      break;
    case KAD_F16:
      if (vec) hipLaunchKernelGGL(ddetect_decode_vec_kernel<half_t>, dim3(blocks), dim3(256), 0, st, *a, total);
      else hipLaunchKernelGGL(ddetect_decode_kernel<half_t>, dim3(blocks), dim3(256), 0, st, *a, total);
      break;
    case KAD_BF16:
      if (vec) hipLaunchKernelGGL(ddetect_decode_vec_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st, *a, total);
      else hipLaunchKernelGGL(ddetect_decode_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st, *a, total);
      break;
    default: return fail(KAD_EINVAL, "kad_ddetect_decode: unknown dtype %d", a->dtype);
  }
  return check_launch("kad_ddetect_decode");
}

extern "C" int64_t kad_nms_mask_words(int n) {
  if (n <= 0) return 0;
  return (int64_t)n * ((n + 63) / 64);
}

extern "C" int kad_nms(const float* boxes, unsigned long long* mask, unsigned char* keep, int n, float iou_thr,
                       void* stream) {
  KAD_CHECK_ARG(boxes && mask && keep, "kad_nms: null pointer");
  KAD_CHECK_ARG(n > 0 && n <= KAD_NMS_MAX, "kad_nms: n=%d outside [1, %d]", n, KAD_NMS_MAX);
  const int nw = (n + 63) / 64;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(nms_mask_kernel, dim3(nw, nw), dim3(64), 0, st, boxes, mask, n, nw, iou_thr);
  int rc = check_launch("kad_nms (mask)");
  if (rc) return rc;
  const size_t lds = (size_t)nw * sizeof(unsigned long long);
  hipLaunchKernelGGL(nms_sweep_kernel, dim3(1), dim3(NMS_SWEEP), lds, st, mask, keep, n, nw);
  return check_launch("kad_nms (sweep)");
}
