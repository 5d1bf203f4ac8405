// Squeeze-excitation (channel attention) and the branch merge.
//
// SE as in KADConv's channel selection (KAD-Conv/kadconv/kad_conv.py:105-109,117):
//   att[n, c] = sigmoid( W2 relu( W1 mean_hw(y[n, c]) + b1 ) + b2 ),  y *= att.
// The reference computes the mean with atomics inside its DCN kernel
// (acceleration/kadc_dcn16_kernel.cu:270-300) and the MLP in Triton
// (acceleration/kadc_fused_sm75.py:1518-1542).  Here the mean comes from
// deterministic per-tile partial sums (written by kad_dcn_fwd or by
// kad_se_pool) reduced in a fixed order inside kad_se_mlp.
//
// Branch merge (kad_conv.py:118-121): out = cat_i( att_i * upsample_i(z_i) ) + x,
// with PyTorch's bilinear align_corners=False rule (acceleration/kadc_fused_sm75.py:1245-1286
// restates it): src = (dst + 0.5) * in / out - 0.5, clamped below at 0,
// i0 = floor(src), i1 = min(i0 + 1, in - 1).  The same kernel, with a per-branch
// scalar coefficient, an all-channel span and a per-channel output gate,
// computes the builder-defined KADDown mixture.
#include "kad_common.h"

#include <type_traits>

namespace kad {

// ---- SE pool: per-(n, c) plane means, one wave per plane (NCHW) ----------------------------
template <typename T>
__global__ __launch_bounds__(256) void se_pool_nchw_kernel(const T* x, float* g, int planes, int hw) {
  const int wave = (blockIdx.x * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= planes) return;
  const T* p = x + (int64_t)wave * hw;
  float acc = 0.f;
  for (int i = lane; i < hw; i += 64) acc += to_f32(p[i]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) g[wave] = acc;
}

// NCHW over the flat tensor in 16-byte pieces (any plane size hw >= 8, which a
// piece then straddles at most once): wave w sums planes [4 w, 4 w + 4).  Each
// lane splits a piece at its plane boundary and adds the parts to the plane's
// running sum; sums are then wave-reduced (fixed order: deterministic).
template <typename T>
__global__ __launch_bounds__(256) void se_pool_flat_kernel(const T* x, float* g, int planes, int hw) {
  typedef T t8 __attribute__((ext_vector_type(8)));
  const int wv = (blockIdx.x * 256 + threadIdx.x) >> 6, lane = threadIdx.x & 63;
  const int pb = wv * 4;
  if (pb >= planes) return;
  const int pe = pb + 4 < planes ? pb + 4 : planes;
  const int v_lo = pb * hw / 8, v_hi = (pe * hw + 7) / 8;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  // batches of KU pieces per lane: every load of a batch is issued before the first use
  constexpr int KU = 8;
  for (int vb = v_lo + lane; vb < v_hi; vb += 64 * KU) {
    t8 xv[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u)
      if (vb + 64 * u < v_hi) xv[u] = *(const t8*)(x + (vb + 64 * u) * 8);
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int v = vb + 64 * u;
      if (v >= v_hi) continue;
      const int e0 = v * 8;
      const int p0 = e0 / hw, nb = (p0 + 1) * hw - e0;  // elements of the piece in plane p0
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float xk = to_f32(xv[u][k]);
        if (k < nb) s0 += xk; else s1 += xk;
      }
      const int k0 = p0 - pb;  // -1 .. 3; parts of planes outside [pb, pe) belong to other waves
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[k] += (k == k0 ? s0 : 0.f) + (k == k0 + 1 ? s1 : 0.f);
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float v = acc[k];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0 && pb + k < pe) g[pb + k] = v;
  }
}

// NHWC: grid (ceil(P / 256), N); block partial sums over 256 pixels per channel.
template <typename T>
__global__ __launch_bounds__(256) void se_pool_nhwc_kernel(const T* x, float* part, int c, int P, int cs,
                                                          int tiles) {
  const int n = blockIdx.y, t = blockIdx.x;
  const int p0 = t * 256, p1 = (p0 + 256 < P) ? p0 + 256 : P;
  for (int ch = threadIdx.x; ch < c; ch += 256) {
    float acc = 0.f;
    for (int p = p0; p < p1; ++p) acc += to_f32(x[((int64_t)n * P + p) * cs + ch]);
    part[((int64_t)n * tiles + t) * c + ch] = acc;
  }
}

// ---- SE MLP: one block per image ---------------------------------------------------------
// partial: [N][tiles][C] sums (tiles = 1 for plane sums); mean = sum * inv_count.
// Small C (everything fits the 160 KB of LDS, KADConv's branches): 512 threads,
// one round of up to 32 loads per thread brings the image's partials and both
// weight matrices into LDS.  Slots past the end load a clamped (valid) address
// and are dropped at the store, so the loads carry no branches and all are in
// flight together.  W2 goes to LDS as [C][hid + 1] (row stride odd: a thread
// per channel reads its row without bank conflicts).  Then, from LDS: tile
// sums (nsl = 512 / C slices per channel, 4 chains each, slices combined in a
// fixed order), the hidden layer (8 threads per unit, shuffle-reduced) and the
// output layer (one thread per channel).
constexpr int SE_MAXLD = 32;   // loads in flight per thread per round
constexpr int SE_ST = 512;     // threads of the staged kernel

__global__ __launch_bounds__(SE_ST) void se_mlp_staged_kernel(const float* partial, int tiles, float inv_count,
                                                             const float* w1, const float* b1, const float* w2,
                                                             const float* b2, float* att, int c, int hid) {
  extern __shared__ float lds[];
  const int nsl = c < SE_ST ? SE_ST / c : 1;
  float* g = lds;                  // [C]
  float* hbuf = g + c;             // [hid]
  float* red = hbuf + hid;         // [nsl][C]
  float* sp = red + nsl * c;       // [tiles][C]
  float* sw1 = sp + tiles * c;     // [hid][C] (right behind sp: one contiguous copy)
  float* sw2 = sw1 + hid * c;      // [C][hid + 1]
  const int n = blockIdx.x, tid = threadIdx.x;
  const float* pn = partial + (int64_t)n * tiles * c;
  const int np = tiles * c, nw = hid * c, ntot = np + 2 * nw;
  const float inv_hid = 1.f / (float)hid;
  for (int b0 = 0; b0 < ntot; b0 += SE_MAXLD * SE_ST) {
    float v[SE_MAXLD];
#pragma unroll
    for (int u = 0; u < SE_MAXLD; ++u) {
      int e = b0 + tid + u * SE_ST;
      e = e < ntot ? e : ntot - 1;
      const float* src = e < np ? pn + e : e < np + nw ? w1 + (e - np) : w2 + (e - np - nw);
      v[u] = *src;
    }
#pragma unroll
    for (int u = 0; u < SE_MAXLD; ++u) {
      const int e = b0 + tid + u * SE_ST;
      if (e < np + nw) {
        sp[e] = v[u];
      } else if (e < ntot) {  // w2 [C][hid] -> [C][hid + 1]
        const int f = e - np - nw, ch = (int)(((float)f + 0.5f) * inv_hid), j = f - ch * hid;
        sw2[ch * (hid + 1) + j] = v[u];
      }
    }
  }
  __syncthreads();
  for (int e = tid; e < nsl * c; e += SE_ST) {
    const int ch = e % c, s = e / c;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int t = s;
    for (; t + 3 * nsl < tiles; t += 4 * nsl) {
      s0 += sp[t * c + ch];
      s1 += sp[(t + nsl) * c + ch];
      s2 += sp[(t + 2 * nsl) * c + ch];
      s3 += sp[(t + 3 * nsl) * c + ch];
    }
    for (; t < tiles; t += nsl) s0 += sp[t * c + ch];
    red[s * c + ch] = (s0 + s1) + (s2 + s3);
  }
  __syncthreads();
  for (int ch = tid; ch < c; ch += SE_ST) {
    float v = 0.f;
    for (int s = 0; s < nsl; ++s) v += red[s * c + ch];
    g[ch] = v * inv_count;
  }
  __syncthreads();
  // hidden unit j: 8 threads, strided channel slices, shuffle-reduced
  for (int j0 = 0; j0 < hid; j0 += SE_ST / 8) {
    const int j = j0 + (tid >> 3), part = tid & 7;
    float a0 = 0.f, a1 = 0.f;
    if (j < hid) {
      int ch = part;
      for (; ch + 8 < c; ch += 16) {
        a0 += sw1[j * c + ch] * g[ch];
        a1 += sw1[j * c + ch + 8] * g[ch + 8];
      }
      for (; ch < c; ch += 8) a0 += sw1[j * c + ch] * g[ch];
    }
    float acc = a0 + a1;
    acc += __shfl_xor(acc, 1);
    acc += __shfl_xor(acc, 2);
    acc += __shfl_xor(acc, 4);
    if (j < hid && part == 0) hbuf[j] = fmaxf(acc + (b1 ? b1[j] : 0.f), 0.f);
  }
  __syncthreads();
  for (int ch = tid; ch < c; ch += SE_ST) {
    const float* wr = sw2 + ch * (hid + 1);
    float a[4] = {b2 ? b2[ch] : 0.f, 0.f, 0.f, 0.f};
    int j = 0;
    for (; j + 4 <= hid; j += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] += wr[j + u] * hbuf[j + u];
    }
    for (; j < hid; ++j) a[0] += wr[j] * hbuf[j];
    att[(int64_t)n * c + ch] = sigmoidf_((a[0] + a[1]) + (a[2] + a[3]));
  }
}

// Large C (the staged copy would not fit): NT threads (256 for C <= 256, 1024
// above: a small block starts sooner next to concurrent kernels, a large one
// keeps more weight loads in flight); three phases, each issuing its loads back to back so that a phase costs a few
// memory round trips, not one per element:
//  1. g[c] = inv_count * (sum over tiles): nsl = NT / C tile slices per
//     channel when C < NT, 8 independent chains each, slices combined in a
//     fixed order (deterministic);
//  2. h[j] = relu(b1[j] + W1[j] . g): each wave takes 8 hidden units at a
//     time, lanes along channels (coalesced W1 rows, 4 channel steps unrolled:
//     32 loads in flight per lane), shuffle-reduced;
//  3. att[c] = sigmoid(b2[c] + W2[c] . h): one thread per channel, its W2 row
//     in 16-byte pieces (rows 16-byte aligned) issued before the products.
constexpr int SE_UJ = 8;  // hidden units per wave per round

template <int NT>
__global__ __launch_bounds__(NT) void se_mlp_kernel(const float* partial, int tiles, float inv_count,
                                                   const float* w1, const float* b1, const float* w2,
                                                   const float* b2, float* att, int c, int hid) {
  extern __shared__ float lds[];
  float* g = lds;           // [C]
  float* hbuf = g + c;      // [hid]
  float* red = hbuf + hid;  // [nsl][C] slice sums
  const int n = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int NWV = NT / 64;
  const float* pn = partial + (int64_t)n * tiles * c;
  const int nsl = c < NT ? NT / c : 1;
  // ---- 1. channel means ----
  for (int base = 0; base < c * nsl; base += NT) {
    const int e = base + tid;
    if (e < c * nsl) {
      const int ch = e % c, s = e / c;
      float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      int t = s;
      for (; t + 7 * nsl < tiles; t += 8 * nsl) {
#pragma unroll
        for (int u = 0; u < 8; ++u) a[u] += pn[(int64_t)(t + u * nsl) * c + ch];
      }
      for (int u = 0; t < tiles; t += nsl, ++u) a[u & 7] += pn[(int64_t)t * c + ch];
      red[s * c + ch] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    }
  }
  __syncthreads();
  for (int ch = tid; ch < c; ch += NT) {
    float v = 0.f;
    for (int s = 0; s < nsl; ++s) v += red[s * c + ch];
    g[ch] = v * inv_count;
  }
  __syncthreads();
  // ---- 2. hidden layer ----
  for (int j0 = wave * SE_UJ; j0 < hid; j0 += NWV * SE_UJ) {
    float acc[SE_UJ];
#pragma unroll
    for (int u = 0; u < SE_UJ; ++u) acc[u] = 0.f;
    int ch = lane;
    for (; ch + 192 < c; ch += 256) {  // 4 channel steps: 32 loads in flight
      float wv[4][SE_UJ];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < SE_UJ; ++u) wv[q][u] = j0 + u < hid ? w1[(int64_t)(j0 + u) * c + ch + 64 * q] : 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float gv = g[ch + 64 * q];
#pragma unroll
        for (int u = 0; u < SE_UJ; ++u) acc[u] += wv[q][u] * gv;
      }
    }
    for (; ch < c; ch += 64) {
      const float gv = g[ch];
#pragma unroll
      for (int u = 0; u < SE_UJ; ++u)
        if (j0 + u < hid) acc[u] += w1[(int64_t)(j0 + u) * c + ch] * gv;
    }
#pragma unroll
    for (int u = 0; u < SE_UJ; ++u) {
      float v = acc[u];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
      if (lane == 0 && j0 + u < hid) hbuf[j0 + u] = fmaxf(v + (b1 ? b1[j0 + u] : 0.f), 0.f);
    }
  }
  __syncthreads();
  // ---- 3. output layer ----
  const bool vec = (hid & 3) == 0 && ((uintptr_t)w2 & 15) == 0;
  for (int ch = tid; ch < c; ch += NT) {
    const float* wr = w2 + (int64_t)ch * hid;
    float a[4] = {b2 ? b2[ch] : 0.f, 0.f, 0.f, 0.f};
    int j = 0;
    if (vec) {
      for (; j + 16 <= hid; j += 16) {  // four 16-byte pieces in flight
        floatx4 wq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) wq[q] = *(const floatx4*)(wr + j + 4 * q);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int u = 0; u < 4; ++u) a[u] += wq[q][u] * hbuf[j + 4 * q + u];
      }
    }
    for (; j < hid; ++j) a[j & 3] += wr[j] * hbuf[j];
    att[(int64_t)n * c + ch] = sigmoidf_((a[0] + a[1]) + (a[2] + a[3]));
  }
}

// Wide C (C <= 1024, C % 64 == 0, hid <= 64, hid % 4 == 0, 16-byte aligned
// weights): every weight load of a layer in one batch.  1024 threads:
//  - thread (j = tid / 16, part = tid % 16) requests its W1 row slice
//    W1[j][64 i + 4 part .. + 4] (C / 64 16-byte pieces) first, so the W1
//    round trip overlaps the channel means;
//  - g[c] = inv_count * sum over tiles (thread c, tiles in index order);
//  - h[j] = relu(b1[j] + W1[j] . g): 16 lanes per unit, shuffle-reduced;
//  - thread c requests its W2 row (hid / 4 pieces) right after its W1 products,
//    then att[c] = sigmoid(b2[c] + W2[c] . h).
constexpr int SE_WIDE = 1024;

__global__ __launch_bounds__(SE_WIDE) void se_mlp_wide_kernel(const float* partial, int tiles, float inv_count,
                                                              const float* w1, const float* b1, const float* w2,
                                                              const float* b2, float* att, int c, int hid) {
  __shared__ __align__(16) float g[SE_WIDE];
  __shared__ __align__(16) float hb[64];
  const int n = blockIdx.x, tid = threadIdx.x;
  const int j = tid >> 4, part = tid & 15, np = c / 64;
  floatx4 wv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    wv[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (i < np && j < hid) wv[i] = *(const floatx4*)(w1 + (int64_t)j * c + 64 * i + 4 * part);
  }
  if (tid < c) {
    const float* pn = partial + (int64_t)n * tiles * c + tid;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int t = 0;
    for (; t + 3 < tiles; t += 4) {
      a0 += pn[(int64_t)t * c];
      a1 += pn[(int64_t)(t + 1) * c];
      a2 += pn[(int64_t)(t + 2) * c];
      a3 += pn[(int64_t)(t + 3) * c];
    }
    for (; t < tiles; ++t) a0 += pn[(int64_t)t * c];
    g[tid] = ((a0 + a1) + (a2 + a3)) * inv_count;
  }
  __syncthreads();
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i < np) {
      const floatx4 gv = *(const floatx4*)&g[64 * i + 4 * part];
      acc += (wv[i][0] * gv[0] + wv[i][1] * gv[1]) + (wv[i][2] * gv[2] + wv[i][3] * gv[3]);
    }
  }
  // W2 row of channel tid (the W1 registers are free now)
  const int nq = hid / 4;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    wv[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (i < nq && tid < c) wv[i] = *(const floatx4*)(w2 + (int64_t)tid * hid + 4 * i);
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 4);
  acc += __shfl_xor(acc, 8);
  if (part == 0 && j < hid) hb[j] = fmaxf(acc + (b1 ? b1[j] : 0.f), 0.f);
  __syncthreads();
  if (tid < c) {
    float o0 = b2 ? b2[tid] : 0.f, o1 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i < nq) {
        const floatx4 hv = *(const floatx4*)&hb[4 * i];
        o0 += wv[i][0] * hv[0] + wv[i][1] * hv[1];
        o1 += wv[i][2] * hv[2] + wv[i][3] * hv[3];
      }
    }
    att[(int64_t)n * c + tid] = sigmoidf_(o0 + o1);
  }
}

// ---- channel scale: out[n, c, :] = x[n, c, :] * att[n, c] (NCHW) or per pixel (NHWC) -------
// NCHW over the flat tensor in 16-byte pieces (hw >= 8): the plane of a piece's
// first element gives its scale; a piece straddles at most one plane boundary.
template <typename T>
__global__ __launch_bounds__(256) void channel_scale_flat_kernel(const T* x, const float* att, T* out, int nvec,
                                                                int hw) {
  typedef T t8 __attribute__((ext_vector_type(8)));
  for (int v = blockIdx.x * 256 + threadIdx.x; v < nvec; v += gridDim.x * 256) {
    const int e0 = v * 8;
    const int p0 = e0 / hw, nb = (p0 + 1) * hw - e0;  // elements of the piece in plane p0 (att index = plane)
    const float s0 = att[p0], s1 = nb < 8 ? att[p0 + 1] : s0;
    const t8 xv = *(const t8*)(x + e0);
    t8 o;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = from_f32<T>(to_f32(xv[k]) * (k < nb ? s0 : s1));
    *(t8*)(out + e0) = o;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void channel_scale_kernel(const T* x, const float* att, T* out, int64_t total,
                                                           int c, int hw, int layout, int cs) {
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int64_t n, ch;
    if (layout == KAD_NCHW) {
      ch = (i / hw) % c;
      n = i / ((int64_t)hw * c);
    } else {
      ch = i % cs;
      n = i / ((int64_t)hw * cs);
      if (ch >= c) { out[i] = x[i]; continue; }
    }
    out[i] = from_f32<T>(to_f32(x[i]) * att[n * c + ch]);
  }
}

// ---- branch merge ------------------------------------------------------------------------
// Per-branch source rows for output row y (same for every column and channel).
struct RowSrc { int y0, y1; float ly; };

__device__ __forceinline__ RowSrc row_src(const kad_merge_args& a, int b, int y) {
  RowSrc r;
  src_index(y, a.br_h[b], a.h, (float)a.br_h[b] / (float)a.h, r.y0, r.y1, r.ly);
  return r;
}

constexpr int MG_XS = 64;   // output columns per block (NCHW path)
constexpr int MG_CH = 16;   // output channels per block (NCHW path)
constexpr int MG_SX = MG_XS + 2;  // staged source columns per branch row (upsampling only shrinks spans)

// NCHW output.  Block = (64 columns, one row, 16 channels, image).  The source
// rows of every branch that owns one of the 16 channels are staged in LDS
// (reads run along channels, the NHWC contiguous axis); outputs are then
// written along x (the NCHW contiguous axis).  Thread t takes column t & 63 and
// channels (t >> 6) + 4k, so the column interpolation is computed once per
// thread and reused for its four channels.
template <typename T>
__global__ __launch_bounds__(256) void merge_nchw_kernel(kad_merge_args a) {
  __shared__ float lds[KAD_MAX_BRANCHES][2][MG_SX][MG_CH + 1];
  __shared__ float s_scale[KAD_MAX_BRANCHES][MG_CH], s_gate[MG_CH];
  __shared__ int s_owner[MG_CH];  // bit b set: branch b covers this channel
  const int tid = threadIdx.x;
  const int xb = blockIdx.x * MG_XS;
  const int y = blockIdx.y;
  const int nch = ceil_div(a.c_end - a.c_begin, MG_CH);
  const int c0 = a.c_begin + (blockIdx.z % nch) * MG_CH;
  const int n = blockIdx.z / nch;
  const int xe = (xb + MG_XS < a.w) ? xb + MG_XS : a.w;
  int sx_lo[KAD_MAX_BRANCHES];
  float ly[KAD_MAX_BRANCHES];
  if (tid < MG_CH) {
    const int c = c0 + tid;
    int owner = 0;
#pragma unroll
    for (int b = 0; b < KAD_MAX_BRANCHES; ++b) {
      float sc = 0.f;
      if (b < a.nbranch && c < a.c_end) {
        const int cb = c - a.br_c_off[b];
        if (cb >= 0 && cb < a.br_c[b]) {
          owner |= 1 << b;
          sc = a.br_coeff[b] * (a.br_att[b] ? a.br_att[b][(int64_t)n * a.br_c[b] + cb] : 1.f);
        }
      }
      s_scale[b][tid] = sc;
    }
    s_owner[tid] = owner;
    s_gate[tid] = (a.gate && c < a.c_end) ? a.gate[c] : 1.f;
  }
#pragma unroll
  for (int b = 0; b < KAD_MAX_BRANCHES; ++b) {
    sx_lo[b] = 0;
    ly[b] = 0.f;
    if (b >= a.nbranch) continue;
    const int lo = a.br_c_off[b], hi = a.br_c_off[b] + a.br_c[b];
    if (hi <= c0 || lo >= c0 + MG_CH) continue;  // branch owns none of these channels
    const RowSrc r = row_src(a, b, y);
    ly[b] = r.ly;
    int x0a, x1a, x0b, x1b;
    float l;
    const float sc = (float)a.br_w[b] / (float)a.w;
    src_index(xb, a.br_w[b], a.w, sc, x0a, x1a, l);
    src_index(xe - 1, a.br_w[b], a.w, sc, x0b, x1b, l);
    sx_lo[b] = x0a;
    const int nsx = x1b - x0a + 1;  // <= MG_SX
    const T* z = (const T*)a.br_z[b];
    const int cl = tid & (MG_CH - 1);
    const int cb = c0 + cl - lo;
    const bool ok = cb >= 0 && cb < a.br_c[b];
    const T* zr0 = z + (((int64_t)n * a.br_h[b] + r.y0) * a.br_w[b] + x0a) * a.br_cs[b] + cb;
    const T* zr1 = z + (((int64_t)n * a.br_h[b] + r.y1) * a.br_w[b] + x0a) * a.br_cs[b] + cb;
    for (int q = tid >> 4; q < 2 * nsx; q += 256 / MG_CH) {
      const int rr = q >= nsx ? 1 : 0;
      const int sx = q - rr * nsx;
      lds[b][rr][sx][cl] = ok ? to_f32((rr ? zr1 : zr0)[(int64_t)sx * a.br_cs[b]]) : 0.f;
    }
  }
  __syncthreads();
  const int x = xb + (tid & 63);
  if (x >= a.w) return;
  int x0[KAD_MAX_BRANCHES], x1[KAD_MAX_BRANCHES];
  float lx[KAD_MAX_BRANCHES];
#pragma unroll
  for (int b = 0; b < KAD_MAX_BRANCHES; ++b) {
    x0[b] = x1[b] = 0;
    lx[b] = 0.f;
    if (b < a.nbranch) {
      src_index(x, a.br_w[b], a.w, (float)a.br_w[b] / (float)a.w, x0[b], x1[b], lx[b]);
      x0[b] -= sx_lo[b];
      x1[b] -= sx_lo[b];
    }
  }
  const T* res = (const T*)a.residual;
#pragma unroll
  for (int k = 0; k < MG_CH / 4; ++k) {
    const int cl = (tid >> 6) + 4 * k;
    const int c = c0 + cl;
    if (c >= a.c_end) continue;
    const int64_t oi = (((int64_t)n * a.c + c) * a.h + y) * a.w + x;
    float v = res ? to_f32(res[oi]) : 0.f;
    const int owner = s_owner[cl];
#pragma unroll
    for (int bb = 0; bb < KAD_MAX_BRANCHES; ++bb) {
      if (!(owner & (1 << bb))) continue;
      const float top = lds[bb][0][x0[bb]][cl] + lx[bb] * (lds[bb][0][x1[bb]][cl] - lds[bb][0][x0[bb]][cl]);
      const float bot = lds[bb][1][x0[bb]][cl] + lx[bb] * (lds[bb][1][x1[bb]][cl] - lds[bb][1][x0[bb]][cl]);
      v += s_scale[bb][cl] * (top + ly[bb] * (bot - top));
    }
    ((T*)a.out)[oi] = from_f32<T>(v * s_gate[cl]);
  }
}

// NCHW output, branches with disjoint channel ranges (KADConv's concat).
// Block = (output row, 32-channel chunk of one branch, image).  Every global
// load of the block is issued in one round: the chunk's one or two source rows
// of the branch map (16-byte pieces of 8 channels, NHWC) and its 32 residual
// rows (8-byte pieces) go to LDS; the outputs are then formed four columns per
// task and written with 8-byte stores.
template <typename T>
__global__ __launch_bounds__(256) void merge_rows_kernel(kad_merge_args a) {
  extern __shared__ __align__(16) char dsm[];
  constexpr int ZS = 40;                     // T per staged source pixel (32 channels + 8 pad)
  const int y = blockIdx.x, chunk = blockIdx.y, n = blockIdx.z;
  const int tid = threadIdx.x;
  int b = 0, k = chunk;
#pragma unroll
  for (int i = 0; i < KAD_MAX_BRANCHES; ++i) {
    if (i == b && i < a.nbranch - 1) {
      const int nc = ceil_div(a.br_c[i], 32);
      if (k >= nc) {
        k -= nc;
        b = i + 1;
      }
    }
  }
  const int cb0 = k * 32;
  const int nch = a.br_c[b] - cb0 < 32 ? a.br_c[b] - cb0 : 32;
  const int cbase = a.br_c_off[b] + cb0;
  const int bh = a.br_h[b], bw = a.br_w[b], cs = a.br_cs[b];
  const int W = a.w;
  const int W4 = ceil_div(W, 4);
  T* zs = (T*)dsm;                           // [2][bw][ZS]
  T* rs = zs + 2 * bw * ZS;                  // [32][W4 * 4]
  __shared__ float s_att[32], s_gate[32];
  const RowSrc r = row_src(a, b, y);
  const int nrow = (bh == a.h) ? 1 : 2;
  const T* z = (const T*)a.br_z[b] + (int64_t)n * bh * bw * cs + cb0;
  const T* res = (const T*)a.residual;
  const int npiece = ceil_div(nch, 8);       // 8-channel pieces that hold real channels
  const int zt = nrow * bw * 4;              // 16-byte source pieces (4 per pixel)
  const int rt = res ? nch * W4 : 0;         // 4-element residual pieces
  const int64_t rbase = (((int64_t)n * a.c + cbase) * a.h + y) * W;
  // one round of loads: up to 8 per thread in flight
  for (int e0 = tid; e0 < zt + rt; e0 += 8 * 256) {
    uint4 zv[8];
    uint2 rv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + u * 256;
      zv[u] = uint4{0u, 0u, 0u, 0u};
      rv[u] = uint2{0u, 0u};
      if (e < zt) {
        const int g = e & 3, q = e >> 2, rr = q >= bw ? 1 : 0, sx = q - rr * bw;
        if (g < npiece) {
          const T* src = z + ((int64_t)(rr ? r.y1 : r.y0) * bw + sx) * cs + g * 8;
          if constexpr (sizeof(T) == 2) zv[u] = *(const uint4*)src;
          else zv[u] = uint4{0u, 0u, 0u, 0u};  // fp32 path loads below
        }
      } else if (e < zt + rt) {
        const int f = e - zt, cl = f / W4, x4 = (f - cl * W4) * 4;
        const T* src = res + rbase + (int64_t)cl * a.h * W + x4;
        if constexpr (sizeof(T) == 2) {
          if (x4 + 4 <= W && ((uintptr_t)src & 7) == 0) {
            rv[u] = *(const uint2*)src;
          } else {
            unsigned short hv[4] = {0, 0, 0, 0};
            for (int j = 0; j < 4; ++j)
              if (x4 + j < W) hv[j] = __builtin_bit_cast(unsigned short, src[j]);
            rv[u] = uint2{hv[0] | ((unsigned)hv[1] << 16), hv[2] | ((unsigned)hv[3] << 16)};
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + u * 256;
      if (e < zt) {
        const int g = e & 3, q = e >> 2;
        T* d = zs + q * ZS + g * 8;
        if constexpr (sizeof(T) == 2) {
          *(uint4*)d = zv[u];
        } else {
          const int rr = q >= bw ? 1 : 0, sx = q - rr * bw;
          const T* src = z + ((int64_t)(rr ? r.y1 : r.y0) * bw + sx) * cs + g * 8;
          for (int j = 0; j < 8; ++j) d[j] = (g * 8 + j < nch) ? src[j] : from_f32<T>(0.f);
        }
      } else if (e < zt + rt) {
        const int f = e - zt, cl = f / W4, x4 = (f - cl * W4) * 4;
        T* d = rs + cl * W4 * 4 + x4;
        if constexpr (sizeof(T) == 2) {
          *(uint2*)d = rv[u];
        } else {
          const T* src = res + rbase + (int64_t)cl * a.h * W + x4;
          for (int j = 0; j < 4; ++j) d[j] = (x4 + j < W) ? src[j] : 0.f;
        }
      }
    }
  }
  if (tid < 32) {
    s_att[tid] = tid < nch ? a.br_coeff[b] * (a.br_att[b] ? a.br_att[b][(int64_t)n * a.br_c[b] + cb0 + tid] : 1.f)
                           : 0.f;
    s_gate[tid] = (a.gate && tid < nch) ? a.gate[cbase + tid] : 1.f;
  }
  __syncthreads();
  const float scale = (float)bw / (float)W;
  const int zr1 = (nrow == 2) ? bw * ZS : 0;
  T* out = (T*)a.out;
  for (int f = tid; f < nch * W4; f += 256) {
    const int cl = f / W4, x4 = (f - cl * W4) * 4;
    const float at = s_att[cl], gt = s_gate[cl];
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int x = x4 + j < W ? x4 + j : W - 1;
      int x0, x1;
      float lx;
      src_index(x, bw, W, scale, x0, x1, lx);
      const float t0 = to_f32(zs[x0 * ZS + cl]), t1 = to_f32(zs[x1 * ZS + cl]);
      const float u0 = to_f32(zs[zr1 + x0 * ZS + cl]), u1 = to_f32(zs[zr1 + x1 * ZS + cl]);
      const float top = t0 + lx * (t1 - t0), bot = u0 + lx * (u1 - u0);
      float o = at * (top + r.ly * (bot - top));
      if (res) o += to_f32(rs[cl * W4 * 4 + x4 + j]);
      v[j] = o * gt;
    }
    T* d = out + rbase + (int64_t)cl * a.h * W + x4;
    if (sizeof(T) == 2 && x4 + 4 <= W && ((uintptr_t)d & 7) == 0) {
      typedef T v4 __attribute__((ext_vector_type(4)));
      v4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = from_f32<T>(v[j]);
      *(v4*)d = o;
    } else {
      for (int j = 0; j < 4; ++j)
        if (x4 + j < W) d[j] = from_f32<T>(v[j]);
    }
  }
}

// NCHW output, branches with disjoint channel ranges, planes of a multiple of 8
// pixels, 16-byte aligned tensors.  Block = (8-channel group of one branch, run
// of MB_E consecutive pixels of the plane, image): the residual reads and the
// output writes are 16-byte vectors over contiguous 2 KB runs of each of the 8
// planes.  The branch-map rows that the run's output rows sample (NHWC, one
// 16-byte piece = the group's 8 channels of a pixel) are staged first, as
// planar fp32 [8][rows][bw], so the interpolation reads consecutive addresses.
constexpr int MB_E = 1024;

template <typename T>
__global__ __launch_bounds__(256) void merge_band_kernel(kad_merge_args a, int srows_cap, int bw_cap, int nruns,
                                                         int ngroups, int grid8) {
  extern __shared__ float zsm[];  // [8][srows_cap][bw_cap]
  __shared__ float s_att[8], s_gate[8];
  typedef T v8 __attribute__((ext_vector_type(8)));
  // XCD-aware order: XCD b % 8 takes a contiguous run of (image, group, run) tiles, so the
  // runs of one plane (which share boundary lines and source rows) stay in one L2
  const int bq = (int)(blockIdx.x & 7) * (grid8 >> 3) + (int)(blockIdx.x >> 3);
  if (bq >= nruns * ngroups * a.n) return;  // whole block, before the barrier
  const int run = bq % nruns, rq = bq / nruns, n = rq / ngroups, tid = threadIdx.x;
  int b = 0, k = rq % ngroups;
#pragma unroll
  for (int i = 0; i < KAD_MAX_BRANCHES; ++i) {
    if (i == b && i < a.nbranch - 1) {
      const int ng = ceil_div(a.br_c[i], 8);
      if (k >= ng) {
        k -= ng;
        b = i + 1;
      }
    }
  }
  const int cb0 = k * 8;
  const int nch = a.br_c[b] - cb0 < 8 ? a.br_c[b] - cb0 : 8;
  const int cbase = a.br_c_off[b] + cb0;
  const int H = a.h, W = a.w, P = H * W;
  const int bh = a.br_h[b], bw = a.br_w[b], cs = a.br_cs[b];
  const int f0 = run * MB_E, f1 = P - f0 < MB_E ? P : f0 + MB_E;
  const float inv_w = 1.f / (float)W;
  const int ya = (int)(((float)f0 + 0.5f) * inv_w), yb = (int)(((float)(f1 - 1) + 0.5f) * inv_w);
  const RowSrc ra = row_src(a, b, ya), rb = row_src(a, b, yb);
  const int sy_lo = ra.y0;
  int srows = rb.y1 - sy_lo + 1;
  srows = srows < srows_cap ? srows : srows_cap;  // the host sizes srows_cap for the longest run
  const T* z = (const T*)a.br_z[b] + (int64_t)n * bh * bw * cs + cb0;
  for (int e = tid; e < srows * bw; e += 256) {
    const int r = e / bw, sx = e - r * bw;
    const v8 v = *(const v8*)(z + ((int64_t)(sy_lo + r) * bw + sx) * cs);
#pragma unroll
    for (int j = 0; j < 8; ++j) zsm[(j * srows_cap + r) * bw_cap + sx] = to_f32(v[j]);
  }
  if (tid < 8) {
    s_att[tid] = tid < nch ? a.br_coeff[b] * (a.br_att[b] ? a.br_att[b][(int64_t)n * a.br_c[b] + cb0 + tid] : 1.f)
                           : 0.f;
    s_gate[tid] = (a.gate && tid < nch) ? a.gate[cbase + tid] : 1.f;
  }
  __syncthreads();
  const float sh = (float)bh / (float)H, sw = (float)bw / (float)W;
  const T* res = (const T*)a.residual;
  T* out = (T*)a.out;
  constexpr int VPP = MB_E / 8;  // vectors per plane and run
  for (int q = tid; q < 8 * VPP; q += 256) {
    const int cl = q / VPP, f = f0 + (q - cl * VPP) * 8;
    if (cl >= nch || f >= f1) continue;
    const int64_t pb = ((int64_t)n * a.c + cbase + cl) * P + f;
    v8 rv;
    if (res) rv = *(const v8*)(res + pb);
    const float at = s_att[cl], gt = s_gate[cl];
    const float* zp = zsm + cl * srows_cap * bw_cap;
    int y = (int)(((float)f + 0.5f) * inv_w), x = f - y * W;
    int y0, y1;
    float ly;
    src_index(y, bh, H, sh, y0, y1, ly);
    v8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (x == W) {  // next output row
        x = 0;
        ++y;
        src_index(y, bh, H, sh, y0, y1, ly);
      }
      int x0, x1;
      float lx;
      src_index(x, bw, W, sw, x0, x1, lx);
      const float* r0 = zp + (y0 - sy_lo) * bw_cap;
      const float* r1 = zp + (y1 - sy_lo) * bw_cap;
      const float top = r0[x0] + lx * (r0[x1] - r0[x0]);
      const float bot = r1[x0] + lx * (r1[x1] - r1[x0]);
      float v = at * (top + ly * (bot - top));
      if (res) v += to_f32(rv[j]);
      o[j] = from_f32<T>(v * gt);
      ++x;
    }
    *(v8*)(out + pb) = o;
  }
}

// NHWC output: block = (one row, image); threads run along channels, so every
// read (branch maps, residual) and the write are contiguous.
template <typename T>
__global__ __launch_bounds__(256) void merge_nhwc_kernel(kad_merge_args a) {
  const int y = blockIdx.x, n = blockIdx.y;
  RowSrc rs[KAD_MAX_BRANCHES];
  for (int b = 0; b < a.nbranch; ++b) rs[b] = row_src(a, b, y);
  const int cw = a.c_end - a.c_begin;
  for (int e = threadIdx.x; e < a.w * cw; e += 256) {
    const int c = a.c_begin + e % cw, x = e / cw;
    const int64_t pix = ((int64_t)n * a.h + y) * a.w + x;
    const int64_t oi = pix * a.out_cs + c;
    float v = a.residual ? to_f32(((const T*)a.residual)[pix * a.res_cs + c]) : 0.f;
    for (int b = 0; b < a.nbranch; ++b) {
      const int cb = c - a.br_c_off[b];
      if (cb < 0 || cb >= a.br_c[b]) continue;
      int x0, x1;
      float lx;
      src_index(x, a.br_w[b], a.w, (float)a.br_w[b] / (float)a.w, x0, x1, lx);
      const T* z = (const T*)a.br_z[b] + (int64_t)n * a.br_h[b] * a.br_w[b] * a.br_cs[b] + cb;
      const int bw = a.br_w[b], cs = a.br_cs[b];
      const float v00 = to_f32(z[((int64_t)rs[b].y0 * bw + x0) * cs]);
      const float v01 = to_f32(z[((int64_t)rs[b].y0 * bw + x1) * cs]);
      const float v10 = to_f32(z[((int64_t)rs[b].y1 * bw + x0) * cs]);
      const float v11 = to_f32(z[((int64_t)rs[b].y1 * bw + x1) * cs]);
      float s = (1.f - rs[b].ly) * ((1.f - lx) * v00 + lx * v01) + rs[b].ly * ((1.f - lx) * v10 + lx * v11);
      if (a.br_att[b]) s *= a.br_att[b][(int64_t)n * a.br_c[b] + cb];
      v += a.br_coeff[b] * s;
    }
    if (a.gate) v *= a.gate[c];
    ((T*)a.out)[oi] = from_f32<T>(v);
  }
}

// NHWC output, channel window and pixel strides multiples of 8.  A block takes 64 pixels with one wave
// per 8-channel group (up to 8 waves; wave w takes groups w, w + 8, ...), a lane per pixel, so the group -- which branches cover it,
// at which channel offset -- is the same across the wave (scalar branches, no divergence), while
// the block's other waves read the other groups of the same pixels' lines.  16-byte loads of the
// residual and 16-byte stores.  Each channel takes its value from the branch whose window holds it;
// a branch at the output's resolution is read at the pixel itself (it may be the output's own
// channel slice: the wave reads it before writing the same 16 bytes), an upsampled one through its
// four bilinear corners.  A branch map whose channel stride is a multiple of 8 is read in aligned
// 8-element pieces (one or two vector loads per corner, whatever the window's offset; a piece is
// read only when it holds a channel of the window, so it lies in a mapped page); others element by
// element.  Lets a channels-last KAD-Conv merge all its branches in one launch.
template <typename T>
__global__ __launch_bounds__(512) void merge_nhwc_vec_kernel(kad_merge_args a, int npix, int ngroups) {
  typedef Vec8<T> V;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // XCD-aware order (gridDim.x a multiple of 8): XCD b % 8 takes a contiguous run of pixels, so the
  // low-resolution rows that neighbouring output rows upsample from are fetched into one L2
  const int bq = (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
  const int p = bq * 64 + (int)(threadIdx.x & 63);
  if (p >= npix) return;
  const int x = p % a.w, t = p / a.w;
  const int y = t % a.h, n = t / a.h;
  const int nwaves = (int)(blockDim.x >> 6);  // one per group up to 8 (no wave takes two of a block's)
  for (int grp = wave; grp < ngroups; grp += nwaves) {
    const int c0 = a.c_begin + 8 * grp;
    const int64_t oi = (int64_t)p * a.out_cs + c0;
    float v[8];
    if (a.residual) {
      const V r = *(const V*)((const T*)a.residual + (int64_t)p * a.res_cs + c0);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_f32(r.v[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
    for (int b = 0; b < a.nbranch; ++b) {
      const int lo = a.br_c_off[b], hi = lo + a.br_c[b];
      if (hi <= c0 || lo >= c0 + 8) continue;
      const T* z = (const T*)a.br_z[b] + (int64_t)n * a.br_h[b] * a.br_w[b] * a.br_cs[b];
      const float* att = a.br_att[b] ? a.br_att[b] + (int64_t)n * a.br_c[b] : nullptr;
      const float coeff = a.br_coeff[b];
      const bool same = a.br_h[b] == a.h && a.br_w[b] == a.w;
      int x0, x1, y0, y1;
      float lx, ly;
      src_index(x, a.br_w[b], a.w, (float)a.br_w[b] / (float)a.w, x0, x1, lx);
      src_index(y, a.br_h[b], a.h, (float)a.br_h[b] / (float)a.h, y0, y1, ly);
      const int cs = a.br_cs[b], bw = a.br_w[b];
      const T* r0 = z + (int64_t)y0 * bw * cs;
      const T* r1 = z + (int64_t)y1 * bw * cs;
      const int d = c0 - lo;  // branch channel of the group's first channel (may be negative)
      const int ea = lo > c0 ? lo - c0 : 0, eb = hi < c0 + 8 ? hi - c0 : 8;  // valid e: [ea, eb)
      if ((cs & 7) == 0 && ((uintptr_t)a.br_z[b] % sizeof(T)) == 0) {
        // channels d .. d + 7 sit OFF elements into an aligned 8-element piece of the map, the same
        // OFF for every pixel
        const int mis = (int)(((uintptr_t)a.br_z[b] / sizeof(T) + (uintptr_t)(int64_t)d) & 7);
        auto body = [&](auto off_tag) {
          constexpr int OFF = decltype(off_tag)::value;
          const bool need0 = ea < 8 - OFF, need1 = OFF > 0 && eb > 8 - OFF;
          auto corner = [&](const T* px, float* r) {  // px: branch channel d of the corner pixel
            const T* al = px - OFF;
            V q0{}, q1{};
            if (need0) q0 = *(const V*)al;
            if (need1) q1 = *(const V*)(al + 8);
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = to_f32(OFF + e < 8 ? q0.v[(OFF + e) & 7] : q1.v[(OFF + e) & 7]);
          };
          float sv[8];
          if (same) {
            corner(r0 + (int64_t)x * cs + d, sv);
          } else {
            float c00[8], c01[8], c10[8], c11[8];
            corner(r0 + (int64_t)x0 * cs + d, c00);
            corner(r0 + (int64_t)x1 * cs + d, c01);
            corner(r1 + (int64_t)x0 * cs + d, c10);
            corner(r1 + (int64_t)x1 * cs + d, c11);
#pragma unroll
            for (int e = 0; e < 8; ++e)
              sv[e] = (1.f - ly) * ((1.f - lx) * c00[e] + lx * c01[e]) + ly * ((1.f - lx) * c10[e] + lx * c11[e]);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (e < ea || e >= eb) continue;
            float se = sv[e];
            if (att) se *= att[d + e];
            v[e] += coeff * se;
          }
        };
        switch (mis) {
          case 0: body(std::integral_constant<int, 0>{}); break;
          case 1: body(std::integral_constant<int, 1>{}); break;
          case 2: body(std::integral_constant<int, 2>{}); break;
          case 3: body(std::integral_constant<int, 3>{}); break;
          case 4: body(std::integral_constant<int, 4>{}); break;
          case 5: body(std::integral_constant<int, 5>{}); break;
          case 6: body(std::integral_constant<int, 6>{}); break;
          default: body(std::integral_constant<int, 7>{}); break;
        }
        continue;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (e < ea || e >= eb) continue;
        const int cb = d + e;
        float sv;
        if (same) {
          sv = to_f32(r0[(int64_t)x * cs + cb]);
        } else {
          const float v00 = to_f32(r0[(int64_t)x0 * cs + cb]), v01 = to_f32(r0[(int64_t)x1 * cs + cb]);
          const float v10 = to_f32(r1[(int64_t)x0 * cs + cb]), v11 = to_f32(r1[(int64_t)x1 * cs + cb]);
          sv = (1.f - ly) * ((1.f - lx) * v00 + lx * v01) + ly * ((1.f - lx) * v10 + lx * v11);
        }
        if (att) sv *= att[cb];
        v[e] += coeff * sv;
      }
    }
    V o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o.v[e] = from_f32<T>(a.gate ? v[e] * a.gate[c0 + e] : v[e]);
    *(V*)((T*)a.out + oi) = o;
  }
}

// ---- NCHW -> NHWC with a padded channel stride (pad channels written 0) ----------------
// 64 x 64 (pixel x channel) tiles transposed through LDS: reads coalesced along
// pixels, writes coalesced along channels.
template <typename T>
__global__ __launch_bounds__(256) void to_nhwc_kernel(const T* x, T* out, int c, int P, int cs) {
  __shared__ T tile[64][65];
  const int n = blockIdx.z;
  const int p0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
  const T* xb = x + (int64_t)n * c * P;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int pl = e & 63, cl = e >> 6;
    const int p = p0 + pl, ch = c0 + cl;
    tile[cl][pl] = (p < P && ch < c) ? xb[(int64_t)ch * P + p] : from_f32<T>(0.f);
  }
  __syncthreads();
  T* ob = out + (int64_t)n * P * cs;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int cl = e & 63, pl = e >> 6;
    const int p = p0 + pl, ch = c0 + cl;
    if (p < P && ch < cs) ob[(int64_t)p * cs + ch] = tile[cl][pl];
  }
}

// 16-bit, planes of a multiple of 8 pixels, 16-byte aligned, cs % 8 == 0: 8-pixel
// (16-byte) loads along each plane, 8-channel (16-byte) stores along each
// pixel.  LDS rows of 72 elements (144 bytes): the 16-byte row stores of 8
// lanes hit distinct banks.
// Flat XCD-aware grid: block b runs on XCD b % 8, which takes a contiguous run of
// (image, channel tile, pixel tile) tiles, so the 128-byte lines that two neighbouring
// pixel tiles share (planes need not be line-aligned) are fetched into one L2.
template <typename T>
__global__ __launch_bounds__(256) void to_nhwc_v8_kernel(const T* x, T* out, int c, int P, int cs, int npt, int nct,
                                                         int total, int grid8) {
  typedef T v8 __attribute__((ext_vector_type(8)));
  __shared__ __align__(16) T tile[64][72];
  const int bq = (int)(blockIdx.x & 7) * (grid8 >> 3) + (int)(blockIdx.x >> 3);
  if (bq >= total) return;  // whole block, before the barrier
  const int pt = bq % npt, r = bq / npt, ct = r % nct, n = r / nct;
  const int p0 = pt * 64, c0 = ct * 64;
  const T* xb = x + (int64_t)n * c * P;
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int v = tid & 7, cl = (tid >> 3) + 32 * u;
    const int p = p0 + 8 * v, ch = c0 + cl;
    v8 val = {};
    if (p < P && ch < c) val = *(const v8*)(xb + (int64_t)ch * P + p);  // P % 8 == 0: the piece is whole
    *(v8*)&tile[cl][8 * v] = val;
  }
  __syncthreads();
  T* ob = out + (int64_t)n * P * cs;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int pl = tid & 63, g = (tid >> 6) + 4 * u;
    const int p = p0 + pl, ch = c0 + 8 * g;
    if (p >= P || ch >= cs) continue;
    v8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = tile[8 * g + j][pl];
    *(v8*)(ob + (int64_t)p * cs + ch) = o;
  }
}

// ---- channels-last with pixel stride x_cs -> NHWC with channel stride cs (pad channels 0) ----
// One thread per output piece of 8 channels of one pixel: the input piece is read as
// elements (x_cs and c need not be multiples of 8), the output written as one vector (16 bytes for 16-bit data).  Consecutive
// threads cover consecutive pieces, so both sides are coalesced along the pixel rows.
template <typename T>
__global__ __launch_bounds__(256) void nhwc_pad_kernel(const T* x, T* out, int c, int x_cs, int cs, int64_t pixels) {
  typedef T v8 __attribute__((ext_vector_type(8)));
  const int pieces = cs >> 3;
  const int64_t total = pixels * pieces;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t p = i / pieces;
    const int c0 = (int)(i - p * pieces) * 8;
    const T* src = x + p * x_cs + c0;
    v8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = c0 + j < c ? src[j] : from_f32<T>(0.f);
    *(v8*)(out + p * cs + c0) = o;
  }
}

// ---- SE over NCHW in two launches (C % 32 == 0, hid <= 64) ---------------------------------
// Both launches give block b the 32 planes [32 b, 32 b + 32) (channels 32 (b % (C / 32)) .. of one
// image) and the same grid, so block b runs on the same XCD in both: the second launch re-reads
// the block's planes from that XCD's L2 (4 MB each: a 20 MB activation is 2.6 MB per XCD).
//  se_pool_l1: plane means, 16 lanes per plane over the 16-byte pieces that overlap it (a piece
//    shared with the neighbour plane is read by both, each adding only its own elements), then the
//    block's share of layer 1, hpart[n][b'][j] = sum over its 32 channels c of W1[j][c] g_c.
//  se_scale_l2: hidden[n] = relu(b1 + sum over the C / 32 shares) (every block of the image forms
//    it from the shares, 8 KB for C = 1024: no cross-block exchange inside a launch), att of the
//    block's 32 channels (16 lanes per channel, shuffle-reduced), then out = x * att, one thread
//    per piece.
// Every sum has a fixed order, so the result does not depend on the grid's timing.
constexpr int SEP_PLANES = 32, SEP_T = 512, SEP_KU = 8, SEP_HID = 64;

// sum of the elements [lo, hi) of an 8-element piece (fp32 accumulation)
template <typename T> struct PieceSum;
template <> struct PieceSum<half_t> {
  typedef half_t t8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ float all(const t8& v, float acc) {
    const half2_t one = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
    for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_fdot2((half2_t){v[2 * k], v[2 * k + 1]}, one, acc, false);
    return acc;
  }
};
template <> struct PieceSum<bf16_t> {
  typedef bf16_t t8 __attribute__((ext_vector_type(8)));
  typedef bf16_t b2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float all(const t8& v, float acc) {
    const b2 one = {(bf16_t)1.0f, (bf16_t)1.0f};
#pragma unroll
    for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_fdot2_f32_bf16((b2){v[2 * k], v[2 * k + 1]}, one, acc, false);
    return acc;
  }
};
template <> struct PieceSum<float> {
  typedef float t8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ float all(const t8& v, float acc) {
#pragma unroll
    for (int k = 0; k < 8; ++k) acc += v[k];
    return acc;
  }
};
template <typename T, typename V>
__device__ __forceinline__ float piece_sum(const V& v, int lo, int hi, float acc) {
  if (lo == 0 && hi == 8) return PieceSum<T>::all(v, acc);
#pragma unroll
  for (int k = 0; k < 8; ++k) acc += (k >= lo && k < hi) ? to_f32(v[k]) : 0.f;
  return acc;
}

template <typename T>
__global__ __launch_bounds__(SEP_T) void se_pool_l1_kernel(const T* __restrict__ x, const float* __restrict__ w1,
                                                           float* __restrict__ hpart, int c, int hw, int hid) {
  typedef T t8 __attribute__((ext_vector_type(8)));
  __shared__ float s_g[SEP_PLANES];
  const int tid = threadIdx.x;
  const int nb = c / SEP_PLANES, b = blockIdx.x, cb = b % nb;
  // layer-1 weights of this thread (unit u = tid / 8, channels 4 q .. 4 q + 3 of the block), early
  const int u1 = tid >> 3, q = tid & 7;
  float wv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wv[i] = u1 < hid ? w1[(int64_t)u1 * c + cb * SEP_PLANES + 4 * q + i] : 0.f;
  const T* xb = x + (int64_t)b * SEP_PLANES * hw;
  const int g = tid >> 4, jl = tid & 15;          // plane g of the block, lane jl of its 16
  const int e_lo = g * hw, e_hi = e_lo + hw;
  const int f = e_lo >> 3, l = (e_hi - 1) >> 3;   // pieces overlapping the plane
  float acc = 0.f;
  for (int p0 = f + jl; p0 <= l; p0 += 16 * SEP_KU) {
    t8 xv[SEP_KU];
#pragma unroll
    for (int k = 0; k < SEP_KU; ++k)
      if (p0 + 16 * k <= l) xv[k] = *(const t8*)(xb + (int64_t)(p0 + 16 * k) * 8);
#pragma unroll
    for (int k = 0; k < SEP_KU; ++k) {
      const int p = p0 + 16 * k;
      if (p > l) continue;
      const int lo = e_lo - 8 * p > 0 ? e_lo - 8 * p : 0, hi = e_hi - 8 * p < 8 ? e_hi - 8 * p : 8;
      acc = piece_sum<T>(xv[k], lo, hi, acc);
    }
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) acc += __shfl_xor(acc, o);
  if (jl == 0) s_g[g] = acc / (float)hw;
  __syncthreads();
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) a += wv[i] * s_g[4 * q + i];
  a += __shfl_xor(a, 1);
  a += __shfl_xor(a, 2);
  a += __shfl_xor(a, 4);
  if (q == 0 && u1 < hid) hpart[(int64_t)b * SEP_HID + u1] = a;
}

template <typename T>
__global__ __launch_bounds__(SEP_T) void se_scale_l2_kernel(const T* __restrict__ x, const float* __restrict__ hpart,
                                                            const float* __restrict__ b1, const float* __restrict__ w2,
                                                            const float* __restrict__ b2, float* __restrict__ att,
                                                            T* __restrict__ out, int c, int hw, int hid) {
  typedef T t8 __attribute__((ext_vector_type(8)));
  __shared__ float s_att[SEP_PLANES];
  __shared__ float s_h[8][SEP_HID];
  const int tid = threadIdx.x;
  const int nb = c / SEP_PLANES, b = blockIdx.x, n = b / nb, c0 = (b - n * nb) * SEP_PLANES;
  const int npc = SEP_PLANES * hw / 8;  // pieces of the block
  const T* xb = x + (int64_t)b * SEP_PLANES * hw;
  T* ob = out + (int64_t)b * SEP_PLANES * hw;
  t8 xv[SEP_KU];
#pragma unroll
  for (int k = 0; k < SEP_KU; ++k)
    if (tid + SEP_T * k < npc) xv[k] = *(const t8*)(xb + (int64_t)(tid + SEP_T * k) * 8);
  // hidden[n]: unit u = tid % 64, slice sl = tid / 64 adds shares sl, sl + 8, ... (loads first)
  {
    const int u = tid & 63, sl = tid >> 6;
    const float* hp = hpart + (int64_t)n * nb * SEP_HID + u;
    float h = 0.f;
    for (int k0 = sl; k0 < nb; k0 += 8 * 8) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (u < hid && k0 + 8 * i < nb) ? hp[(int64_t)(k0 + 8 * i) * SEP_HID] : 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) h += v[i];
    }
    s_h[sl][u] = h;
  }
  // this thread's W2 slice: channel c0 + tid / 16, hidden units 4 (tid % 16) .. + 3
  const int cl = tid >> 4, q = tid & 15;
  float wv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wv[i] = 4 * q + i < hid ? w2[(int64_t)(c0 + cl) * hid + 4 * q + i] : 0.f;
  __syncthreads();
  if (tid < SEP_HID) {
    float t = s_h[0][tid];
#pragma unroll
    for (int k = 1; k < 8; ++k) t += s_h[k][tid];
    s_h[0][tid] = tid < hid ? fmaxf(t + (b1 ? b1[tid] : 0.f), 0.f) : 0.f;
  }
  __syncthreads();
  {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) a += wv[i] * s_h[0][4 * q + i];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) a += __shfl_xor(a, o);
    if (q == 0) {
      const float v = sigmoidf_(a + (b2 ? b2[c0 + cl] : 0.f));
      s_att[cl] = v;
      att[(int64_t)n * c + c0 + cl] = v;
    }
  }
  __syncthreads();
  const float inv_hw = 1.f / (float)hw;
  for (int v0 = tid; v0 < npc; v0 += SEP_T * SEP_KU) {
    if (v0 != tid) {
#pragma unroll
      for (int k = 0; k < SEP_KU; ++k)
        if (v0 + SEP_T * k < npc) xv[k] = *(const t8*)(xb + (int64_t)(v0 + SEP_T * k) * 8);
    }
#pragma unroll
    for (int k = 0; k < SEP_KU; ++k) {
      const int v = v0 + SEP_T * k;
      if (v >= npc) continue;
      const int e0 = v * 8;
      int p0 = (int)((float)e0 * inv_hw);  // e0 < 2^24: within one of the true quotient
      p0 -= p0 * hw > e0;
      p0 += (p0 + 1) * hw <= e0;
      const int nfirst = (p0 + 1) * hw - e0;
      const float s0 = s_att[p0], s1 = nfirst < 8 ? s_att[p0 + 1] : s0;
      t8 o;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) o[kk] = from_f32<T>(to_f32(xv[k][kk]) * (kk < nfirst ? s0 : s1));
      *(t8*)(ob + (int64_t)e0) = o;
    }
  }
}

static int grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  return (int)(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

}  // namespace kad

using namespace kad;

// ---- SE MLP over the whole batch, two launches (caller-owned hidden buffer) -------------------
// One block per image pulls both weight matrices (2 x hid x C fp32: 512 KB at C = 1024) through
// a single CU; here both layers are spread over (unit, 4-image group) waves:
//  layer 1: wave (j, images 4 y .. 4 y + 3): lane l holds W1[j][l + 64 k] and the four images'
//           tile-summed g at the same channels (every load issued before the first add), then
//           four interleaved wave reductions; grid (ceil(hid / 4), ceil(n / 4)) x 4 waves;
//  layer 2: block (64 channels, 4 images): the block's W2 rows, one contiguous span, are staged
//           in LDS with an odd row stride by coalesced loads; thread (image, channel) forms
//           att = sigmoid(W2[ch] . h[i] + b2[ch]).
// Each output is a fixed-order sum, independent of the grid.
constexpr int SEL_MAXC = 1024;    // layer 1: C / 64 <= 16 channels per lane
constexpr int SEL_MAXHID = 64;    // layer 2: W2 slice [64][hid + 1] and h [4][hid] in LDS

__global__ __launch_bounds__(256) void se_mlp_l1_kernel(const float* partial, int tiles, float inv_count,
                                                        const float* w1, const float* b1, float* hbuf, int n, int c,
                                                        int hid) {
  constexpr int KC = SEL_MAXC / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = blockIdx.x * 4 + wave, i0 = blockIdx.y * 4;
  if (j >= hid) return;  // no barrier in this kernel
  float wv[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) wv[k] = lane + 64 * k < c ? w1[(int64_t)j * c + lane + 64 * k] : 0.f;
  float gv[4][KC];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int k = 0; k < KC; ++k) gv[q][k] = 0.f;
  for (int t = 0; t < tiles; ++t) {
    float ld[4][KC];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const int i = i0 + q, ch = lane + 64 * k;
        ld[q][k] = (i < n && ch < c) ? partial[((int64_t)i * tiles + t) * c + ch] : 0.f;
      }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int k = 0; k < KC; ++k) gv[q][k] += ld[q][k];
  }
  float a[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    a[q] = 0.f;
#pragma unroll
    for (int k = 0; k < KC; ++k) a[q] += wv[k] * (gv[q][k] * inv_count);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] += __shfl_xor(a[q], o);
  const float bj = b1 ? b1[j] : 0.f;
  if (lane < 4 && i0 + lane < n) {
    float v = a[0];
#pragma unroll
    for (int q = 1; q < 4; ++q) v = lane == q ? a[q] : v;
    hbuf[(int64_t)(i0 + lane) * hid + j] = fmaxf(v + bj, 0.f);
  }
}

__global__ __launch_bounds__(256) void se_mlp_l2_kernel(const float* hbuf, const float* w2, const float* b2,
                                                        float* att, int n, int c, int hid) {
  __shared__ float ws[64 * (SEL_MAXHID + 1)];  // [64 channels][hid + 1]
  __shared__ float hs[4 * SEL_MAXHID];         // [4 images][hid]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c0 = blockIdx.x * 64, i0 = blockIdx.y * 4, i = i0 + wave, ch = c0 + lane;
  const int nrow = c - c0 < 64 ? c - c0 : 64, span = nrow * hid;  // W2 rows c0 .. c0 + nrow - 1
  constexpr int PER = 64 * SEL_MAXHID / 256;
  float wl[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) wl[u] = tid + 256 * u < span ? w2[(int64_t)c0 * hid + tid + 256 * u] : 0.f;
  const float hv = (wave < 4 && lane < hid && i < n) ? hbuf[(int64_t)i * hid + lane] : 0.f;
  const float bc = (b2 && ch < c) ? b2[ch] : 0.f;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = tid + 256 * u;
    if (e < span) {
      const int r = e / hid;
      ws[r * (hid + 1) + e - r * hid] = wl[u];
    }
  }
  if (lane < hid) hs[wave * hid + lane] = hv;
  __syncthreads();
  if (ch >= c || i >= n) return;  // after the only barrier
  const float* wr = ws + lane * (hid + 1);
  const float* hi = hs + wave * hid;
  float a0 = 0.f, a1 = 0.f;
  for (int k = 0; k + 1 < hid; k += 2) {
    a0 += wr[k] * hi[k];
    a1 += wr[k + 1] * hi[k + 1];
  }
  if (hid & 1) a0 += wr[hid - 1] * hi[hid - 1];
  att[(int64_t)i * c + ch] = sigmoidf_(a0 + a1 + bc);
}

// ---- SE layer 2 fused into the channel scale (NCHW) ---------------------------------------------
// out = x * sigmoid(W2[c] . h[n] + b2[c]): block b scales the flat elements [2048 b, 2048 b + 2048)
// (one 16-byte piece per thread, loaded first) and computes the attention of the planes that range
// touches (at most 2048 / hw + 2 <= 34), four threads per plane (16 hidden units each, every load
// issued before the first product, shuffle-reduced), into LDS; att[n][c] is also written (planes
// shared by two blocks get the same value twice).  hw >= 64, hid <= 64.
constexpr int SS_ELEMS = 2048, SS_MINHW = 64, SS_MAXPL = SS_ELEMS / SS_MINHW + 2;

template <typename T>
__global__ __launch_bounds__(256) void se_scale_flat_kernel(const T* x, const float* hbuf, const float* w2,
                                                           const float* b2, float* att, T* out, int64_t total, int hw,
                                                           int c, int hid) {
  typedef T t8 __attribute__((ext_vector_type(8)));
  __shared__ float s_att[SS_MAXPL];
  const int tid = threadIdx.x;
  const int64_t b0 = (int64_t)blockIdx.x * SS_ELEMS, e0 = b0 + 8 * tid;
  t8 xv;
  if (e0 < total) xv = *(const t8*)(x + e0);
  const int64_t blast = (b0 + SS_ELEMS < total ? b0 + SS_ELEMS : total) - 1;
  const int p_lo = (int)(b0 / hw), npl = (int)(blast / hw) - p_lo + 1;
  const int pt = tid >> 2, q = tid & 3;
  if (pt < npl) {  // 4 * npl <= 136 threads: whole quads, so the shuffles stay inside live lanes
    const int p = p_lo + pt, n = p / c, ch = p - n * c;
    const float* wr = w2 + (int64_t)ch * hid + 16 * q;
    const float* hr = hbuf + (int64_t)n * hid + 16 * q;
    float wv[16], hv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool ok = 16 * q + j < hid;
      wv[j] = ok ? wr[j] : 0.f;
      hv[j] = ok ? hr[j] : 0.f;
    }
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      a0 += wv[j] * hv[j];
      a1 += wv[j + 1] * hv[j + 1];
    }
    float a = a0 + a1;
    a += __shfl_xor(a, 1);
    a += __shfl_xor(a, 2);
    if (q == 0) {
      const float v = sigmoidf_(a + (b2 ? b2[ch] : 0.f));
      s_att[pt] = v;
      att[p] = v;
    }
  }
  __syncthreads();
  if (e0 >= total) return;  // after the only barrier
  const int pe = (int)(e0 / hw);
  const int64_t off = e0 - (int64_t)pe * hw;          // position of the piece in plane pe
  const int n0 = (int)(hw - off < 8 ? hw - off : 8);  // elements of the piece in plane pe
  const float s0 = s_att[pe - p_lo], s1 = n0 < 8 ? s_att[pe + 1 - p_lo] : s0;
  t8 o;
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = from_f32<T>(to_f32(xv[k]) * (k < n0 ? s0 : s1));
  *(t8*)(out + e0) = o;
}

extern "C" int kad_se_pool(const void* x, float* partial, int n, int c, int h, int w, int layout, int x_cs,
                           int dtype, void* stream) {
  KAD_CHECK_ARG(x && partial, "kad_se_pool: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0, "kad_se_pool: bad shape");
  hipStream_t st = (hipStream_t)stream;
  const int P = h * w;
  if (layout == KAD_NCHW) {
    const int planes = n * c;
    dim3 grid(ceil_div(planes, 4));
    const int64_t total = (int64_t)planes * P;
    if (P >= 8 && total % 8 == 0 && total < (1ll << 31) && (uintptr_t)x % (8 * dtype_size(dtype)) == 0) {
      dim3 gridf(ceil_div(planes, 16));  // 4 waves x 4 planes per block
      switch (dtype) {
        case KAD_F32: hipLaunchKernelGGL(se_pool_flat_kernel<float>, gridf, dim3(256), 0, st, (const float*)x, partial, planes, P); break;
        case KAD_F16: hipLaunchKernelGGL(se_pool_flat_kernel<half_t>, gridf, dim3(256), 0, st, (const half_t*)x, partial, planes, P); break;
        case KAD_BF16: hipLaunchKernelGGL(se_pool_flat_kernel<bf16_t>, gridf, dim3(256), 0, st, (const bf16_t*)x, partial, planes, P); break;
        default: return fail(KAD_EINVAL, "kad_se_pool: unknown dtype %d", dtype);
      }
      return check_launch("kad_se_pool");
    }
    switch (dtype) {
      case KAD_F32: hipLaunchKernelGGL(se_pool_nchw_kernel<float>, grid, dim3(256), 0, st, (const float*)x, partial, planes, P); break;
      case KAD_F16: hipLaunchKernelGGL(se_pool_nchw_kernel<half_t>, grid, dim3(256), 0, st, (const half_t*)x, partial, planes, P); break;
      case KAD_BF16: hipLaunchKernelGGL(se_pool_nchw_kernel<bf16_t>, grid, dim3(256), 0, st, (const bf16_t*)x, partial, planes, P); break;
      default: return fail(KAD_EINVAL, "kad_se_pool: unknown dtype %d", dtype);
    }
  } else if (layout == KAD_NHWC) {
    KAD_CHECK_ARG(x_cs >= c, "kad_se_pool: channel stride < C");
    const int tiles = ceil_div(P, 256);
    dim3 grid(tiles, n);
    switch (dtype) {
      case KAD_F32: hipLaunchKernelGGL(se_pool_nhwc_kernel<float>, grid, dim3(256), 0, st, (const float*)x, partial, c, P, x_cs, tiles); break;
      case KAD_F16: hipLaunchKernelGGL(se_pool_nhwc_kernel<half_t>, grid, dim3(256), 0, st, (const half_t*)x, partial, c, P, x_cs, tiles); break;
      case KAD_BF16: hipLaunchKernelGGL(se_pool_nhwc_kernel<bf16_t>, grid, dim3(256), 0, st, (const bf16_t*)x, partial, c, P, x_cs, tiles); break;
      default: return fail(KAD_EINVAL, "kad_se_pool: unknown dtype %d", dtype);
    }
  } else {
    return fail(KAD_EINVAL, "kad_se_pool: bad layout %d", layout);
  }
  return check_launch("kad_se_pool");
}

extern "C" int kad_se_pool_tiles(int h, int w, int layout) {
  return layout == KAD_NCHW ? 1 : ceil_div(h * w, 256);
}

extern "C" int kad_se_mlp(const float* partial, int tiles, float inv_count, const float* w1, const float* b1,
                          const float* w2, const float* b2, float* att, int n, int c, int hid, void* stream) {
  KAD_CHECK_ARG(partial && w1 && w2 && att, "kad_se_mlp: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && hid > 0 && tiles > 0, "kad_se_mlp: bad shape");
  const int nsl_s = c < SE_ST ? SE_ST / c : 1;
  const size_t lds_staged =
      (size_t)(c + hid + (size_t)(nsl_s + tiles) * c + (size_t)hid * c + (size_t)c * (hid + 1)) * sizeof(float);
  if (lds_staged <= 160 * 1024) {  // gfx950: 160 KB of LDS per CU (KADConv's C -> C -> C SE at 100 x 100: 89 KB)
    allow_lds(se_mlp_staged_kernel, lds_staged);
    hipLaunchKernelGGL(se_mlp_staged_kernel, dim3(n), dim3(SE_ST), lds_staged, (hipStream_t)stream, partial, tiles,
                       inv_count, w1, b1, w2, b2, att, c, hid);
    return check_launch("kad_se_mlp");
  }
  if (c <= SE_WIDE && c % 64 == 0 && hid <= 64 && hid % 4 == 0 && ((uintptr_t)w1 | (uintptr_t)w2) % 16 == 0) {
    hipLaunchKernelGGL(se_mlp_wide_kernel, dim3(n), dim3(SE_WIDE), 0, (hipStream_t)stream, partial, tiles, inv_count,
                       w1, b1, w2, b2, att, c, hid);
    return check_launch("kad_se_mlp");
  }
  const int nt = c <= 256 ? 256 : 1024;
  const int nsl = c < nt ? nt / c : 1;
  const size_t lds = (size_t)(c + hid + (size_t)nsl * c) * sizeof(float);
  KAD_CHECK_ARG(lds <= 64 * 1024, "kad_se_mlp: C + hidden too large");
  if (nt == 256)
    hipLaunchKernelGGL(se_mlp_kernel<256>, dim3(n), dim3(256), lds, (hipStream_t)stream, partial, tiles, inv_count, w1,
                       b1, w2, b2, att, c, hid);
  else
    hipLaunchKernelGGL(se_mlp_kernel<1024>, dim3(n), dim3(1024), lds, (hipStream_t)stream, partial, tiles, inv_count,
                       w1, b1, w2, b2, att, c, hid);
  return check_launch("kad_se_mlp");
}

extern "C" int kad_se_mlp_ws(const float* partial, int tiles, float inv_count, const float* w1, const float* b1,
                             const float* w2, const float* b2, float* att, int n, int c, int hid, float* hidden,
                             void* stream) {
  KAD_CHECK_ARG(partial && w1 && w2 && att && hidden, "kad_se_mlp_ws: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && hid > 0 && tiles > 0, "kad_se_mlp_ws: bad shape");
  if (c > SEL_MAXC || hid > SEL_MAXHID || n > 65535 * 4)
    return kad_se_mlp(partial, tiles, inv_count, w1, b1, w2, b2, att, n, c, hid, stream);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(se_mlp_l1_kernel, dim3(ceil_div(hid, 4), ceil_div(n, 4)), dim3(256), 0, st, partial, tiles,
                     inv_count, w1, b1, hidden, n, c, hid);
  int rc = check_launch("kad_se_mlp_ws");
  if (rc) return rc;
  hipLaunchKernelGGL(se_mlp_l2_kernel, dim3(ceil_div(c, 64), ceil_div(n, 4)), dim3(256), 0, st,
                     (const float*)hidden, w2, b2, att, n, c, hid);
  return check_launch("kad_se_mlp_ws");
}

extern "C" int kad_se_hidden(const float* partial, int tiles, float inv_count, const float* w1, const float* b1,
                             float* hidden, int n, int c, int hid, void* stream) {
  KAD_CHECK_ARG(partial && w1 && hidden, "kad_se_hidden: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && hid > 0 && tiles > 0, "kad_se_hidden: bad shape");
  KAD_CHECK_ARG(c <= SEL_MAXC && n <= 65535 * 4, "kad_se_hidden: C = %d above %d", c, SEL_MAXC);
  hipLaunchKernelGGL(se_mlp_l1_kernel, dim3(ceil_div(hid, 4), ceil_div(n, 4)), dim3(256), 0, (hipStream_t)stream,
                     partial, tiles, inv_count, w1, b1, hidden, n, c, hid);
  return check_launch("kad_se_hidden");
}

extern "C" int kad_se_nchw_fits(int n, int c, int h, int w, int hid) {
  return n > 0 && c > 0 && c % SEP_PLANES == 0 && hid > 0 && hid <= SEP_HID && h > 0 && w > 0 && h * w >= 8 &&
         (int64_t)h * w * SEP_PLANES < (1 << 24) && (int64_t)n * c * h * w < (1ll << 31);
}

extern "C" int kad_se_nchw(const void* x, void* out, const float* w1, const float* b1, const float* w2,
                           const float* b2, float* att, float* hpart, int n, int c, int h, int w, int hid, int dtype,
                           void* stream) {
  KAD_CHECK_ARG(x && out && w1 && w2 && att && hpart, "kad_se_nchw: null pointer");
  KAD_CHECK_ARG(kad_se_nchw_fits(n, c, h, w, hid),
                "kad_se_nchw: needs C %% 32 == 0, hidden <= 64, H W >= 8 (n %d, c %d, %dx%d, hid %d)", n, c, h, w, hid);
  const int vb = 8 * dtype_size(dtype);
  KAD_CHECK_ARG((uintptr_t)x % vb == 0 && (uintptr_t)out % vb == 0, "kad_se_nchw: x / out not %d-byte aligned", vb);
  const int hw = h * w, grid = n * (c / SEP_PLANES);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case KAD_F32:
      hipLaunchKernelGGL(se_pool_l1_kernel<float>, dim3(grid), dim3(SEP_T), 0, st, (const float*)x, w1, hpart, c, hw, hid);
      hipLaunchKernelGGL(se_scale_l2_kernel<float>, dim3(grid), dim3(SEP_T), 0, st, (const float*)x, hpart, b1, w2, b2, att,
                         (float*)out, c, hw, hid);
      break;
    case KAD_F16:
      hipLaunchKernelGGL(se_pool_l1_kernel<half_t>, dim3(grid), dim3(SEP_T), 0, st, (const half_t*)x, w1, hpart, c, hw, hid);
      hipLaunchKernelGGL(se_scale_l2_kernel<half_t>, dim3(grid), dim3(SEP_T), 0, st, (const half_t*)x, hpart, b1, w2, b2,
                         att, (half_t*)out, c, hw, hid);
      break;
    case KAD_BF16:
      hipLaunchKernelGGL(se_pool_l1_kernel<bf16_t>, dim3(grid), dim3(SEP_T), 0, st, (const bf16_t*)x, w1, hpart, c, hw, hid);
      hipLaunchKernelGGL(se_scale_l2_kernel<bf16_t>, dim3(grid), dim3(SEP_T), 0, st, (const bf16_t*)x, hpart, b1, w2, b2,
                         att, (bf16_t*)out, c, hw, hid);
      break;
    default: return fail(KAD_EINVAL, "kad_se_nchw: unknown dtype %d", dtype);
  }
  return check_launch("kad_se_nchw");
}

extern "C" int kad_se_scale(const void* x, const float* hidden, const float* w2, const float* b2, float* att,
                            void* out, int n, int c, int h, int w, int hid, int dtype, void* stream) {
  KAD_CHECK_ARG(x && hidden && w2 && att && out, "kad_se_scale: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0 && hid > 0, "kad_se_scale: bad shape");
  const int64_t total = (int64_t)n * c * h * w;
  const int vb = 8 * dtype_size(dtype);
  hipStream_t st = (hipStream_t)stream;
  if (h * w >= SS_MINHW && hid <= SEL_MAXHID && total % 8 == 0 && total / SS_ELEMS < (1ll << 31) &&
      (uintptr_t)x % vb == 0 && (uintptr_t)out % vb == 0) {
    const dim3 grid((unsigned)((total + SS_ELEMS - 1) / SS_ELEMS));
    switch (dtype) {
      case KAD_F32: hipLaunchKernelGGL(se_scale_flat_kernel<float>, grid, dim3(256), 0, st, (const float*)x, hidden, w2, b2, att, (float*)out, total, h * w, c, hid); break;
      case KAD_F16: hipLaunchKernelGGL(se_scale_flat_kernel<half_t>, grid, dim3(256), 0, st, (const half_t*)x, hidden, w2, b2, att, (half_t*)out, total, h * w, c, hid); break;
      case KAD_BF16: hipLaunchKernelGGL(se_scale_flat_kernel<bf16_t>, grid, dim3(256), 0, st, (const bf16_t*)x, hidden, w2, b2, att, (bf16_t*)out, total, h * w, c, hid); break;
      default: return fail(KAD_EINVAL, "kad_se_scale: unknown dtype %d", dtype);
    }
    return check_launch("kad_se_scale");
  }
  // small planes or unaligned tensors: att by the layer-2 kernel, then the plain channel scale
  KAD_CHECK_ARG(hid <= SEL_MAXHID, "kad_se_scale: hidden width %d above %d", hid, SEL_MAXHID);
  hipLaunchKernelGGL(se_mlp_l2_kernel, dim3(ceil_div(c, 64), ceil_div(n, 4)), dim3(256), 0, st, hidden, w2, b2, att, n,
                     c, hid);
  int rc = check_launch("kad_se_scale");
  if (rc) return rc;
  return kad_channel_scale(x, att, out, n, c, h, w, KAD_NCHW, c, dtype, stream);
}

extern "C" int kad_channel_scale(const void* x, const float* att, void* out, int n, int c, int h, int w, int layout,
                                 int x_cs, int dtype, void* stream) {
  KAD_CHECK_ARG(x && att && out, "kad_channel_scale: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0, "kad_channel_scale: bad shape");
  const int cs = layout == KAD_NHWC ? x_cs : c;
  KAD_CHECK_ARG(cs >= c, "kad_channel_scale: channel stride < C");
  const int64_t total = (int64_t)n * h * w * cs;
  hipStream_t st = (hipStream_t)stream;
  const int vb = 8 * dtype_size(dtype);
  if (layout == KAD_NCHW && h * w >= 8 && total % 8 == 0 && total < (1ll << 31) && (uintptr_t)x % vb == 0 &&
      (uintptr_t)out % vb == 0) {
    const int nvec = (int)(total / 8);
    const dim3 grid(grid_for(nvec));
    switch (dtype) {
      case KAD_F32: hipLaunchKernelGGL(channel_scale_flat_kernel<float>, grid, dim3(256), 0, st, (const float*)x, att, (float*)out, nvec, h * w); break;
      case KAD_F16: hipLaunchKernelGGL(channel_scale_flat_kernel<half_t>, grid, dim3(256), 0, st, (const half_t*)x, att, (half_t*)out, nvec, h * w); break;
      case KAD_BF16: hipLaunchKernelGGL(channel_scale_flat_kernel<bf16_t>, grid, dim3(256), 0, st, (const bf16_t*)x, att, (bf16_t*)out, nvec, h * w); break;
      default: return fail(KAD_EINVAL, "kad_channel_scale: unknown dtype %d", dtype);
    }
    return check_launch("kad_channel_scale");
  }
  switch (dtype) {
    case KAD_F32: hipLaunchKernelGGL(channel_scale_kernel<float>, dim3(grid_for(total)), dim3(256), 0, st, (const float*)x, att, (float*)out, total, c, h * w, layout, cs); break;
    case KAD_F16: hipLaunchKernelGGL(channel_scale_kernel<half_t>, dim3(grid_for(total)), dim3(256), 0, st, (const half_t*)x, att, (half_t*)out, total, c, h * w, layout, cs); break;
    case KAD_BF16: hipLaunchKernelGGL(channel_scale_kernel<bf16_t>, dim3(grid_for(total)), dim3(256), 0, st, (const bf16_t*)x, att, (bf16_t*)out, total, c, h * w, layout, cs); break;
    default: return fail(KAD_EINVAL, "kad_channel_scale: unknown dtype %d", dtype);
  }
  return check_launch("kad_channel_scale");
}

// ---- in-place att * out + residual over a channel slice ---------------------------------------
// NCHW: block = one channel plane (n, j), 16-byte vectors along the plane, all
// loads of a thread issued before its stores.
template <typename T>
__global__ __launch_bounds__(256) void scale_residual_nchw_kernel(T* out, const float* att, const T* res, int c,
                                                                  int hw, int img_c, int c_off) {
  constexpr int V = 16 / (int)sizeof(T), UNR = 8;  // a 10^4-pixel 16-bit plane is one batch per thread
  const int plane = blockIdx.x, n = plane / c, j = plane - n * c;
  const float at = att[plane];
  const int64_t base = ((int64_t)n * img_c + c_off + j) * hw;
  T* o = out + base;
  const T* r = res ? res + base : nullptr;
  const int nv = ((hw * (int)sizeof(T)) % 16 == 0) ? hw / V : 0;  // whole-plane vectors when aligned
  typedef T vec __attribute__((ext_vector_type(V)));
  for (int v0 = threadIdx.x; v0 < nv; v0 += 256 * UNR) {
    vec ov[UNR], rv[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int v = v0 + u * 256;
      if (v < nv) {
        ov[u] = ((const vec*)o)[v];
        if (r) rv[u] = ((const vec*)r)[v];
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int v = v0 + u * 256;
      if (v < nv) {
        vec y;
#pragma unroll
        for (int e = 0; e < V; ++e) y[e] = from_f32<T>(at * to_f32(ov[u][e]) + (r ? to_f32(rv[u][e]) : 0.f));
        ((vec*)o)[v] = y;
      }
    }
  }
  for (int i = nv * V + threadIdx.x; i < hw; i += 256)  // unaligned planes: scalar
    o[i] = from_f32<T>(at * to_f32(o[i]) + (r ? to_f32(r[i]) : 0.f));
}

// NHWC: block = 64 pixels; threads run along the slice's channels.
template <typename T>
__global__ __launch_bounds__(256) void scale_residual_nhwc_kernel(T* out, const float* att, const T* res, int c,
                                                                  int hw, int img_c, int c_off, int64_t npix) {
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  for (int e = threadIdx.x; e < 64 * c; e += 256) {
    const int64_t p = p0 + e / c;
    const int j = e % c;
    if (p >= npix) break;
    const int64_t n = p / hw;
    const int64_t i = p * img_c + c_off + j;
    out[i] = from_f32<T>(att[n * c + j] * to_f32(out[i]) + (res ? to_f32(res[i]) : 0.f));
  }
}

extern "C" int kad_scale_residual(void* out, const float* att, const void* residual, int n, int c, int h, int w,
                                  int img_c, int c_off, int layout, int dtype, void* stream) {
  KAD_CHECK_ARG(out && att, "kad_scale_residual: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0 && c_off >= 0 && c_off + c <= img_c,
                "kad_scale_residual: bad shape (c=%d c_off=%d img_c=%d)", c, c_off, img_c);
  KAD_CHECK_ARG(layout == KAD_NCHW || layout == KAD_NHWC, "kad_scale_residual: bad layout");
  KAD_CHECK_ARG(((uintptr_t)out | (uintptr_t)residual) % 16 == 0, "kad_scale_residual: 16-byte alignment");
  hipStream_t st = (hipStream_t)stream;
  const int hw = h * w;
  if (layout == KAD_NCHW) {
    dim3 grid(n * c);
    switch (dtype) {
      case KAD_F32: hipLaunchKernelGGL(scale_residual_nchw_kernel<float>, grid, dim3(256), 0, st, (float*)out, att, (const float*)residual, c, hw, img_c, c_off); break;
      case KAD_F16: hipLaunchKernelGGL(scale_residual_nchw_kernel<half_t>, grid, dim3(256), 0, st, (half_t*)out, att, (const half_t*)residual, c, hw, img_c, c_off); break;
      case KAD_BF16: hipLaunchKernelGGL(scale_residual_nchw_kernel<bf16_t>, grid, dim3(256), 0, st, (bf16_t*)out, att, (const bf16_t*)residual, c, hw, img_c, c_off); break;
      default: return fail(KAD_EINVAL, "kad_scale_residual: unknown dtype %d", dtype);
    }
  } else {
    const int64_t npix = (int64_t)n * hw;
    dim3 grid((unsigned)((npix + 63) / 64));
    switch (dtype) {
      case KAD_F32: hipLaunchKernelGGL(scale_residual_nhwc_kernel<float>, grid, dim3(256), 0, st, (float*)out, att, (const float*)residual, c, hw, img_c, c_off, npix); break;
      case KAD_F16: hipLaunchKernelGGL(scale_residual_nhwc_kernel<half_t>, grid, dim3(256), 0, st, (half_t*)out, att, (const half_t*)residual, c, hw, img_c, c_off, npix); break;
      case KAD_BF16: hipLaunchKernelGGL(scale_residual_nhwc_kernel<bf16_t>, grid, dim3(256), 0, st, (bf16_t*)out, att, (const bf16_t*)residual, c, hw, img_c, c_off, npix); break;
      default: return fail(KAD_EINVAL, "kad_scale_residual: unknown dtype %d", dtype);
    }
  }
  return check_launch("kad_scale_residual");
}

extern "C" int kad_branch_merge(const kad_merge_args* a_in, void* stream) {
  KAD_CHECK_ARG(a_in && a_in->out, "kad_branch_merge: null pointer");
  kad_merge_args win = *a_in;
  if (win.c_begin == 0 && win.c_end == 0) win.c_end = win.c;
  KAD_CHECK_ARG(win.layout == KAD_NHWC || (win.out_cs == 0 && win.res_cs == 0),
                "kad_branch_merge: out_cs / res_cs apply to NHWC only");
  if (win.out_cs == 0) win.out_cs = win.c;
  if (win.res_cs == 0) win.res_cs = win.c;
  KAD_CHECK_ARG(win.out_cs >= win.c && win.res_cs >= win.c, "kad_branch_merge: out_cs %d / res_cs %d < c=%d",
                win.out_cs, win.res_cs, win.c);
  const kad_merge_args* a = &win;
  KAD_CHECK_ARG(a->c_begin >= 0 && a->c_begin < a->c_end && a->c_end <= a->c,
                "kad_branch_merge: channel window [%d, %d) outside [0, %d)", a->c_begin, a->c_end, a->c);
  KAD_CHECK_ARG(a->n > 0 && a->c > 0 && a->h > 0 && a->w > 0, "kad_branch_merge: bad shape");
  KAD_CHECK_ARG(a->nbranch >= 0 && a->nbranch <= KAD_MAX_BRANCHES, "kad_branch_merge: nbranch %d out of range",
                a->nbranch);
  KAD_CHECK_ARG(a->layout == KAD_NCHW || a->layout == KAD_NHWC, "kad_branch_merge: bad layout");
  for (int b = 0; b < a->nbranch; ++b) {
    KAD_CHECK_ARG(a->br_z[b], "kad_branch_merge: branch %d has no input", b);
    KAD_CHECK_ARG(a->br_c[b] > 0 && a->br_c_off[b] >= 0 && a->br_c_off[b] + a->br_c[b] <= a->c &&
                      a->br_h[b] > 0 && a->br_w[b] > 0 && a->br_cs[b] >= a->br_c[b],
                  "kad_branch_merge: branch %d has a bad shape", b);
  }
  for (int b = 0; b < a->nbranch; ++b)
    KAD_CHECK_ARG(a->br_h[b] <= a->h && a->br_w[b] <= a->w, "kad_branch_merge: branch %d larger than the output", b);
  hipStream_t st = (hipStream_t)stream;
  // disjoint, ordered channel ranges covering exactly the window: the row kernel (one branch per block)
  bool disjoint = a->nbranch > 0;
  int cover = a->c_begin, nchunks = 0, maxbw = 0;
  for (int b = 0; b < a->nbranch; ++b) {
    disjoint = disjoint && a->br_c_off[b] == cover;
    cover += a->br_c[b];
    nchunks += ceil_div(a->br_c[b], 32);
    maxbw = a->br_w[b] > maxbw ? a->br_w[b] : maxbw;
  }
  disjoint = disjoint && cover == a->c_end;
  const int tsz = a->dtype == KAD_F32 ? 4 : 2;
  const size_t row_lds = (size_t)2 * maxbw * 40 * tsz + (size_t)32 * ceil_div(a->w, 4) * 4 * tsz;
  // band kernel: rows of the longest run of MB_E pixels, and the source rows they sample
  const int64_t P = (int64_t)a->h * a->w;
  const int run_rows = ceil_div(MB_E, a->w) + 1;
  int srows_cap = 0, ngroups = 0;
  bool band = a->layout == KAD_NCHW && disjoint && P % 8 == 0 && P < (1ll << 23) &&  // float pixel -> row exact
              ((uintptr_t)a->out % 16) == 0 && ((uintptr_t)a->residual % 16) == 0;
  for (int b = 0; b < a->nbranch; ++b) {
    const int r = (int)((double)(run_rows - 1) * a->br_h[b] / a->h) + 3;
    srows_cap = r > srows_cap ? r : srows_cap;
    ngroups += ceil_div(a->br_c[b], 8);
    band = band && a->br_cs[b] % 8 == 0 && a->br_cs[b] >= round_up(a->br_c[b], 8) &&
           ((uintptr_t)a->br_z[b] % (8 * tsz)) == 0;
  }
  const size_t band_lds = (size_t)8 * srows_cap * maxbw * sizeof(float);
  const int nruns = ceil_div((int)P, MB_E);
  if (band && band_lds <= 64 * 1024 && (int64_t)nruns * ngroups * a->n * 8 < (1ll << 31)) {
    const int grid8 = round_up(nruns * ngroups * a->n, 8);
    dim3 grid(grid8);
    switch (a->dtype) {
      case KAD_F32: hipLaunchKernelGGL(merge_band_kernel<float>, grid, dim3(256), band_lds, st, *a, srows_cap, maxbw, nruns, ngroups, grid8); break;
      case KAD_F16: hipLaunchKernelGGL(merge_band_kernel<half_t>, grid, dim3(256), band_lds, st, *a, srows_cap, maxbw, nruns, ngroups, grid8); break;
      case KAD_BF16: hipLaunchKernelGGL(merge_band_kernel<bf16_t>, grid, dim3(256), band_lds, st, *a, srows_cap, maxbw, nruns, ngroups, grid8); break;
      default: return fail(KAD_EINVAL, "kad_branch_merge: unknown dtype %d", a->dtype);
    }
  } else if (a->layout == KAD_NCHW && disjoint && row_lds <= 64 * 1024) {
    dim3 grid(a->h, nchunks, a->n);
    switch (a->dtype) {
      case KAD_F32: hipLaunchKernelGGL(merge_rows_kernel<float>, grid, dim3(256), row_lds, st, *a); break;
      case KAD_F16: hipLaunchKernelGGL(merge_rows_kernel<half_t>, grid, dim3(256), row_lds, st, *a); break;
      case KAD_BF16: hipLaunchKernelGGL(merge_rows_kernel<bf16_t>, grid, dim3(256), row_lds, st, *a); break;
      default: return fail(KAD_EINVAL, "kad_branch_merge: unknown dtype %d", a->dtype);
    }
  } else if (a->layout == KAD_NCHW) {
    dim3 grid(ceil_div(a->w, MG_XS), a->h, a->n * ceil_div(a->c_end - a->c_begin, MG_CH));
    switch (a->dtype) {
      case KAD_F32: hipLaunchKernelGGL(merge_nchw_kernel<float>, grid, dim3(256), 0, st, *a); break;
      case KAD_F16: hipLaunchKernelGGL(merge_nchw_kernel<half_t>, grid, dim3(256), 0, st, *a); break;
      case KAD_BF16: hipLaunchKernelGGL(merge_nchw_kernel<bf16_t>, grid, dim3(256), 0, st, *a); break;
      default: return fail(KAD_EINVAL, "kad_branch_merge: unknown dtype %d", a->dtype);
    }
  } else if (a->layout == KAD_NHWC && a->out_cs % 8 == 0 && a->res_cs % 8 == 0 && a->c_begin % 8 == 0 &&
             a->c_end % 8 == 0 && ((uintptr_t)a->out % 16) == 0 && ((uintptr_t)a->residual % 16) == 0 &&
             (int64_t)a->n * a->h * a->w < ((int64_t)1 << 31) - 64) {
    const int npix = a->n * a->h * a->w;
    const int ngroups = (a->c_end - a->c_begin) / 8;
    const int blocks = round_up(ceil_div(npix, 64), 8);
    const int threads = 64 * (ngroups < 8 ? ngroups : 8);
    switch (a->dtype) {
      case KAD_F32: hipLaunchKernelGGL(merge_nhwc_vec_kernel<float>, dim3(blocks), dim3(threads), 0, st, *a, npix, ngroups); break;
      case KAD_F16: hipLaunchKernelGGL(merge_nhwc_vec_kernel<half_t>, dim3(blocks), dim3(threads), 0, st, *a, npix, ngroups); break;
      case KAD_BF16: hipLaunchKernelGGL(merge_nhwc_vec_kernel<bf16_t>, dim3(blocks), dim3(threads), 0, st, *a, npix, ngroups); break;
      default: return fail(KAD_EINVAL, "kad_branch_merge: unknown dtype %d", a->dtype);
    }
  } else {
    dim3 grid(a->h, a->n);
    switch (a->dtype) {
      case KAD_F32: hipLaunchKernelGGL(merge_nhwc_kernel<float>, grid, dim3(256), 0, st, *a); break;
      case KAD_F16: hipLaunchKernelGGL(merge_nhwc_kernel<half_t>, grid, dim3(256), 0, st, *a); break;
      case KAD_BF16: hipLaunchKernelGGL(merge_nhwc_kernel<bf16_t>, grid, dim3(256), 0, st, *a); break;
      default: return fail(KAD_EINVAL, "kad_branch_merge: unknown dtype %d", a->dtype);
    }
  }
  return check_launch("kad_branch_merge");
}

extern "C" int kad_nhwc_pad(const void* x, int x_cs, void* out, int out_cs, int n, int c, int h, int w, int dtype,
                            void* stream) {
  KAD_CHECK_ARG(x && out, "kad_nhwc_pad: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0 && x_cs >= c && out_cs >= c && out_cs % 8 == 0,
                "kad_nhwc_pad: bad shape (n %d, c %d, %dx%d, x_cs %d, out_cs %d: need x_cs, out_cs >= c, out_cs %% 8 == 0)",
                n, c, h, w, x_cs, out_cs);
  KAD_CHECK_ARG(dtype == KAD_F16 || dtype == KAD_BF16 || dtype == KAD_F32, "kad_nhwc_pad: unknown dtype %d", dtype);
  KAD_CHECK_ARG((uintptr_t)out % 16 == 0, "kad_nhwc_pad: out must be 16-byte aligned");
  const int64_t pixels = (int64_t)n * h * w;
  hipStream_t st = (hipStream_t)stream;
  const int grid = grid_for(pixels * (out_cs / 8));
  if (dtype == KAD_F16)
    hipLaunchKernelGGL(nhwc_pad_kernel<half_t>, dim3(grid), dim3(256), 0, st, (const half_t*)x, (half_t*)out, c, x_cs,
                       out_cs, pixels);
  else if (dtype == KAD_F32)
    hipLaunchKernelGGL(nhwc_pad_kernel<float>, dim3(grid), dim3(256), 0, st, (const float*)x, (float*)out, c, x_cs,
                       out_cs, pixels);
  else
    hipLaunchKernelGGL(nhwc_pad_kernel<bf16_t>, dim3(grid), dim3(256), 0, st, (const bf16_t*)x, (bf16_t*)out, c, x_cs,
                       out_cs, pixels);
  return check_launch("kad_nhwc_pad");
}

extern "C" int kad_to_nhwc(const void* x, void* out, int n, int c, int h, int w, int out_cs, int dtype,
                           void* stream) {
  KAD_CHECK_ARG(x && out, "kad_to_nhwc: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0 && out_cs >= c, "kad_to_nhwc: bad shape");
  const int P = h * w;
  dim3 grid(ceil_div(P, 64), ceil_div(out_cs, 64), n);
  hipStream_t st = (hipStream_t)stream;
  const int64_t tiles = (int64_t)ceil_div(P, 64) * ceil_div(out_cs, 64) * n;
  if (dtype != KAD_F32 && P % 8 == 0 && out_cs % 8 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0 &&
      tiles * 8 < (1ll << 31)) {
    const int npt = ceil_div(P, 64), nct = ceil_div(out_cs, 64), total = (int)tiles, grid8 = round_up(total, 8);
    if (dtype == KAD_F16)
      hipLaunchKernelGGL(to_nhwc_v8_kernel<half_t>, dim3(grid8), dim3(256), 0, st, (const half_t*)x, (half_t*)out, c,
                         P, out_cs, npt, nct, total, grid8);
    else if (dtype == KAD_BF16)
      hipLaunchKernelGGL(to_nhwc_v8_kernel<bf16_t>, dim3(grid8), dim3(256), 0, st, (const bf16_t*)x, (bf16_t*)out, c,
                         P, out_cs, npt, nct, total, grid8);
    else
      return fail(KAD_EINVAL, "kad_to_nhwc: unknown dtype %d", dtype);
    return check_launch("kad_to_nhwc");
  }
  switch (dtype) {
    case KAD_F32: hipLaunchKernelGGL(to_nhwc_kernel<float>, grid, dim3(256), 0, st, (const float*)x, (float*)out, c, P, out_cs); break;
    case KAD_F16: hipLaunchKernelGGL(to_nhwc_kernel<half_t>, grid, dim3(256), 0, st, (const half_t*)x, (half_t*)out, c, P, out_cs); break;
    case KAD_BF16: hipLaunchKernelGGL(to_nhwc_kernel<bf16_t>, grid, dim3(256), 0, st, (const bf16_t*)x, (bf16_t*)out, c, P, out_cs); break;
    default: return fail(KAD_EINVAL, "kad_to_nhwc: unknown dtype %d", dtype);
  }
  return check_launch("kad_to_nhwc");
}
