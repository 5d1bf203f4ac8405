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
__global__ __launch_bounds__(256) void se_mlp_kernel(const float* partial, int tiles, float inv_count,
                                                    const float* w1, const float* b1, const float* w2,
                                                    const float* b2, float* att, int c, int hid) {
  extern __shared__ float lds[];
  float* g = lds;        // [C]
  float* hbuf = g + c;   // [hid]
  const int n = blockIdx.x;
  for (int ch = threadIdx.x; ch < c; ch += 256) {
    float acc = 0.f;
    for (int t = 0; t < tiles; ++t) acc += partial[((int64_t)n * tiles + t) * c + ch];
    g[ch] = acc * inv_count;
  }
  __syncthreads();
  for (int j = threadIdx.x; j < hid; j += 256) {
    float acc = b1 ? b1[j] : 0.f;
    const float* wr = w1 + (int64_t)j * c;
    for (int ch = 0; ch < c; ++ch) acc += wr[ch] * g[ch];
    hbuf[j] = fmaxf(acc, 0.f);
  }
  __syncthreads();
  for (int ch = threadIdx.x; ch < c; ch += 256) {
    float acc = b2 ? b2[ch] : 0.f;
    const float* wr = w2 + (int64_t)ch * hid;
    for (int j = 0; j < hid; ++j) acc += wr[j] * hbuf[j];
    att[(int64_t)n * c + ch] = sigmoidf_(acc);
  }
}

// ---- channel scale: out[n, c, :] = x[n, c, :] * att[n, c] (NCHW) or per pixel (NHWC) -------
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
__device__ __forceinline__ void src_index(int dst, int in, int out, float scale, int& i0, int& i1, float& l1) {
  if (in == out) {
    i0 = i1 = dst;
    l1 = 0.f;
    return;
  }
  float s = scale * ((float)dst + 0.5f) - 0.5f;
  if (s < 0.f) s = 0.f;
  i0 = (int)s;
  i1 = i0 + ((i0 < in - 1) ? 1 : 0);
  l1 = s - (float)i0;
}

template <typename T>
__global__ __launch_bounds__(256) void merge_kernel(kad_merge_args a) {
  const int64_t total = (int64_t)a.n * a.c * a.h * a.w;
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int n, c, y, x;
    if (a.layout == KAD_NCHW) {
      x = (int)(i % a.w);
      y = (int)((i / a.w) % a.h);
      c = (int)((i / ((int64_t)a.w * a.h)) % a.c);
      n = (int)(i / ((int64_t)a.w * a.h * a.c));
    } else {
      c = (int)(i % a.c);
      x = (int)((i / a.c) % a.w);
      y = (int)((i / ((int64_t)a.c * a.w)) % a.h);
      n = (int)(i / ((int64_t)a.c * a.w * a.h));
    }
    float v = 0.f;
    if (a.residual) v = to_f32(((const T*)a.residual)[i]);
    for (int b = 0; b < a.nbranch; ++b) {
      const int cb = c - a.br_c_off[b];
      if (cb < 0 || cb >= a.br_c[b]) continue;
      const int bh = a.br_h[b], bw = a.br_w[b], bcs = a.br_cs[b];
      const T* z = (const T*)a.br_z[b] + (int64_t)n * bh * bw * bcs + cb;
      int y0, y1, x0, x1;
      float ly, lx;
      src_index(y, bh, a.h, (float)bh / (float)a.h, y0, y1, ly);
      src_index(x, bw, a.w, (float)bw / (float)a.w, x0, x1, lx);
      const float v00 = to_f32(z[((int64_t)y0 * bw + x0) * bcs]);
      const float v01 = to_f32(z[((int64_t)y0 * bw + x1) * bcs]);
      const float v10 = to_f32(z[((int64_t)y1 * bw + x0) * bcs]);
      const float v11 = to_f32(z[((int64_t)y1 * bw + x1) * bcs]);
      float s = (1.f - ly) * ((1.f - lx) * v00 + lx * v01) + ly * ((1.f - lx) * v10 + lx * v11);
      if (a.br_att[b]) s *= a.br_att[b][(int64_t)n * a.br_c[b] + cb];
      v += a.br_coeff[b] * s;
    }
    if (a.gate) v *= a.gate[c];
    ((T*)a.out)[i] = from_f32<T>(v);
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

static int grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  return (int)(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

}  // namespace kad

using namespace kad;

extern "C" int kad_se_pool(const void* x, float* partial, int n, int c, int h, int w, int layout, int x_cs,
                           int dtype, void* stream) {
  KAD_CHECK_ARG(x && partial, "kad_se_pool: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0, "kad_se_pool: bad shape");
  hipStream_t st = (hipStream_t)stream;
  const int P = h * w;
  if (layout == KAD_NCHW) {
    const int planes = n * c;
    dim3 grid(ceil_div(planes, 4));
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
  const size_t lds = (size_t)(c + hid) * sizeof(float);
  KAD_CHECK_ARG(lds <= 64 * 1024, "kad_se_mlp: C + hidden too large");
  hipLaunchKernelGGL(se_mlp_kernel, dim3(n), dim3(256), lds, (hipStream_t)stream, partial, tiles, inv_count, w1, b1,
                     w2, b2, att, c, hid);
  return check_launch("kad_se_mlp");
}

extern "C" int kad_channel_scale(const void* x, const float* att, void* out, int n, int c, int h, int w, int layout,
                                 int x_cs, int dtype, void* stream) {
  KAD_CHECK_ARG(x && att && out, "kad_channel_scale: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0, "kad_channel_scale: bad shape");
  const int cs = layout == KAD_NHWC ? x_cs : c;
  KAD_CHECK_ARG(cs >= c, "kad_channel_scale: channel stride < C");
  const int64_t total = (int64_t)n * h * w * cs;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case KAD_F32: hipLaunchKernelGGL(channel_scale_kernel<float>, dim3(grid_for(total)), dim3(256), 0, st, (const float*)x, att, (float*)out, total, c, h * w, layout, cs); break;
    case KAD_F16: hipLaunchKernelGGL(channel_scale_kernel<half_t>, dim3(grid_for(total)), dim3(256), 0, st, (const half_t*)x, att, (half_t*)out, total, c, h * w, layout, cs); break;
    case KAD_BF16: hipLaunchKernelGGL(channel_scale_kernel<bf16_t>, dim3(grid_for(total)), dim3(256), 0, st, (const bf16_t*)x, att, (bf16_t*)out, total, c, h * w, layout, cs); break;
    default: return fail(KAD_EINVAL, "kad_channel_scale: unknown dtype %d", dtype);
  }
  return check_launch("kad_channel_scale");
}

extern "C" int kad_branch_merge(const kad_merge_args* a, void* stream) {
  KAD_CHECK_ARG(a && a->out, "kad_branch_merge: null pointer");
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
  const int64_t total = (int64_t)a->n * a->c * a->h * a->w;
  hipStream_t st = (hipStream_t)stream;
  switch (a->dtype) {
    case KAD_F32: hipLaunchKernelGGL(merge_kernel<float>, dim3(grid_for(total)), dim3(256), 0, st, *a); break;
    case KAD_F16: hipLaunchKernelGGL(merge_kernel<half_t>, dim3(grid_for(total)), dim3(256), 0, st, *a); break;
    case KAD_BF16: hipLaunchKernelGGL(merge_kernel<bf16_t>, dim3(grid_for(total)), dim3(256), 0, st, *a); break;
    default: return fail(KAD_EINVAL, "kad_branch_merge: unknown dtype %d", a->dtype);
  }
  return check_launch("kad_branch_merge");
}

extern "C" int kad_to_nhwc(const void* x, void* out, int n, int c, int h, int w, int out_cs, int dtype,
                           void* stream) {
  KAD_CHECK_ARG(x && out, "kad_to_nhwc: null pointer");
  KAD_CHECK_ARG(n > 0 && c > 0 && h > 0 && w > 0 && out_cs >= c, "kad_to_nhwc: bad shape");
  const int P = h * w;
  dim3 grid(ceil_div(P, 64), ceil_div(out_cs, 64), n);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case KAD_F32: hipLaunchKernelGGL(to_nhwc_kernel<float>, grid, dim3(256), 0, st, (const float*)x, (float*)out, c, P, out_cs); break;
    case KAD_F16: hipLaunchKernelGGL(to_nhwc_kernel<half_t>, grid, dim3(256), 0, st, (const half_t*)x, (half_t*)out, c, P, out_cs); break;
    case KAD_BF16: hipLaunchKernelGGL(to_nhwc_kernel<bf16_t>, grid, dim3(256), 0, st, (const bf16_t*)x, (bf16_t*)out, c, P, out_cs); break;
    default: return fail(KAD_EINVAL, "kad_to_nhwc: unknown dtype %d", dtype);
  }
  return check_launch("kad_to_nhwc");
}
