// Shared definitions for the KAD-Conv gfx950 HIP library.
//
// Conventions used by every kernel in this library:
//  * Feature maps handed between kernels are NHWC with a channel stride that is
//    a multiple of 8 elements (16 bytes for fp16/bf16); the stride's padding
//    channels hold zeros, so 16-byte vector loads never need a tail case.
//  * Per-pixel side tensors (offsets, masks) are fp32, addressed through
//    explicit (image, pixel, channel) strides so both pixel-major [N, P, C] and
//    torchvision's plane-major [N, C, P] layouts are read in place.
//  * Accumulation is fp32 everywhere; fp16/bf16 only at storage and MFMA inputs.
//  * Entry points never allocate, never synchronise, and launch on the stream
//    they are given; they return 0 or a negative KAD_E* code and record a
//    message retrievable with kad_last_error() (thread-local).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kadconv_hip.h"

namespace kad {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16_t;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef int intx4 __attribute__((ext_vector_type(4)));

int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(half_t v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ half_t from_f32<half_t>(float v) { return (half_t)v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) { return (bf16_t)v; }

// Logistic function built on the HIP device expf.  1 / d (d = 1 + e^-v >= 1) as the hardware
// reciprocal plus one Newton step, r + r (1 - d r): the correctly rounded quotient but for rare
// last-bit cases, at a third of the instructions of the IEEE division (the epilogues of the
// 1x1 GEMM and 3x3 conv are bound by this SiLU).  d = inf (v < -88.7) gives 0, as 1 / inf does.
__device__ __forceinline__ float sigmoidf_(float v) {
  const float d = 1.0f + __expf(-v);
  const float r = __builtin_amdgcn_rcpf(d);
  const float q = __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
  return d == __builtin_inff() ? 0.0f : q;
}

// Cross-block exchange inside one kernel (8 XCDs, each with its own L2): a relaxed device-scope
// atomic load or exchange is performed at the memory-side coherence point, so it neither returns
// a stale line of the reader's L2 nor leaves the value in the writer's.  rmw_store uses the
// returning form and consumes the result, so the thread's wait for it covers the store.
__device__ __forceinline__ float dev_load(const float* p) {
  return __uint_as_float(__hip_atomic_load((const unsigned*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void rmw_store(float* p, float v) {
  const unsigned old = __hip_atomic_exchange((unsigned*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::"v"(old));
}

// Raw buffer access: a load at a byte offset at or past the descriptor's size
// returns 0 (no fault), so out-of-range pieces need no branch.  Offsets are
// 32-bit: callers keep the addressed range below 2^31 bytes, which keeps
// KAD_OOB out of range.  A descriptor must be wave-uniform.
constexpr uint32_t KAD_OOB = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Buffer -> LDS loads of 16 / 4 bytes per lane: lane i's bytes land at
// dst + size * i (dst wave-uniform); the global address is base + soffset
// (wave-uniform) + voff (per lane).  They count in vmcnt like other loads.
// __syncthreads() fences wait for all of them (vmcnt(0)); a software pipeline
// waits for its own stage with an explicit s_waitcnt and a bare s_barrier, and
// keeps each stage in a __shared__ object of its own so that the compiler's
// wait counts for LDS reads stay per stage.
#define KAD_LDS(p) ((__attribute__((address_space(3))) void*)(p))
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, KAD_LDS(dst), 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, char* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, KAD_LDS(dst), 4, voff, soff, 0, 0);
}

// v summed over lanes l and l ^ 16 (sum_xor16) or l and l ^ 32 (sum_xor32) of the wave,
// on the VALU: v_permlane16_swap / v_permlane32_swap of v with itself leaves every lane
// holding its own value and its partner's, in one order or the other (a + b == b + a, so
// the sum equals v + __shfl_xor(v, 16 / 32) bit for bit, without an LDS-path round trip).
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Bilinear resize source index (PyTorch, align_corners=False, output size
// given): s = max(scale * (dst + 0.5) - 0.5, 0) with scale = in / out; rows
// i0 = floor(s) and i1 = min(i0 + 1, in - 1), weight of i1 = s - i0.
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

// 8 consecutive elements, moved as 16-byte (16-bit types) or 2 x 16-byte (fp32) pieces.
template <typename T> struct alignas(16) Vec8 { T v[8]; };

__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ inline int round_up(int a, int b) { return ceil_div(a, b) * b; }

// Raise a kernel's dynamic-LDS limit above the 64 KB default when it needs
// more (gfx950 has 160 KB per CU).  Host-side attribute, not a stream op.
template <typename F>
inline void allow_lds(F* kernel, size_t bytes) {
  if (bytes > 64 * 1024)
    (void)hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

// kad_conv_fwd's 16-bit NHWC-output path (kad_conv3.hip): returns 1 when the launch is not one it
// handles (the caller then runs its general path), else 0 or a KAD_E* code.
int convolution_igemm(const kad_dcn_args& a, int ho, int wo, hipStream_t st);

inline int dtype_size(int dtype) {
  return dtype == KAD_F32 ? 4 : 2;
}

}  // namespace kad

#define KAD_CHECK_ARG(cond, ...) \
  do { if (!(cond)) return ::kad::fail(KAD_EINVAL, __VA_ARGS__); } while (0)
