// Shared device helpers for the gfx950 3D-DSA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

#include "dropout.h"
#include "megaslide_dsa3d.h"

namespace msd {

// Kernel-side dropout parameters of a call (threshold 0 = off).
inline DropoutArgs dropout_args(const msd_dsa3d_desc& d) {
  DropoutArgs r{};
  if (d.dropout_p > 0.0f) {
    const double t = std::floor(static_cast<double>(d.dropout_p) * 4294967296.0);
    r.threshold = t >= 4294967295.0 ? 0xFFFFFFFFu : static_cast<uint32_t>(t);
    r.scale = 1.0f / (1.0f - d.dropout_p);
  }
  r.key0 = static_cast<uint32_t>(d.dropout_seed);
  r.key1 = static_cast<uint32_t>(d.dropout_seed >> 32);
  r.offset = d.dropout_offset;
  return r;
}

// ---------------------------------------------------------------------------
// element types: fp32 and bf16 stored as raw 16-bit words
// ---------------------------------------------------------------------------

struct bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);

template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }

// Round to nearest even; NaN stays a quiet NaN.
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  uint32_t u = __float_as_uint(v);
  bf16 r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = static_cast<uint16_t>((u >> 16) | 0x40u);
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    r.bits = static_cast<uint16_t>(u >> 16);
  }
  return r;
}

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }

template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = from_f32<T>(v); }

// Exact-erf GELU (nn.GELU() default) and its derivative.
__device__ __forceinline__ float gelu_erf(float z) {
  return 0.5f * z * (1.0f + erff(z * 0.70710678118654752440f));
}
__device__ __forceinline__ float gelu_erf_grad(float z) {
  const float cdf = 0.5f * (1.0f + erff(z * 0.70710678118654752440f));
  const float pdf = 0.39894228040143267794f * __expf(-0.5f * z * z);
  return cdf + z * pdf;
}

// Sum over aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = G / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, G);
  return v;
}

// Fill a float buffer with zeros (a kernel, not hipMemsetAsync, so that the
// call stays correct inside captured graphs).  Grid-stride loop.
static __global__ void fill_zero_f32(float* __restrict__ p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0.0f;
}

inline unsigned fill_blocks(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return static_cast<unsigned>(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

}  // namespace msd

// Internal launchers (defined in dsa3d.hip / dwconv3d.hip), called by abi.cpp
// after argument validation.  They return a hipError_t.
namespace msd {
hipError_t launch_dsa3d_fwd_direct(const msd_dsa3d_desc& d, const void* q, const void* k,
                                   const void* v, const void* off, const void* ek, const void* ev,
                                   void* out, float* lse, hipStream_t s);
hipError_t launch_dsa3d_bwd_direct(const msd_dsa3d_desc& d, const void* q, const void* k,
                                   const void* v, const void* off, const void* ek, const void* ev,
                                   const void* out, const void* dout, const float* lse,
                                   const float* dlse, void* dq, void* dk, void* dv, void* doff,
                                   void* dek, void* dev, void* ws, hipStream_t s);
bool dsa3d_tiled_supported(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v);
hipError_t launch_dsa3d_fwd_tiled(const msd_dsa3d_desc& d, const void* q, const void* k,
                                  const void* v, const void* off, const void* ek, const void* ev,
                                  void* out, float* lse, hipStream_t s);
hipError_t launch_dsa3d_bwd_tiled(const msd_dsa3d_desc& d, const void* q, const void* k,
                                  const void* v, const void* off, const void* ek, const void* ev,
                                  const void* out, const void* dout, const float* lse,
                                  const float* dlse, void* dq, void* dk, void* dv, void* doff,
                                  void* dek, void* dev, void* ws, hipStream_t s);
size_t dsa3d_bwd_ws_bytes(const msd_dsa3d_desc& d);
size_t dsa3d_tiled_bwd_ws_bytes(const msd_dsa3d_desc& d);
hipError_t launch_dwconv3d_fwd(const msd_dwconv3d_desc& d, const void* x, const void* w,
                               const void* b, void* y, void* z, hipStream_t s);
hipError_t launch_dwconv3d_bwd(const msd_dwconv3d_desc& d, const void* x, const void* w,
                               const void* b, const void* z, const void* dy, void* dx, void* dw,
                               void* db, void* ws, hipStream_t s);
size_t dwconv3d_bwd_ws_bytes(const msd_dwconv3d_desc& d);
int dsa3d_max_head_dim();
}  // namespace msd
