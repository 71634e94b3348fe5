// Depthwise 3-D convolution (channel-last) for gfx950, forward and backward.
//
// Restates nn.Conv3d(C, C, (kt, kh, kw), padding=(kt/2, kh/2, kw/2), groups=C)
// with zero padding, as the reference uses it for dw_conv
// (infinity/video/attention.py:58-65) and offset_net[0] (:71), optionally
// followed by exact-erf GELU (offset_net[1], :72):
//   z[p, c] = b[c] + sum_tap w[c, tap] x[p + tap - pad, c],  y = act(z).
// Backward: dz = dy * act'(z) (z recomputed), dx[r] = sum_tap w[tap] dz[r - tap + pad],
// dw[c, tap] = sum_p dz[p, c] x[p + tap - pad, c], db[c] = sum_p dz[p, c].
#include "common.h"

namespace msd {

namespace {

struct ConvArgs {
  int B, T, H, W, C, kt, kh, kw;
  int64_t N;
};

// One thread per output element (token, channel); consecutive threads take
// consecutive channels so x loads coalesce along C.
template <typename T, bool GELU>
__global__ __launch_bounds__(256) void dwconv3d_fwd_kernel(ConvArgs a, const T* __restrict__ x,
                                                           const T* __restrict__ wt,
                                                           const T* __restrict__ bias,
                                                           T* __restrict__ y) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(a.B) * a.N * a.C;
  if (i >= total) return;
  const int c = static_cast<int>(i % a.C);
  const int64_t bn = i / a.C;
  const int b = static_cast<int>(bn / a.N);
  const int64_t n = bn - static_cast<int64_t>(b) * a.N;
  const int w = static_cast<int>(n % a.W);
  const int h = static_cast<int>((n / a.W) % a.H);
  const int t = static_cast<int>(n / (static_cast<int64_t>(a.W) * a.H));
  const int K = a.kt * a.kh * a.kw;
  const T* __restrict__ wc = wt + static_cast<int64_t>(c) * K;
  float acc = bias != nullptr ? ld(bias, c) : 0.0f;
  int tap = 0;
  for (int dt = 0; dt < a.kt; ++dt) {
    const int tt = t + dt - a.kt / 2;
    for (int dh = 0; dh < a.kh; ++dh) {
      const int hh = h + dh - a.kh / 2;
      for (int dw = 0; dw < a.kw; ++dw, ++tap) {
        const int ww = w + dw - a.kw / 2;
        if (tt < 0 || tt >= a.T || hh < 0 || hh >= a.H || ww < 0 || ww >= a.W) continue;
        const int64_t r = static_cast<int64_t>(b) * a.N + (static_cast<int64_t>(tt) * a.H + hh) * a.W + ww;
        acc += ld(wc, tap) * ld(x, r * a.C + c);
      }
    }
  }
  st(y, i, GELU ? gelu_erf(acc) : acc);
}

// dz = dy * gelu'(z) with z recomputed; written as fp32.
template <typename T>
__global__ __launch_bounds__(256) void dwconv3d_gelu_dz_kernel(ConvArgs a, const T* __restrict__ x,
                                                               const T* __restrict__ wt,
                                                               const T* __restrict__ bias,
                                                               const T* __restrict__ dy,
                                                               float* __restrict__ dz) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(a.B) * a.N * a.C;
  if (i >= total) return;
  const int c = static_cast<int>(i % a.C);
  const int64_t bn = i / a.C;
  const int b = static_cast<int>(bn / a.N);
  const int64_t n = bn - static_cast<int64_t>(b) * a.N;
  const int w = static_cast<int>(n % a.W);
  const int h = static_cast<int>((n / a.W) % a.H);
  const int t = static_cast<int>(n / (static_cast<int64_t>(a.W) * a.H));
  const int K = a.kt * a.kh * a.kw;
  const T* __restrict__ wc = wt + static_cast<int64_t>(c) * K;
  float z = bias != nullptr ? ld(bias, c) : 0.0f;
  int tap = 0;
  for (int dt = 0; dt < a.kt; ++dt) {
    const int tt = t + dt - a.kt / 2;
    for (int dh = 0; dh < a.kh; ++dh) {
      const int hh = h + dh - a.kh / 2;
      for (int dw = 0; dw < a.kw; ++dw, ++tap) {
        const int ww = w + dw - a.kw / 2;
        if (tt < 0 || tt >= a.T || hh < 0 || hh >= a.H || ww < 0 || ww >= a.W) continue;
        const int64_t r = static_cast<int64_t>(b) * a.N + (static_cast<int64_t>(tt) * a.H + hh) * a.W + ww;
        z += ld(wc, tap) * ld(x, r * a.C + c);
      }
    }
  }
  dz[i] = ld(dy, i) * gelu_erf_grad(z);
}

// dx[r, c] = sum_tap w[c, tap] dz[r - tap + pad, c]
template <typename T, typename G>
__global__ __launch_bounds__(256) void dwconv3d_dx_kernel(ConvArgs a, const G* __restrict__ dz,
                                                          const T* __restrict__ wt,
                                                          T* __restrict__ dx) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(a.B) * a.N * a.C;
  if (i >= total) return;
  const int c = static_cast<int>(i % a.C);
  const int64_t bn = i / a.C;
  const int b = static_cast<int>(bn / a.N);
  const int64_t n = bn - static_cast<int64_t>(b) * a.N;
  const int w = static_cast<int>(n % a.W);
  const int h = static_cast<int>((n / a.W) % a.H);
  const int t = static_cast<int>(n / (static_cast<int64_t>(a.W) * a.H));
  const int K = a.kt * a.kh * a.kw;
  const T* __restrict__ wc = wt + static_cast<int64_t>(c) * K;
  float acc = 0.0f;
  int tap = 0;
  for (int dt = 0; dt < a.kt; ++dt) {
    const int tt = t - dt + a.kt / 2;
    for (int dh = 0; dh < a.kh; ++dh) {
      const int hh = h - dh + a.kh / 2;
      for (int dw = 0; dw < a.kw; ++dw, ++tap) {
        const int ww = w - dw + a.kw / 2;
        if (tt < 0 || tt >= a.T || hh < 0 || hh >= a.H || ww < 0 || ww >= a.W) continue;
        const int64_t r = static_cast<int64_t>(b) * a.N + (static_cast<int64_t>(tt) * a.H + hh) * a.W + ww;
        acc += ld(wc, tap) * ld(dz, r * a.C + c);
      }
    }
  }
  st(dx, i, acc);
}

// Partial weight/bias gradients: block (channel tile, tap, token chunk); each
// thread one channel; fp32 atomics into acc[c * (K + 1) + tap], tap == K is the bias.
constexpr int kChunk = 512;

template <typename T, typename G>
__global__ __launch_bounds__(64) void dwconv3d_dw_kernel(ConvArgs a, const T* __restrict__ x,
                                                         const G* __restrict__ dz,
                                                         float* __restrict__ acc) {
  const int c = blockIdx.x * 64 + threadIdx.x;
  const int tap = blockIdx.y;
  const int K = a.kt * a.kh * a.kw;
  if (c >= a.C) return;
  const int64_t rows = static_cast<int64_t>(a.B) * a.N;
  const int64_t r0 = static_cast<int64_t>(blockIdx.z) * kChunk;
  const int64_t r1 = r0 + kChunk < rows ? r0 + kChunk : rows;
  float s = 0.0f;
  if (tap == K) {
    for (int64_t r = r0; r < r1; ++r) s += ld(dz, r * a.C + c);
  } else {
    const int dt = tap / (a.kh * a.kw) - a.kt / 2;
    const int dh = (tap / a.kw) % a.kh - a.kh / 2;
    const int dw = tap % a.kw - a.kw / 2;
    for (int64_t r = r0; r < r1; ++r) {
      const int b = static_cast<int>(r / a.N);
      const int64_t n = r - static_cast<int64_t>(b) * a.N;
      const int w = static_cast<int>(n % a.W) + dw;
      const int h = static_cast<int>((n / a.W) % a.H) + dh;
      const int t = static_cast<int>(n / (static_cast<int64_t>(a.W) * a.H)) + dt;
      if (t < 0 || t >= a.T || h < 0 || h >= a.H || w < 0 || w >= a.W) continue;
      const int64_t rs = static_cast<int64_t>(b) * a.N + (static_cast<int64_t>(t) * a.H + h) * a.W + w;
      s += ld(dz, r * a.C + c) * ld(x, rs * a.C + c);
    }
  }
  atomicAdd(acc + static_cast<int64_t>(c) * (K + 1) + tap, s);
}

template <typename T>
__global__ __launch_bounds__(256) void dwconv3d_dw_finish_kernel(const float* __restrict__ acc,
                                                                 int C, int K, T* __restrict__ dw,
                                                                 T* __restrict__ db) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(C) * (K + 1)) return;
  const int c = static_cast<int>(i / (K + 1));
  const int tap = static_cast<int>(i - static_cast<int64_t>(c) * (K + 1));
  if (tap < K) {
    if (dw != nullptr) st(dw, static_cast<int64_t>(c) * K + tap, acc[i]);
  } else if (db != nullptr) {
    st(db, c, acc[i]);
  }
}

ConvArgs make_args(const msd_dwconv3d_desc& d) {
  ConvArgs a;
  a.B = d.B;
  a.T = d.T;
  a.H = d.H;
  a.W = d.W;
  a.C = d.C;
  a.kt = d.kt;
  a.kh = d.kh;
  a.kw = d.kw;
  a.N = static_cast<int64_t>(d.T) * d.H * d.W;
  return a;
}

template <typename T>
hipError_t fwd_typed(const msd_dwconv3d_desc& d, const void* x, const void* w, const void* b,
                     void* y, hipStream_t s) {
  const ConvArgs a = make_args(d);
  const int64_t total = static_cast<int64_t>(a.B) * a.N * a.C;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  if (d.act == 1)
    hipLaunchKernelGGL((dwconv3d_fwd_kernel<T, true>), grid, dim3(256), 0, s, a,
                       static_cast<const T*>(x), static_cast<const T*>(w),
                       static_cast<const T*>(b), static_cast<T*>(y));
  else
    hipLaunchKernelGGL((dwconv3d_fwd_kernel<T, false>), grid, dim3(256), 0, s, a,
                       static_cast<const T*>(x), static_cast<const T*>(w),
                       static_cast<const T*>(b), static_cast<T*>(y));
  return hipGetLastError();
}

template <typename T, typename G>
hipError_t bwd_grads(const ConvArgs& a, const void* x, const void* w, const G* dz, void* dx,
                     void* dw, void* db, float* acc, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.N;
  const int64_t total = rows * a.C;
  const int K = a.kt * a.kh * a.kw;
  if (dx != nullptr) {
    hipLaunchKernelGGL((dwconv3d_dx_kernel<T, G>), dim3(static_cast<unsigned>((total + 255) / 256)),
                       dim3(256), 0, s, a, dz, static_cast<const T*>(w), static_cast<T*>(dx));
  }
  if (dw != nullptr || db != nullptr) {
    const int64_t nacc = static_cast<int64_t>(a.C) * (K + 1);
    hipLaunchKernelGGL(fill_zero_f32, dim3(fill_blocks(nacc)), dim3(256), 0, s, acc, nacc);
    const dim3 grid(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(K + 1),
                    static_cast<unsigned>((rows + kChunk - 1) / kChunk));
    hipLaunchKernelGGL((dwconv3d_dw_kernel<T, G>), grid, dim3(64), 0, s, a,
                       static_cast<const T*>(x), dz, acc);
    hipLaunchKernelGGL((dwconv3d_dw_finish_kernel<T>), dim3(static_cast<unsigned>((nacc + 255) / 256)),
                       dim3(256), 0, s, acc, a.C, K, static_cast<T*>(dw), static_cast<T*>(db));
  }
  return hipGetLastError();
}

template <typename T>
hipError_t bwd_typed(const msd_dwconv3d_desc& d, const void* x, const void* w, const void* b,
                     const void* dy, void* dx, void* dw, void* db, void* ws, hipStream_t s) {
  const ConvArgs a = make_args(d);
  const int K = a.kt * a.kh * a.kw;
  float* acc = static_cast<float*>(ws);
  const int64_t nacc = static_cast<int64_t>(a.C) * (K + 1);
  if (d.act == 1) {
    float* dz = acc + ((nacc + 63) / 64) * 64;
    const int64_t total = static_cast<int64_t>(a.B) * a.N * a.C;
    hipLaunchKernelGGL((dwconv3d_gelu_dz_kernel<T>), dim3(static_cast<unsigned>((total + 255) / 256)),
                       dim3(256), 0, s, a, static_cast<const T*>(x), static_cast<const T*>(w),
                       static_cast<const T*>(b), static_cast<const T*>(dy), dz);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return bwd_grads<T, float>(a, x, w, dz, dx, dw, db, acc, s);
  }
  return bwd_grads<T, T>(a, x, w, static_cast<const T*>(dy), dx, dw, db, acc, s);
}

}  // namespace

size_t dwconv3d_bwd_ws_bytes(const msd_dwconv3d_desc& d) {
  const int64_t K = static_cast<int64_t>(d.kt) * d.kh * d.kw;
  const int64_t nacc = ((static_cast<int64_t>(d.C) * (K + 1) + 63) / 64) * 64;
  int64_t n = nacc;
  if (d.act == 1) n += static_cast<int64_t>(d.B) * d.T * d.H * d.W * d.C;
  return static_cast<size_t>(n) * sizeof(float);
}

hipError_t launch_dwconv3d_fwd(const msd_dwconv3d_desc& d, const void* x, const void* w,
                               const void* b, void* y, hipStream_t s) {
  if (d.dtype == MSD_BF16) return fwd_typed<bf16>(d, x, w, b, y, s);
  return fwd_typed<float>(d, x, w, b, y, s);
}

hipError_t launch_dwconv3d_bwd(const msd_dwconv3d_desc& d, const void* x, const void* w,
                               const void* b, const void* dy, void* dx, void* dw, void* db,
                               void* ws, hipStream_t s) {
  if (d.dtype == MSD_BF16) return bwd_typed<bf16>(d, x, w, b, dy, dx, dw, db, ws, s);
  return bwd_typed<float>(d, x, w, b, dy, dx, dw, db, ws, s);
}

}  // namespace msd
