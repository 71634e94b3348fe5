// Depthwise 3-D convolution (channel-last) for gfx950, forward and backward.
//
// Restates nn.Conv3d(C, C, (kt, kh, kw), padding=(kt/2, kh/2, kw/2), groups=C)
// with zero padding, as the reference uses it for dw_conv
// (infinity/video/attention.py:58-65) and offset_net[0] (:71), optionally
// followed by exact-erf GELU (offset_net[1], :72):
//   z[p, c] = b[c] + sum_tap w[c, tap] x[p + tap - pad, c],  y = act(z).
// Backward: dz = dy * act'(z) (z recomputed), dx = conv(dz, flipped w),
// dw[c, tap] = sum_p dz[p, c] x[p + tap - pad, c], db[c] = sum_p dz[p, c].
//
// Row kernels (kw in {3, 5, 7}, kt, kh <= 7): a thread owns one channel and a
// run of kRun consecutive outputs along W; for every (dt, dh) it loads the
// input row segment once into registers (kRun + kw - 1 values) and applies the
// kw taps to all kRun outputs.  A wave covers 64 consecutive channels, so every
// load is one 128-byte (bf16) or 256-byte (fp32) segment.  The weight-gradient
// kernel keeps all kt*kh*kw tap sums of its channel in registers over a strip
// of rows and flushes them with one fp32 atomic per (thread, tap).  With bf16
// data, kw in {5, 7} and channels a multiple of 8, the weight gradient runs on
// the matrix cores instead (dwconv_dw_mfma_kernel).
// Other odd kernel sizes use the simple one-output-per-thread kernels.
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace msd {

namespace {

struct ConvArgs {
  int B, T, H, W, C, kt, kh, kw;
  int64_t N;
};

constexpr int kRun = 16;        // outputs per thread along W
constexpr int kRowWaves = 4;    // waves per block in the row kernels
constexpr int kStripRows = 8;   // (b, t, h) rows per weight-gradient work item

enum Epilogue { kPlain = 0, kGelu = 1, kGeluGrad = 2, kGeluGradT = 3, kGeluSave = 4 };

// ---------------------------------------------------------------------------
// row kernels: forward, GELU-gradient recompute, input gradient
// ---------------------------------------------------------------------------

// out[p] = epilogue(sum_tap w[tap'] in[p + tap - pad]) with tap' = tap, or the
// mirrored tap K-1-tap when flip (input gradient of the convolution).
// mode kGeluGrad writes dz = dy * gelu'(z) as fp32 into out2, kGeluGradT in
// the element type into out; kGeluSave writes gelu(z) into out and the
// pre-activation z (element type) into out2.
template <typename T, typename G, int KW, int MODE>
__global__ __launch_bounds__(64 * kRowWaves) void dwconv_rows_kernel(
    ConvArgs a, const G* __restrict__ in, const T* __restrict__ wt, const T* __restrict__ bias,
    const T* __restrict__ dy, T* __restrict__ out, void* __restrict__ out2, int flip) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = blockIdx.y * 64 + lane;
  const int runs = (a.W + kRun - 1) / kRun;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kRowWaves + wave;  // (b, t, h, run)
  const int64_t items = static_cast<int64_t>(a.B) * a.T * a.H * runs;
  if (item >= items || c >= a.C) return;
  const int run = static_cast<int>(item % runs);
  const int64_t bth = item / runs;
  const int h = static_cast<int>(bth % a.H);
  const int t = static_cast<int>((bth / a.H) % a.T);
  const int b = static_cast<int>(bth / (static_cast<int64_t>(a.H) * a.T));
  const int w0 = run * kRun;
  const int K = a.kt * a.kh * KW;
  const int pt = a.kt / 2, ph = a.kh / 2, pw = KW / 2;
  const T* __restrict__ wc = wt + static_cast<int64_t>(c) * K;

  float acc[kRun];
  const float b0 = bias != nullptr ? ld(bias, c) : 0.0f;
#pragma unroll
  for (int r = 0; r < kRun; ++r) acc[r] = b0;

  for (int dt = 0; dt < a.kt; ++dt) {
    const int tt = t + dt - pt;
    if (tt < 0 || tt >= a.T) continue;
    for (int dh = 0; dh < a.kh; ++dh) {
      const int hh = h + dh - ph;
      if (hh < 0 || hh >= a.H) continue;
      float wk[KW];
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        const int tap = (dt * a.kh + dh) * KW + k;
        wk[k] = ld(wc, flip ? K - 1 - tap : tap);
      }
      const int64_t row = (static_cast<int64_t>(b) * a.T + tt) * a.H + hh;
      const G* __restrict__ ir = in + row * a.W * static_cast<int64_t>(a.C) + c;
      float xr[kRun + KW - 1];
#pragma unroll
      for (int j = 0; j < kRun + KW - 1; ++j) {
        const int ww = w0 + j - pw;
        xr[j] = (ww >= 0 && ww < a.W) ? ld(ir, static_cast<int64_t>(ww) * a.C) : 0.0f;
      }
#pragma unroll
      for (int r = 0; r < kRun; ++r) {
#pragma unroll
        for (int k = 0; k < KW; ++k) acc[r] += wk[k] * xr[r + k];
      }
    }
  }
  const int64_t orow = ((static_cast<int64_t>(b) * a.T + t) * a.H + h) * a.W;
#pragma unroll
  for (int r = 0; r < kRun; ++r) {
    const int w = w0 + r;
    if (w >= a.W) continue;
    const int64_t i = (orow + w) * a.C + c;
    if (MODE == kPlain) st(out, i, acc[r]);
    if (MODE == kGelu) st(out, i, gelu_erf(acc[r]));
    if (MODE == kGeluSave) {
      st(out, i, gelu_erf(acc[r]));
      st(static_cast<T*>(out2), i, acc[r]);
    }
    if (MODE == kGeluGrad) static_cast<float*>(out2)[i] = ld(dy, i) * gelu_erf_grad(acc[r]);
    if (MODE == kGeluGradT) st(out, i, ld(dy, i) * gelu_erf_grad(acc[r]));
  }
}

// ---------------------------------------------------------------------------
// block kernels for square (kh, kw) in {3, 5, 7}: a thread owns one channel and
// an R x kRun block of outputs (R rows along H, kRun along W) of one frame.  Per
// input row it loads kRun + KW - 1 values once and applies them to every output
// row the row reaches (up to min(R, KH) of them); the KH x KW weights of the
// current dt stay in registers.
// ---------------------------------------------------------------------------

constexpr int kBlockRows = 4;  // R: output rows per thread

// Element `lane_off` (a 32-bit per-lane offset) past the wave-uniform pointer
// `base`: written so the compiler addresses it as scalar base + vector offset
// instead of building (and hoisting) a 64-bit vector address per load.
template <typename T>
__device__ __forceinline__ float ldu(const T* base, uint32_t lane_off) {
  const uint32_t bytes = lane_off * static_cast<uint32_t>(sizeof(T));  // 32-bit: zero-extended offset
  return to_f32(*reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + bytes));
}

template <typename T>
__device__ __forceinline__ void stu(T* base, uint32_t lane_off, float v) {
  const uint32_t bytes = lane_off * static_cast<uint32_t>(sizeof(T));
  *reinterpret_cast<T*>(reinterpret_cast<char*>(base) + bytes) = from_f32<T>(v);
}

// Input value at column ww of a row, 0 outside [0, W): the column is clamped and
// the value selected, so the loads of a row form one branch-free block.
template <typename G>
__device__ __forceinline__ float ld_col(const G* row, int ww, int W, int C, uint32_t lc) {
  const int wc = min(max(ww, 0), W - 1);
  const float v = ldu(row + static_cast<int64_t>(wc) * C, lc);
  return ww == wc ? v : 0.0f;
}

template <typename T, typename G, int KH, int KW, int MODE>
__global__ __launch_bounds__(64 * kRowWaves) void dwconv_block_kernel(
    ConvArgs a, const G* __restrict__ in, const T* __restrict__ wt, const T* __restrict__ bias,
    const T* __restrict__ dy, T* __restrict__ out, void* __restrict__ out2, int flip) {
  constexpr int R = kBlockRows, PH = KH / 2, PW = KW / 2, NX = kRun + KW - 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = blockIdx.y * 64 + lane;
  const int runs = (a.W + kRun - 1) / kRun;
  const int hblocks = (a.H + R - 1) / R;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kRowWaves + wave;  // (b, t, hblock, run)
  const int64_t items = static_cast<int64_t>(a.B) * a.T * hblocks * runs;
  if (item >= items) return;
  const bool c_ok = c < a.C;
  const uint32_t lc = c_ok ? c : a.C - 1;  // lanes past C read a valid channel and store nothing
  const int run = static_cast<int>(item % runs);
  const int64_t rest = item / runs;
  const int hb = static_cast<int>(rest % hblocks);
  const int64_t bt = rest / hblocks;
  const int t = static_cast<int>(bt % a.T);
  const int b = static_cast<int>(bt / a.T);
  const int h0 = hb * R, w0 = run * kRun;
  const int K = a.kt * KH * KW;
  const int64_t rowstride = static_cast<int64_t>(a.W) * a.C;

  float acc[R][kRun];
  const float b0 = bias != nullptr ? ldu(bias, lc) : 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < kRun; ++j) acc[r][j] = b0;

  for (int dt = 0; dt < a.kt; ++dt) {
    const int tt = t + dt - a.kt / 2;
    if (tt < 0 || tt >= a.T) continue;
    float wk[KH][KW];
#pragma unroll
    for (int dh = 0; dh < KH; ++dh)
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        const int tap = (dt * KH + dh) * KW + k;
        wk[dh][k] = ldu(wt + (flip ? K - 1 - tap : tap), lc * K);
      }
    const G* plane = in + (static_cast<int64_t>(b) * a.T + tt) * a.H * rowstride;
#pragma unroll
    for (int ii = 0; ii < R + KH - 1; ++ii) {
      const int hh = h0 + ii - PH;
      if (hh < 0 || hh >= a.H) continue;
      const G* row = plane + hh * rowstride;
      float x[NX];
#pragma unroll
      for (int j = 0; j < NX; ++j) {
        const int ww = w0 + j - PW;
        x[j] = ld_col(row, ww, a.W, a.C, lc);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int dh = ii - r;
        if (dh < 0 || dh >= KH) continue;
#pragma unroll
        for (int j = 0; j < kRun; ++j)
#pragma unroll
          for (int k = 0; k < KW; ++k) acc[r][j] = __builtin_fmaf(wk[dh][k], x[j + k], acc[r][j]);
      }
    }
  }
  if (!c_ok) return;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int h = h0 + r;
    if (h >= a.H) continue;
    const int64_t orow = ((static_cast<int64_t>(b) * a.T + t) * a.H + h) * a.W;
#pragma unroll
    for (int j = 0; j < kRun; ++j) {
      const int w = w0 + j;
      if (w >= a.W) continue;
      const int64_t i0 = (orow + w) * a.C;  // uniform; + lc per lane
      if (MODE == kPlain) stu(out + i0, lc, acc[r][j]);
      if (MODE == kGelu) stu(out + i0, lc, gelu_erf(acc[r][j]));
      if (MODE == kGeluSave) {
        stu(out + i0, lc, gelu_erf(acc[r][j]));
        stu(static_cast<decltype(out)>(out2) + i0, lc, acc[r][j]);
      }
      if (MODE == kGeluGrad) static_cast<float*>(out2)[i0 + lc] = ldu(dy + i0, lc) * gelu_erf_grad(acc[r][j]);
      if (MODE == kGeluGradT) stu(out + i0, lc, ldu(dy + i0, lc) * gelu_erf_grad(acc[r][j]));
    }
  }
}

// bf16 input and weights: the same blocking, with each pair of taps along W
// as one v_dot2 (two exact bf16 products added into the fp32 accumulator); the
// odd last tap stays an fp32 FMA.  Pairs (x[m], x[m+1]) of the loaded row
// segment are packed once and shared by every output of the run.
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_dot_t;

__device__ __forceinline__ uint32_t ldu_bits(const bf16* base, uint32_t lane_off) {
  return reinterpret_cast<const bf16*>(reinterpret_cast<const char*>(base) + lane_off * 2u)->bits;
}

__device__ __forceinline__ float dot2_bf16(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_dot_t, w),
                                         __builtin_bit_cast(bf16x2_dot_t, x), acc, false);
}

// bf16 rows read through a buffer resource: the lane's channel is the vector
// offset (the same for every load of a thread) and the voxel a scalar byte
// offset, so a load costs no vector instruction (64-bit per-load vector
// addresses, and the scalar registers they were built from, had made a third
// of these kernels' instructions).  The host admits tensors below 2^31 bytes.
constexpr int64_t kBufMaxBytes = int64_t{1} << 31;
constexpr int kBufWord3 = 0x00020000;  // raw 32-bit dwords, no swizzle (gfx9)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bf16_rows(const bf16* p, int64_t elems) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(p), 0, static_cast<int>(elems * 2),
                                           kBufWord3);
}
__device__ __forceinline__ uint32_t buf_bits(__amdgpu_buffer_rsrc_t r, uint32_t lane_bytes,
                                             uint32_t voxel_bytes) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, lane_bytes, voxel_bytes, 0);
}

template <int KH, int KW, int MODE>
__global__ __launch_bounds__(64 * kRowWaves) void dwconv_block_dot2_kernel(
    ConvArgs a, const bf16* __restrict__ in, const bf16* __restrict__ wt,
    const bf16* __restrict__ bias, const bf16* __restrict__ dy, bf16* __restrict__ out,
    void* __restrict__ out2, int flip) {
  constexpr int R = kBlockRows, PH = KH / 2, PW = KW / 2, NX = kRun + KW - 1, KP = KW / 2;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = blockIdx.y * 64 + lane;
  const int runs = (a.W + kRun - 1) / kRun;
  const int hblocks = (a.H + R - 1) / R;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kRowWaves + wave;  // (b, t, hblock, run)
  const int64_t items = static_cast<int64_t>(a.B) * a.T * hblocks * runs;
  if (item >= items) return;
  const bool c_ok = c < a.C;
  const uint32_t lc = c_ok ? c : a.C - 1;  // lanes past C read a valid channel and store nothing
  const int run = static_cast<int>(item % runs);
  const int64_t rest = item / runs;
  const int hb = static_cast<int>(rest % hblocks);
  const int64_t bt = rest / hblocks;
  const int t = static_cast<int>(bt % a.T);
  const int b = static_cast<int>(bt / a.T);
  const int h0 = hb * R, w0 = run * kRun;
  const int K = a.kt * KH * KW;
  // wide rows (kw >= 5) through a buffer resource; three-tap rows, whose
  // loads outnumber their products, measured faster with plain loads
  constexpr bool kBuf = KW >= 5;
  const __amdgpu_buffer_rsrc_t xr = bf16_rows(in, kBuf ? a.B * a.N * a.C : 0);
  const uint32_t lb = lc * 2u, cb = static_cast<uint32_t>(a.C) * 2u;  // lane, voxel bytes
  const int64_t rowstride = static_cast<int64_t>(a.W) * a.C;

  float acc[R][kRun];
  const float b0 = bias != nullptr ? ldu(bias, lc) : 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < kRun; ++j) acc[r][j] = b0;

  for (int dt = 0; dt < a.kt; ++dt) {
    const int tt = t + dt - a.kt / 2;
    if (tt < 0 || tt >= a.T) continue;
    uint32_t wp[KH][KP];  // taps (2kp, 2kp+1) of row dh, packed bf16
    uint32_t wl[KH];      // tap KW-1 as the pair (w, 0): one dot2 with (x, 0)
#pragma unroll
    for (int dh = 0; dh < KH; ++dh) {
      const int tap0 = (dt * KH + dh) * KW;
#pragma unroll
      for (int kp = 0; kp < KP; ++kp) {
        const int ta = tap0 + 2 * kp, tb = ta + 1;
        const uint32_t lo = ldu_bits(wt + (flip ? K - 1 - ta : ta), lc * K);
        const uint32_t hi = ldu_bits(wt + (flip ? K - 1 - tb : tb), lc * K);
        wp[dh][kp] = lo | (hi << 16);
      }
      const int tl = tap0 + KW - 1;
      wl[dh] = ldu_bits(wt + (flip ? K - 1 - tl : tl), lc * K);
    }
    const bf16* plane = in + (static_cast<int64_t>(b) * a.T + tt) * a.H * rowstride;
    const uint32_t plane_v = static_cast<uint32_t>((b * a.T + tt) * a.H);  // row index of hh = 0
#pragma unroll
    for (int ii = 0; ii < R + KH - 1; ++ii) {
      const int hh = h0 + ii - PH;
      if (hh < 0 || hh >= a.H) continue;
      const bf16* row = plane + hh * rowstride;
      const uint32_t row_v = (plane_v + hh) * static_cast<uint32_t>(a.W);  // voxel of ww = 0
      uint32_t xb[NX];
#pragma unroll
      for (int j = 0; j < NX; ++j) {
        const int ww = w0 + j - PW;
        const int wc = min(max(ww, 0), a.W - 1);
        const uint32_t v = kBuf ? buf_bits(xr, lb, (row_v + wc) * cb)
                                : ldu_bits(row + static_cast<int64_t>(wc) * a.C, lc);
        xb[j] = ww == wc ? v : 0u;
      }
      uint32_t xp[NX - 1];
#pragma unroll
      for (int m = 0; m < NX - 1; ++m) xp[m] = xb[m] | (xb[m + 1] << 16);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int dh = ii - r;
        if (dh < 0 || dh >= KH) continue;
#pragma unroll
        for (int j = 0; j < kRun; ++j) {
          float v = acc[r][j];
#pragma unroll
          for (int kp = 0; kp < KP; ++kp) v = dot2_bf16(wp[dh][kp], xp[j + 2 * kp], v);
          // xb holds the bf16 bits zero-extended: the pair (x, 0)
          acc[r][j] = dot2_bf16(wl[dh], xb[j + KW - 1], v);
        }
      }
    }
  }
  if (!c_ok) return;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int h = h0 + r;
    if (h >= a.H) continue;
    const int64_t orow = ((static_cast<int64_t>(b) * a.T + t) * a.H + h) * a.W;
#pragma unroll
    for (int j = 0; j < kRun; ++j) {
      const int w = w0 + j;
      if (w >= a.W) continue;
      const int64_t i0 = (orow + w) * a.C;  // uniform; + lc per lane
      if (MODE == kPlain) stu(out + i0, lc, acc[r][j]);
      if (MODE == kGelu) stu(out + i0, lc, gelu_erf(acc[r][j]));
      if (MODE == kGeluSave) {
        stu(out + i0, lc, gelu_erf(acc[r][j]));
        stu(static_cast<decltype(out)>(out2) + i0, lc, acc[r][j]);
      }
      if (MODE == kGeluGrad) static_cast<float*>(out2)[i0 + lc] = ldu(dy + i0, lc) * gelu_erf_grad(acc[r][j]);
      if (MODE == kGeluGradT) stu(out + i0, lc, ldu(dy + i0, lc) * gelu_erf_grad(acc[r][j]));
    }
  }
}

// Weight / bias gradient for square (kh, kw) in {3, 5, 7}: a thread owns one
// channel and one dt (KH x KW tap sums in registers) and walks a strip of
// kDwStripBlocks blocks of R = kDwRows output rows of one frame.  For every R-row block and
// run it keeps the R x kRun dz values in registers and loads each input row once.
// acc[tap*C + c] += partial sums; acc[K*C + c] += sum dz (dt == 0 threads).  The
// tap-major layout puts a wave's 64 channels of one tap on two cache lines.
constexpr int kDwRows = 4;         // output rows per weight-gradient step
constexpr int kDwStripBlocks = 2;  // steps per work item

template <typename T, typename G, int KH, int KW>
__global__ __launch_bounds__(64 * kRowWaves) void dwconv_dw_block_kernel(ConvArgs a,
                                                                         const T* __restrict__ x,
                                                                         const G* __restrict__ dz,
                                                                         float* __restrict__ acc) {
  constexpr int R = kDwRows, PH = KH / 2, PW = KW / 2, NX = kRun + KW - 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = blockIdx.y * 64 + lane;
  const int dt = blockIdx.z;
  const int hblocks = (a.H + R - 1) / R;
  const int strips_per_frame = (hblocks + kDwStripBlocks - 1) / kDwStripBlocks;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kRowWaves + wave;  // (b, t, strip)
  const int64_t items = static_cast<int64_t>(a.B) * a.T * strips_per_frame;
  if (item >= items) return;
  const int strip = static_cast<int>(item % strips_per_frame);
  const int64_t bt = item / strips_per_frame;
  const int t = static_cast<int>(bt % a.T);
  const int b = static_cast<int>(bt / a.T);
  const int tt = t + dt - a.kt / 2;
  const bool plane_ok = tt >= 0 && tt < a.T;
  if (!plane_ok && dt != 0) return;  // no taps; the dt == 0 threads still sum dz for the bias
  const bool c_ok = c < a.C;
  const uint32_t lc = c_ok ? c : a.C - 1;
  const int K = a.kt * KH * KW;
  const int64_t rowstride = static_cast<int64_t>(a.W) * a.C;
  float s[KH][KW];
#pragma unroll
  for (int dh = 0; dh < KH; ++dh)
#pragma unroll
    for (int k = 0; k < KW; ++k) s[dh][k] = 0.0f;
  float sb = 0.0f;
  const T* plane = x + (static_cast<int64_t>(b) * a.T + (plane_ok ? tt : 0)) * a.H * rowstride;
  const G* gplane = dz + (static_cast<int64_t>(b) * a.T + t) * a.H * rowstride;
  const int hb_end = min(hblocks, (strip + 1) * kDwStripBlocks);
  for (int hb = strip * kDwStripBlocks; hb < hb_end; ++hb) {
    const int h0 = hb * R;
    for (int w0 = 0; w0 < a.W; w0 += kRun) {
      float g[R][kRun];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < kRun; ++j) {
          const int h = h0 + r, w = w0 + j;
          g[r][j] = h < a.H ? ld_col(gplane + h * rowstride, w, a.W, a.C, lc) : 0.0f;
          if (dt == 0) sb += g[r][j];
        }
      if (!plane_ok) continue;
#pragma unroll
      for (int ii = 0; ii < R + KH - 1; ++ii) {
        const int hh = h0 + ii - PH;
        if (hh < 0 || hh >= a.H) continue;
        const T* row = plane + hh * rowstride;
        float xv[NX];
#pragma unroll
        for (int j = 0; j < NX; ++j) {
          const int ww = w0 + j - PW;
          xv[j] = ld_col(row, ww, a.W, a.C, lc);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int dh = ii - r;
          if (dh < 0 || dh >= KH) continue;
#pragma unroll
          for (int k = 0; k < KW; ++k) {
            float part = 0.0f;
#pragma unroll
            for (int j = 0; j < kRun; ++j) part = __builtin_fmaf(g[r][j], xv[j + k], part);
            s[dh][k] += part;
          }
        }
      }
    }
  }
  if (!c_ok) return;
  float* __restrict__ ac = acc + static_cast<int64_t>(dt * KH * KW) * a.C + c;
#pragma unroll
  for (int dh = 0; dh < KH; ++dh)
#pragma unroll
    for (int k = 0; k < KW; ++k)
      if (s[dh][k] != 0.0f) atomicAdd(ac + static_cast<int64_t>(dh * KW + k) * a.C, s[dh][k]);
  if (dt == 0 && sb != 0.0f) atomicAdd(acc + static_cast<int64_t>(K) * a.C + c, sb);
}

// bf16 x and dz: the same walk with the sums over W taken two outputs at a
// time, sum_j dz[j] x[j+k] as v_dot2 of the packed pairs (dz[j], dz[j+1]) and
// (x[j+k], x[j+k+1]) (exact bf16 products into fp32); the packed dz block also
// takes half the registers.
// dz rows and columns per block of the dot2 weight gradient, per kernel size:
// 2-row blocks for kw >= 5, where 4 rows of dz pairs beside the kh x kw sums
// took 172 registers at 7x7 (2 waves per SIMD); at 124 (4 waves) the 3x7x7
// backward went 6.13 -> 4.85 ms at 131,072 tokens for 60% more x-row loads
// (8-column runs instead: 4.89 ms)
template <int KS>
constexpr int kDw2Rows = KS >= 5 ? 2 : kDwRows;
template <int KS>
constexpr int kDw2Run = kRun;

template <int KH, int KW, int R = kDwRows, int RUN = kRun>
__global__ __launch_bounds__(64 * kRowWaves) void dwconv_dw_block_dot2_kernel(
    ConvArgs a, const bf16* __restrict__ x, const bf16* __restrict__ dz, float* __restrict__ acc) {
  constexpr int PH = KH / 2, PW = KW / 2, NX = RUN + KW - 1, JP = RUN / 2;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = blockIdx.y * 64 + lane;
  const int dt = blockIdx.z;
  const int hblocks = (a.H + R - 1) / R;
  const int strips_per_frame = (hblocks + kDwStripBlocks - 1) / kDwStripBlocks;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kRowWaves + wave;  // (b, t, strip)
  const int64_t items = static_cast<int64_t>(a.B) * a.T * strips_per_frame;
  if (item >= items) return;
  const int strip = static_cast<int>(item % strips_per_frame);
  const int64_t bt = item / strips_per_frame;
  const int t = static_cast<int>(bt % a.T);
  const int b = static_cast<int>(bt / a.T);
  const int tt = t + dt - a.kt / 2;
  const bool plane_ok = tt >= 0 && tt < a.T;
  if (!plane_ok && dt != 0) return;  // no taps; the dt == 0 threads still sum dz for the bias
  const bool c_ok = c < a.C;
  const uint32_t lc = c_ok ? c : a.C - 1;
  const int K = a.kt * KH * KW;
  // x and dz rows through buffer resources (lane channel as vector offset,
  // voxel as scalar offset); the host admits tensors below 2^31 bytes
  const __amdgpu_buffer_rsrc_t xr = bf16_rows(x, a.B * a.N * a.C);
  const __amdgpu_buffer_rsrc_t gr = bf16_rows(dz, a.B * a.N * a.C);
  const uint32_t lb = lc * 2u, cb = static_cast<uint32_t>(a.C) * 2u;
  float s[KH][KW];
#pragma unroll
  for (int dh = 0; dh < KH; ++dh)
#pragma unroll
    for (int k = 0; k < KW; ++k) s[dh][k] = 0.0f;
  float sb = 0.0f;
  // row indices of h = 0 in the x plane tt and the dz plane t
  const uint32_t plane = static_cast<uint32_t>((b * a.T + (plane_ok ? tt : 0)) * a.H);
  const uint32_t gplane = static_cast<uint32_t>((b * a.T + t) * a.H);
  const int hb_end = min(hblocks, (strip + 1) * kDwStripBlocks);
  for (int hb = strip * kDwStripBlocks; hb < hb_end; ++hb) {
    const int h0 = hb * R;
    for (int w0 = 0; w0 < a.W; w0 += RUN) {
      uint32_t gp[R][JP];  // (dz[2jp], dz[2jp+1]) of row r, packed bf16
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int h = h0 + r;
#pragma unroll
        for (int jp = 0; jp < JP; ++jp) {
          uint32_t lo = 0u, hi = 0u;
          if (h < a.H) {
            const uint32_t grow = (gplane + h) * static_cast<uint32_t>(a.W);
            const int w = w0 + 2 * jp;
            const int wl = min(w, a.W - 1), wh = min(w + 1, a.W - 1);
            lo = w < a.W ? buf_bits(gr, lb, (grow + wl) * cb) : 0u;
            hi = w + 1 < a.W ? buf_bits(gr, lb, (grow + wh) * cb) : 0u;
          }
          gp[r][jp] = lo | (hi << 16);
          if (dt == 0) sb += __uint_as_float(lo << 16) + __uint_as_float(hi << 16);
        }
      }
      if (!plane_ok) continue;
#pragma unroll
      for (int ii = 0; ii < R + KH - 1; ++ii) {
        const int hh = h0 + ii - PH;
        if (hh < 0 || hh >= a.H) continue;
        const uint32_t row = (plane + hh) * static_cast<uint32_t>(a.W);
        uint32_t xb[NX];
#pragma unroll
        for (int j = 0; j < NX; ++j) {
          const int ww = w0 + j - PW;
          const int wc = min(max(ww, 0), a.W - 1);
          const uint32_t v = buf_bits(xr, lb, (row + wc) * cb);
          xb[j] = ww == wc ? v : 0u;
        }
        uint32_t xp[NX - 1];
#pragma unroll
        for (int m = 0; m < NX - 1; ++m) xp[m] = xb[m] | (xb[m + 1] << 16);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int dh = ii - r;
          if (dh < 0 || dh >= KH) continue;
#pragma unroll
          for (int k = 0; k < KW; ++k) {
            float part = 0.0f;
#pragma unroll
            for (int jp = 0; jp < JP; ++jp) part = dot2_bf16(gp[r][jp], xp[2 * jp + k], part);
            s[dh][k] += part;
          }
        }
      }
    }
  }
  if (!c_ok) return;
  float* __restrict__ ac = acc + static_cast<int64_t>(dt * KH * KW) * a.C + c;
#pragma unroll
  for (int dh = 0; dh < KH; ++dh)
#pragma unroll
    for (int k = 0; k < KW; ++k)
      if (s[dh][k] != 0.0f) atomicAdd(ac + static_cast<int64_t>(dh * KW + k) * a.C, s[dh][k]);
  if (dt == 0 && sb != 0.0f) atomicAdd(acc + static_cast<int64_t>(K) * a.C + c, sb);
}

// ---------------------------------------------------------------------------
// Weight / bias gradient on the matrix cores (bf16 x and dz, kw <= 16,
// kt * kh <= 32).  One dz row (b, t, h) of one channel contributes
//   G[dw][n] = sum_w dz[w] x[t + dt - pt][h + dh - ph][w + dw - pw],  n = dt kh + dh,
// which is a product over the row's x positions w' = w + dw - pw (k = w' + pw):
//   G = A B,  A[m][k] = dz[k - m] (0 outside the row: the Toeplitz matrix of
//   the dz row),  B[k][n] = x_n[k - pw] (x row n of the tap's (dt, dh), zero
//   padded).
// The row is taken in segments of 32 dz positions (k < 64: two 16x16x32 MFMAs
// per tile of 16 n).  A workgroup owns kDwmCh channels, one per wave, and
// walks bands of R dz rows of consecutive (b, t) items.  Per band it stages
// into LDS, channel-major, the dz rows (each 32-position segment as [16 zeros
// | 32 values | 40 zeros], so A's reads outside the segment fall on zeros, in
// two copies, the second shifted by one element: lane m's 8-element window of
// A starts 4-byte aligned in copy m & 1) and the kt (R + kh - 1) x rows they
// reach (x_n[w] at element w + pw of a zero-padded row).  G stays in the MFMA
// accumulators across the workgroup's bands and is flushed with one fp32
// atomic per (channel, tap).
// ---------------------------------------------------------------------------
constexpr int kDwmCh = 8;    // channels (one per wave) per workgroup
typedef __attribute__((ext_vector_type(8))) __bf16 dwm_bf16x8_t;
typedef __attribute__((ext_vector_type(8))) uint16_t dwm_u16x8_t;
typedef __attribute__((ext_vector_type(4))) float dwm_f32x4_t;
constexpr int kDwmSeg = 88;  // LDS elements per staged dz row segment (one copy)

struct DwmGeom {
  int R;        // dz rows per band
  int nseg;     // 32-position segments per row
  int xps;      // LDS stride of a staged x row (elements)
  int xr;       // staged x rows per plane: R + kh - 1
  int bands;    // bands per (b, t)
  int ipw;      // (b, t, band) items per workgroup
  int x_elems;  // staged x elements per channel: kt * xr * xps
  int dz_elems; // staged dz elements per channel: 2 copies * R * nseg * kDwmSeg
  float rW;     // 1 / W and 1 / xr: exact quotients of the small staging
  float rxr;    // indices (below 2^20) by float multiply and truncation
};

template <int KH, int KW>
__global__ __launch_bounds__(64 * kDwmCh) void dwconv_dw_mfma_kernel(ConvArgs a, DwmGeom g,
                                                                     const bf16* __restrict__ x,
                                                                     const bf16* __restrict__ dz,
                                                                     float* __restrict__ acc) {
  static_assert(KW <= 16, "the 16 MFMA rows hold the kw taps");
  constexpr int PH = KH / 2, PW = KW / 2;
  extern __shared__ __attribute__((aligned(16))) uint16_t s_dwm[];
  uint16_t* const s_x = s_dwm;                       // [ch][dt][xr][xps]
  uint16_t* const s_dz = s_dwm + kDwmCh * g.x_elems;  // [ch][copy][R][nseg][kDwmSeg]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c0 = blockIdx.y * kDwmCh;
  const int nk = a.kt * KH;  // used MFMA columns
  const int nnt = (nk + 15) / 16;
  const int64_t rowstride = static_cast<int64_t>(a.W) * a.C;

  // the pads must read as zeros; value positions are rewritten every band
  {
    const int n32 = kDwmCh * (g.x_elems + g.dz_elems) / 2;
    uint32_t* const z = reinterpret_cast<uint32_t*>(s_dwm);
    for (int i = threadIdx.x; i < n32; i += blockDim.x) z[i] = 0u;
  }
  __syncthreads();

  // B operand rows of this lane's column n = 16 nt + lane % 16 (clamped: unused
  // columns read a valid row and are discarded)
  const int m = lane & 15, kg = lane >> 4;
  int brow[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = min(16 * nt + m, nk - 1);
    const int dt = n / KH, dh = n - dt * KH;
    brow[nt] = (dt * g.xr + dh) * g.xps + 8 * kg;
  }
  const uint16_t* const xw = s_x + wave * g.x_elems;
  const uint16_t* const dzw = s_dz + wave * g.dz_elems;
  dwm_f32x4_t gacc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  float sb = 0.0f;

  const int64_t items = static_cast<int64_t>(a.B) * a.T * g.bands;
  const int64_t it0 = static_cast<int64_t>(blockIdx.x) * g.ipw;
  const int64_t it1 = min(items, it0 + g.ipw);
  for (int64_t it = it0; it < it1; ++it) {
    const int band = static_cast<int>(it % g.bands);
    const int64_t bt = it / g.bands;
    const int t = static_cast<int>(bt % a.T);
    const int b = static_cast<int>(bt / a.T);
    const int h0 = band * g.R;
    __syncthreads();  // the previous band's reads are done
    // Stage the band: voxel e < nx is x voxel (row q = e / W, column e % W) of
    // the kt x xr halo rows, the rest are the R dz rows; 16 bytes (8
    // channels) per voxel, four voxels per thread with their loads issued
    // before any LDS write.  Rows outside the volume stage zeros.
    const int nx = a.kt * g.xr * a.W, ntot = nx + g.R * a.W;
    for (int e0 = threadIdx.x; e0 < ntot; e0 += 4 * 64 * kDwmCh) {
      // LDS destinations as element offsets (-1: none), so the stores stay DS stores
      uint4 v[4];
      int dst[4], stride[4];
      bool dup[4];  // dz voxel: also into the shifted copy
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = e0 + u * 64 * kDwmCh;
        v[u] = uint4{0u, 0u, 0u, 0u};
        dst[u] = -1;
        stride[u] = 0;
        dup[u] = false;
        if (e >= ntot) continue;
        const bool is_x = e < nx;
        const int ee = is_x ? e : e - nx;
        const int q = static_cast<int>((static_cast<float>(ee) + 0.5f) * g.rW);
        const int w = ee - q * a.W;
        const bf16* src = nullptr;
        if (is_x) {
          const int dt = static_cast<int>((static_cast<float>(q) + 0.5f) * g.rxr);
          const int rr = q - dt * g.xr;
          const int tt = t + dt - a.kt / 2, hh = h0 + rr - PH;
          if (tt >= 0 && tt < a.T && hh >= 0 && hh < a.H)
            src = x + ((static_cast<int64_t>(b) * a.T + tt) * a.H + hh) * rowstride;
          dst[u] = q * g.xps + w + PW;
          stride[u] = g.x_elems;
        } else {
          const int h = h0 + q;
          if (h < a.H) src = dz + ((static_cast<int64_t>(b) * a.T + t) * a.H + h) * rowstride;
          dst[u] = kDwmCh * g.x_elems + (q * g.nseg + (w >> 5)) * kDwmSeg + 16 + (w & 31);
          stride[u] = g.dz_elems;
          dup[u] = true;
        }
        if (src != nullptr)
          v[u] = *reinterpret_cast<const uint4*>(src + static_cast<int64_t>(w) * a.C + c0);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (dst[u] < 0) continue;
        const uint32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int ch = 0; ch < kDwmCh; ++ch) {
          const uint16_t h = static_cast<uint16_t>(vv[ch >> 1] >> (16 * (ch & 1)));
          s_dwm[dst[u] + ch * stride[u]] = h;
          if (dup[u]) s_dwm[dst[u] + ch * stride[u] + g.dz_elems / 2 + 1] = h;
        }
      }
    }
    __syncthreads();
    // this wave's channel: every valid row of the band, every segment
    const int rows = min(g.R, a.H - h0);
    for (int r = 0; r < rows; ++r) {
      for (int s = 0; s < g.nseg; ++s) {
        // window start 16 + 8 kg + 32 kb - m, made even in copy m & 1
        const uint16_t* const da =
            dzw + (m & 1) * (g.dz_elems / 2) + (r * g.nseg + s) * kDwmSeg + 16 + 8 * kg - m + (m & 1);
        const uint16_t* const xb = xw + r * g.xps + 32 * s;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          // four aligned dword reads (volatile: not merged into one misaligned
          // 16-byte read, which stalls)
          typedef const volatile __attribute__((address_space(3))) uint32_t lds_u32;
          lds_u32* const pa = (lds_u32*)(da + 32 * kb);
          uint32_t aw[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) aw[j] = pa[j];
          const dwm_u16x8_t av = __builtin_bit_cast(dwm_u16x8_t, aw);
          const dwm_bf16x8_t A = __builtin_bit_cast(dwm_bf16x8_t, av);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            if (nt >= nnt) break;
            dwm_u16x8_t bv;
            __builtin_memcpy(&bv, xb + brow[nt] + 32 * kb, sizeof(bv));
            gacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                A, __builtin_bit_cast(dwm_bf16x8_t, bv), gacc[nt], 0, 0, 0);
          }
        }
      }
      // bias: the row's dz values of this channel
      for (int w = lane; w < a.W; w += 64)
        sb += __uint_as_float(static_cast<uint32_t>(dzw[(r * g.nseg + (w >> 5)) * kDwmSeg + 16 +
                                                        (w & 31)])
                              << 16);
    }
  }
  // flush: gacc[nt][i] = G[dw = 4 (lane / 16) + i][n = 16 nt + lane % 16]
  const int c = c0 + wave;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = 16 * nt + m;
    if (n >= nk) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int dw = 4 * kg + i;
      if (dw < KW && gacc[nt][i] != 0.0f)
        atomicAdd(acc + static_cast<int64_t>(n * KW + dw) * a.C + c, gacc[nt][i]);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) sb += __shfl_xor(sb, o);
  if (lane == 0 && sb != 0.0f) atomicAdd(acc + static_cast<int64_t>(nk * KW) * a.C + c, sb);
}

// LDS geometry of the matrix-core weight gradient (at most 64 KB of dynamic
// LDS: two workgroups per CU), or R = 0 where it does not apply (then the VALU
// kernels run).  Bands of fewer than 4 rows stage too many halo rows per dz
// row (kt (R + kh - 1) / R): at W = 80 (1-row bands) it took 2.95 ms against
// 0.82 for the dot2 kernel.
constexpr int64_t kDwmLdsMax = 64 * 1024;

inline int64_t dwm_lds_bytes(const DwmGeom& g) {
  return 2LL * kDwmCh * (static_cast<int64_t>(g.x_elems) + g.dz_elems);
}

inline DwmGeom dwm_geometry(const ConvArgs& a) {
  DwmGeom g{};
  if (a.kw > 16 || a.kt * a.kh > 32 || a.C % kDwmCh != 0 || a.W < 1 || a.W > 4096) return g;
  g.nseg = (a.W + 31) / 32;
  g.xps = 32 * g.nseg + 40;
  for (int R = 8; R >= 4; R >>= 1) {
    const int xr = R + a.kh - 1;
    const int64_t bytes = 2LL * kDwmCh * (static_cast<int64_t>(a.kt) * xr * g.xps +
                                          2LL * R * g.nseg * kDwmSeg);
    if (bytes <= kDwmLdsMax) {
      g.R = R;
      g.xr = xr;
      g.x_elems = a.kt * xr * g.xps;
      g.dz_elems = 2 * R * g.nseg * kDwmSeg;
      break;
    }
  }
  if (g.R == 0) return g;
  g.bands = (a.H + g.R - 1) / g.R;
  g.rW = 1.0f / static_cast<float>(a.W);
  g.rxr = 1.0f / static_cast<float>(g.xr);
  // enough workgroups for two per CU several times over, few atomics each
  const int64_t items = static_cast<int64_t>(a.B) * a.T * g.bands;
  const int64_t cblocks = a.C / kDwmCh;
  const int64_t ipw = (items * cblocks + 2047) / 2048;
  g.ipw = static_cast<int>(ipw > 0 ? ipw : 1);
  return g;
}

// ---------------------------------------------------------------------------
// Convolution (forward, and the input gradient with mirrored taps) on the
// matrix cores: bf16, kh = kw in {5, 7}, kt in {1, 3}, W a multiple of 4, no
// activation.  (3x3 rows stay on the dot2 kernels: with 9 tap rows per frame
// the staging outweighs the products, and the matrix-core version of the
// offset net's 3x3x3 + GELU measured 0.187 ms against 0.176 at 65,536 tokens.)
// For one channel, one tap row (dt, dh) and one segment of 16 outputs
// w0 .. w0 + 15 of an output row h, with the input row staged from w0 - 4:
//   out[w0 + m] += sum_k A[m][k] x[t + dt - pt][h + dh - ph][w0 - 4 + k],  k < 32,
//   A[m][k] = wt[dt][dh][k - m - (4 - pw)]  (0 outside [0, kw)),
// the banded Toeplitz matrix of the tap row: D = A B with B[k][n] the 32
// input values of segment n, so one 16x16x32 MFMA takes 16 segments (any rows
// and x tiles) for one tap row.  A workgroup owns kFwmCh channels, one per
// wave, a band of R output rows and a run of consecutive frames of one batch
// entry.  Each wave keeps its channel's kt kh A operands in registers for the
// run.  The staged input frames form a ring of kt slots in LDS (channel-major,
// x[w] at element w + kFwmPadL of a zero-padded row), so each input frame of
// the run is staged once; per output frame the kernel runs kt kh MFMAs per 16
// segments (segment s = (xt, r) = divmod(s, R), x tile major, with a row
// stride the host picks so that a wave's 16-byte B reads fall on distinct
// banks) and writes the band through LDS as 16-byte (8-channel) stores.
// Products are exact and summed in fp32, as in the dot2 kernels; only the
// order of the fp32 sums differs.
// Work order: workgroup L runs on XCD L % 8; within an XCD consecutive
// workgroups take consecutive channel blocks of the same work item, so the
// 128-byte lines of a voxel's channels are read and written through one L2.
// ---------------------------------------------------------------------------
constexpr int kFwmCh = 8;          // channels (one per wave) per workgroup
constexpr int kFwmMaxTiles = 4;    // MFMA tiles of 16 segments per band
constexpr int kFwmGrp = 2;         // staged 4-voxel groups per thread and frame (at most)
constexpr int kFwmPadL = 4;        // staged row: voxel w at element w + kFwmPadL
typedef __attribute__((ext_vector_type(4))) unsigned int fwm_u32x4_t;
constexpr int kFwmTopRow = 96;     // Toeplitz row in LDS: two 48-element copies
constexpr int64_t kFwmLdsMax = 80 * 1024;  // two workgroups per CU

struct FwmGeom {
  int R;        // output rows per band (0: the kernel does not apply)
  int nxt;      // 16-position x tiles per row
  int xps;      // LDS stride of a staged row (elements, a multiple of 8)
  int xr;       // staged rows per frame: R + kh - 1
  int tiles;    // ceil(R nxt / 16)
  int bands;    // bands per frame
  int tr;       // output frames per work item (a run along T)
  int nruns;    // runs per (b, band): ceil(T / tr)
  int nig;      // work items per channel block, rounded up to a multiple of 8
  int x_elems;  // staged elements per channel: kt xr xps
  int ng;       // 4-voxel staging groups per staged row: W / 4
  int lds;      // dynamic LDS bytes
  float rW;     // 1 / W and 1 / ng: exact quotients of the staging and output
  float rng;    // indices (below 2^20) by float multiply and truncation
};

template <int KT, int KS>
__global__ __launch_bounds__(64 * kFwmCh) void dwconv_fwd_mfma_kernel(
    ConvArgs a, FwmGeom g, const bf16* __restrict__ in, const bf16* __restrict__ wt,
    const bf16* __restrict__ bias, bf16* __restrict__ out, int flip) {
  constexpr int KH = KS, KW = KS, PT = KT / 2, PH = KH / 2, PW = KW / 2, K = KT * KH * KW;
  extern __shared__ __attribute__((aligned(16))) uint16_t s_fwm[];
  uint16_t* const s_x = s_fwm;                       // [ch][dt][xr][xps]
  uint16_t* const s_o = s_fwm + kFwmCh * g.x_elems;  // [R][W (+1)][ch] band outputs
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ncb = a.C / kFwmCh;
  const int j = static_cast<int>(blockIdx.x >> 3);
  const int cb = j % ncb, ig = (j / ncb) * 8 + static_cast<int>(blockIdx.x & 7);
  // work item ig: a run of g.tr output frames of band `band` of batch b
  if (ig >= a.B * g.bands * g.nruns) return;
  const int run = ig % g.nruns, bb = ig / g.nruns;
  const int band = bb % g.bands, b = bb / g.bands;
  const int t0 = run * g.tr, t1 = min(a.T, t0 + g.tr), h0 = band * g.R;
  const int c0 = cb * kFwmCh, c = c0 + wave;
  const int m = lane & 15, kg = lane >> 4;

  // A operands.  Row (dt, dh) of this wave's Toeplitz table: elements [0, 48)
  // hold P[e] = w[e - 16 - (kFwmPadL - pw)] (0 outside [0, kw)), [48, 96) the
  // copy shifted by one, P[e + 1].  Lane (m, kg) needs P[s .. s + 7],
  // s = 16 + 8 kg - m in [1, 40] (A[m][k] = P[16 + k - m]): from the first copy
  // when s is even, else from the second at s - 1, so its four dword reads are
  // aligned.
  {
    // the channel's K weights (mirrored for the input gradient) into LDS with
    // independent loads, then the table rows from them
    constexpr int KP = (K + 7) / 8 * 8;
    uint16_t* const tw = s_fwm + wave * (KT * KH * kFwmTopRow);
    uint16_t* const rw = s_fwm + kFwmCh * (KT * KH * kFwmTopRow) + wave * KP;
    const bf16* const wc = wt + static_cast<int64_t>(c) * K;
    uint16_t wv[(K + 63) / 64];
#pragma unroll
    for (int u = 0; u < (K + 63) / 64; ++u) {
      const int i = lane + 64 * u;
      wv[u] = i < K ? wc[flip ? K - 1 - i : i].bits : uint16_t{0};
    }
#pragma unroll
    for (int u = 0; u < (K + 63) / 64; ++u)
      if (lane + 64 * u < K) rw[lane + 64 * u] = wv[u];
    __syncthreads();
    for (int i = lane; i < KT * KH * kFwmTopRow; i += 64) {
      const int row = i / kFwmTopRow, e = i - row * kFwmTopRow;
      const int dw = (e < 48 ? e - 16 : e - 63) - (kFwmPadL - PW);
      tw[i] = (dw >= 0 && dw < KW) ? rw[row * KW + dw] : uint16_t{0};
    }
  }
  __syncthreads();
  dwm_bf16x8_t A[KT][KH];
  {
    const int s = 16 + 8 * kg - m;
    const int off = (m & 1) ? 48 + s - 1 : s;
    typedef const volatile __attribute__((address_space(3))) uint32_t lds_u32;
#pragma unroll
    for (int dt = 0; dt < KT; ++dt)
#pragma unroll
      for (int dh = 0; dh < KH; ++dh) {
        lds_u32* const p =
            (lds_u32*)(s_fwm + wave * (KT * KH * kFwmTopRow) + (dt * KH + dh) * kFwmTopRow + off);
        uint32_t w4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) w4[q] = p[q];
        A[dt][dh] = __builtin_bit_cast(dwm_bf16x8_t, w4);
      }
  }
  __syncthreads();  // every wave holds its A operands: the table space is reused
  {
    const int n32 = kFwmCh * g.x_elems / 2;  // the row pads must read as zeros
    uint32_t* const z = reinterpret_cast<uint32_t*>(s_fwm);
    for (int i = threadIdx.x; i < n32; i += blockDim.x) z[i] = 0u;
  }
  __syncthreads();

  const float bc = bias != nullptr ? to_f32(bias[c]) : 0.0f;
  const int S = g.R * g.nxt;
  const int orow = a.W * kFwmCh + 8;  // output staging row (elements): 16-byte pad
  const int64_t rowstride = static_cast<int64_t>(a.W) * a.C;
  // LDS byte address of this wave's staged rows
  const uint32_t xw = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_x + wave * g.x_elems));
  typedef const __attribute__((address_space(3))) dwm_u16x8_t lds_u16x8;

  // The staged frames form a ring of kt slots: input frame f sits in slot
  // (f + kt) mod kt, so output frame t reads frames t - pt .. t + pt and each
  // input frame of the run is staged once.  Staging in groups of four voxels
  // along W (W is a multiple of 4): group (q, j) of a frame's staged row q holds
  // voxels w = 4j .. 4j + 3 at elements 4j + kFwmPadL .. (8-byte aligned),
  // written per channel as one 8-byte LDS store.  The loads go through a
  // buffer resource: rows and frames outside the volume get an offset past the
  // buffer's end and read zeros, and the four voxels of a group differ only in
  // the scalar offset.  Group gi goes to thread gi mod 512; the next frame's
  // groups are loaded into registers while the current frame's MFMAs run.
  const int ng = g.ng, nfg = g.xr * ng;
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(in), 0,
                                        static_cast<int>(static_cast<int64_t>(a.B) * a.N * a.C * 2), kBufWord3);
  const int vb = a.C * 2;  // bytes per voxel
  fwm_u32x4_t pv[kFwmGrp][4];
  auto prefetch = [&](int tt) {
#pragma unroll
    for (int u = 0; u < kFwmGrp; ++u) {
      const int gi = threadIdx.x + u * 64 * kFwmCh;
      if (u > 0 && gi >= nfg) break;  // no group (u = 0 loads zeros from past the end instead)
      const int q = static_cast<int>((static_cast<float>(gi) + 0.5f) * g.rng);
      const int jg = gi - q * ng, hh = h0 + q - PH;
      const bool ok = gi < nfg && tt >= 0 && tt < a.T && hh >= 0 && hh < a.H;
      const uint32_t off = ok ? static_cast<uint32_t>((((b * a.T + tt) * a.H + hh) * a.W + 4 * jg) * vb + c0 * 2)
                              : 0x80000000u;
#pragma unroll
      for (int v = 0; v < 4; ++v) pv[u][v] = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, v * vb, 0);
    }
  };
  auto commit = [&](int tt) {
    const int slot = (tt + KT) % KT;
#pragma unroll
    for (int u = 0; u < kFwmGrp; ++u) {
      const int gi = threadIdx.x + u * 64 * kFwmCh;
      if (gi >= nfg) continue;
      const int q = static_cast<int>((static_cast<float>(gi) + 0.5f) * g.rng);
      uint16_t* const dst = s_x + (slot * g.xr + q) * g.xps + 4 * (gi - q * ng) + kFwmPadL;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // channels 2k (low halves) and 2k + 1 (high halves) of the four voxels
        const uint2 lo = {__builtin_amdgcn_perm(pv[u][1][k], pv[u][0][k], 0x05040100u),
                          __builtin_amdgcn_perm(pv[u][3][k], pv[u][2][k], 0x05040100u)};
        const uint2 hi = {__builtin_amdgcn_perm(pv[u][1][k], pv[u][0][k], 0x07060302u),
                          __builtin_amdgcn_perm(pv[u][3][k], pv[u][2][k], 0x07060302u)};
        *reinterpret_cast<uint2*>(dst + (2 * k) * g.x_elems) = lo;
        *reinterpret_cast<uint2*>(dst + (2 * k + 1) * g.x_elems) = hi;
      }
    }
  };
  // Per tile, this lane's B column n = m: segment s = (xt, r) = divmod(s, R),
  // clamped to the last segment where the tile is partial (its results are
  // not stored); its LDS address in a frame's rows and its output slot.
  uint32_t taddr[kFwmMaxTiles];
  int to[kFwmMaxTiles], tx[kFwmMaxTiles];
  bool tval[kFwmMaxTiles];
#pragma unroll
  for (int tile = 0; tile < kFwmMaxTiles; ++tile) {
    const int sr = 16 * tile + m;
    const int sg = min(sr, S - 1);
    const int xt = sg / g.R, r = sg - xt * g.R;
    taddr[tile] = xw + 2u * static_cast<uint32_t>(r * g.xps + 16 * xt + 8 * kg);
    tx[tile] = 16 * xt + 4 * kg;
    to[tile] = r * orow + tx[tile] * kFwmCh + wave;
    tval[tile] = sr < S;
  }
  // the ring's first kt - 1 frames, then the loads of the next one
  for (int f = t0 - PT; f < t0 + PT; ++f) {
    prefetch(f);
    commit(f);
  }
  prefetch(t0 + PT);
  commit(t0 + PT);

  for (int t = t0; t < t1; ++t) {
    __syncthreads();  // frame t + pt is staged; the previous frame's output reads are done
    if (t + 1 < t1) prefetch(t + 1 + PT);
    for (int tile = 0; tile < g.tiles; ++tile) {
      const uint32_t addr = taddr[tile];
      dwm_f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      // a frame's kh B operands are read together; the next frame's reads are
      // issued before this frame's MFMAs
      dwm_u16x8_t bv[2][KH];
      auto read_frame = [&](int dt, dwm_u16x8_t* dst) {
        const int slot = (t + dt - PT + KT) % KT;
#pragma unroll
        for (int dh = 0; dh < KH; ++dh)
          dst[dh] = *reinterpret_cast<lds_u16x8*>(
              addr + 2u * static_cast<uint32_t>((slot * g.xr + dh) * g.xps));
      };
      read_frame(0, bv[0]);
#pragma unroll
      for (int dt = 0; dt < KT; ++dt) {
        if (dt + 1 < KT) read_frame(dt + 1, bv[(dt + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
        for (int dh = 0; dh < KH; ++dh)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              A[dt][dh], __builtin_bit_cast(dwm_bf16x8_t, bv[dt & 1][dh]), acc, 0, 0, 0);
      }
      // acc[i] = out[row r][x = 16 xt + 4 kg + i] of this wave's channel
      if (tval[tile]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // the hardware conversion rounds to nearest even, as from_f32 does
          if (tx[tile] + i < a.W)
            s_o[to[tile] + i * kFwmCh] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(acc[i] + bc));
        }
      }
    }
    __syncthreads();  // every wave's B reads of this frame and output writes are done
    // the next frame into the ring slot of frame t - pt (no longer read), and
    // this frame's outputs from LDS to the token rows
    if (t + 1 < t1) commit(t + 1 + PT);
    const int rows = min(g.R, a.H - h0);
    bf16* const obase = out + ((static_cast<int64_t>(b) * a.T + t) * a.H + h0) * rowstride + c0;
    for (int e = threadIdx.x; e < rows * a.W; e += 64 * kFwmCh) {
      const int r = static_cast<int>((static_cast<float>(e) + 0.5f) * g.rW);
      const int x = e - r * a.W;
      *reinterpret_cast<uint4*>(obase + r * rowstride + static_cast<int64_t>(x) * a.C) =
          *reinterpret_cast<const uint4*>(s_o + r * orow + x * kFwmCh);
    }
  }
}

// Cycles of a wave's 16-byte B reads of one tile under the LDS bank model
// (64 banks of 4 bytes; lanes served in four passes of 16, pass = 2 (l >> 5) +
// parity of bits 2-4 of l; 4 = conflict-free).
inline int fwm_read_cycles(int xps, int R, int S, int tile) {
  int addr[64], pass[64];
  for (int l = 0; l < 64; ++l) {
    const int n = l & 15, kg = l >> 4;
    const int s = std::min(16 * tile + n, S - 1);
    const int xt = s / R, r = s - xt * R;
    addr[l] = 2 * (r * xps + 16 * xt + 8 * kg);
    pass[l] = 2 * (l >> 5) + (__builtin_popcount((l >> 2) & 7) & 1);
  }
  int cyc = 0;
  for (int p = 0; p < 4; ++p) {
    int cnt[16] = {};
    for (int l = 0; l < 64; ++l) {
      if (pass[l] != p) continue;
      bool dup = false;
      for (int k = 0; k < l; ++k) dup = dup || (pass[k] == p && addr[k] == addr[l]);
      if (!dup) ++cnt[(addr[l] / 16) % 16];
    }
    cyc += *std::max_element(cnt, cnt + 16);
  }
  return cyc;
}

// Read cycles per band (all tiles) by x tiles (1..16), band rows (32, 16, 8,
// 4, 2, 1) and row padding (0, 8, ..., 120 elements), computed once.
struct FwmCycles {
  int c[16][6][16];
};
inline const FwmCycles& fwm_cycles() {
  static const FwmCycles tab = [] {
    FwmCycles t{};
    for (int nxt = 1; nxt <= 16; ++nxt)
      for (int ri = 0; ri < 6; ++ri)
        for (int pi = 0; pi < 16; ++pi) {
          const int R = 32 >> ri, S = R * nxt, xps = 16 * nxt + 16 + 8 * pi;
          int cyc = 0;
          if (S <= 16 * kFwmMaxTiles)
            for (int tile = 0; tile < (S + 15) / 16; ++tile) cyc += fwm_read_cycles(xps, R, S, tile);
          t.c[nxt - 1][ri][pi] = cyc;
        }
    return t;
  }();
  return tab;
}

// Geometry of the matrix-core convolution, or R = 0 where it does not apply.
inline FwmGeom fwm_geometry(const ConvArgs& a) {
  FwmGeom g{};
  if (a.C % kFwmCh != 0 || a.W % 4 != 0 || a.W < 4 || a.W > 256 || a.H < 1) return g;
  // the input is read through a buffer resource (32-bit byte offsets)
  if (static_cast<int64_t>(a.B) * a.N * a.C * 2 >= kBufMaxBytes) return g;
  if (static_cast<int64_t>(a.B) * a.T * a.H >= (int64_t{1} << 30)) return g;  // 32-bit indices
  g.nxt = (a.W + 15) / 16;
  for (int R = 32; R >= 1; R >>= 1) {
    if (R > 1 && R / 2 >= a.H) continue;  // bands no taller than needed
    const int S = R * g.nxt;
    if (S > 16 * kFwmMaxTiles) continue;
    const int xr = R + a.kh - 1;
    if (xr * (a.W / 4) > kFwmGrp * 64 * kFwmCh) continue;  // staged groups per thread
    const int tiles = (S + 15) / 16;
    int best = -1, best_cyc = 1 << 30;
    const int ri = 31 - __builtin_clz(32 / R);
    for (int pi = 0; pi < 16; ++pi) {
      const int xps = 16 * g.nxt + 16 + 8 * pi;
      const int64_t bytes = 2LL * (kFwmCh * static_cast<int64_t>(a.kt) * xr * xps +
                                   static_cast<int64_t>(R) * (a.W * kFwmCh + 8));
      if (bytes > kFwmLdsMax) break;
      const int cyc = fwm_cycles().c[g.nxt - 1][ri][pi];
      if (cyc < best_cyc) {
        best_cyc = cyc;
        best = xps;
      }
    }
    if (best < 0) continue;
    g.R = R;
    g.xr = xr;
    g.xps = best;
    g.tiles = tiles;
    break;
  }
  if (g.R == 0) return g;
  g.x_elems = a.kt * g.xr * g.xps;
  const int64_t stage = 2LL * (kFwmCh * static_cast<int64_t>(g.x_elems) +
                               static_cast<int64_t>(g.R) * (a.W * kFwmCh + 8));
  const int kp = (a.kt * a.kh * a.kw + 7) / 8 * 8;  // raw weight row
  const int64_t table = 2LL * kFwmCh * (a.kt * a.kh * kFwmTopRow + kp);
  g.lds = static_cast<int>(std::max(stage, table));
  g.bands = (a.H + g.R - 1) / g.R;
  g.rW = 1.0f / static_cast<float>(a.W);
  g.ng = a.W / 4;
  g.rng = 1.0f / static_cast<float>(g.ng);
  // runs along T: as long as leaves about two rounds of two workgroups per CU
  // (each run stages kt - 1 frames beyond its own)
  const int64_t ncb = a.C / kFwmCh;
  g.tr = a.T;
  while (g.tr > 8 && static_cast<int64_t>(a.B) * g.bands * ((a.T + g.tr - 1) / g.tr) * ncb < 1024)
    g.tr = (g.tr + 1) / 2;
  g.nruns = (a.T + g.tr - 1) / g.tr;
  g.nig = static_cast<int>((static_cast<int64_t>(a.B) * g.bands * g.nruns + 7) / 8 * 8);
  return g;
}

// ---------------------------------------------------------------------------
// weight / bias gradient
// ---------------------------------------------------------------------------

// acc[tap*C + c] += sum over a strip of kStripRows rows (all of W) of
// dz[p, c] * x[p + tap - pad, c]; acc[K*C + c] += sum dz[p, c].
template <typename T, typename G, int KT, int KH, int KW>
__global__ __launch_bounds__(64 * kRowWaves) void dwconv_dw_rows_kernel(ConvArgs a,
                                                                        const T* __restrict__ x,
                                                                        const G* __restrict__ dz,
                                                                        float* __restrict__ acc) {
  constexpr int K = KT * KH * KW;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = blockIdx.y * 64 + lane;
  const int64_t rows = static_cast<int64_t>(a.B) * a.T * a.H;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * kRowWaves + wave) * kStripRows;
  if (c >= a.C || r0 >= rows) return;
  const int64_t r1 = r0 + kStripRows < rows ? r0 + kStripRows : rows;
  float s[K];
  float sb = 0.0f;
#pragma unroll
  for (int i = 0; i < K; ++i) s[i] = 0.0f;
  for (int64_t bth = r0; bth < r1; ++bth) {
    const int h = static_cast<int>(bth % a.H);
    const int t = static_cast<int>((bth / a.H) % a.T);
    const int b = static_cast<int>(bth / (static_cast<int64_t>(a.H) * a.T));
    for (int w0 = 0; w0 < a.W; w0 += kRun) {
      float g[kRun];
      const G* __restrict__ gr = dz + (bth * a.W) * static_cast<int64_t>(a.C) + c;
#pragma unroll
      for (int r = 0; r < kRun; ++r) {
        const int w = w0 + r;
        g[r] = w < a.W ? ld(gr, static_cast<int64_t>(w) * a.C) : 0.0f;
        sb += g[r];
      }
#pragma unroll
      for (int dt = 0; dt < KT; ++dt) {
        const int tt = t + dt - KT / 2;
        if (tt < 0 || tt >= a.T) continue;
#pragma unroll
        for (int dh = 0; dh < KH; ++dh) {
          const int hh = h + dh - KH / 2;
          if (hh < 0 || hh >= a.H) continue;
          const int64_t row = (static_cast<int64_t>(b) * a.T + tt) * a.H + hh;
          const T* __restrict__ xr = x + row * a.W * static_cast<int64_t>(a.C) + c;
          float xv[kRun + KW - 1];
#pragma unroll
          for (int j = 0; j < kRun + KW - 1; ++j) {
            const int ww = w0 + j - KW / 2;
            xv[j] = (ww >= 0 && ww < a.W) ? ld(xr, static_cast<int64_t>(ww) * a.C) : 0.0f;
          }
#pragma unroll
          for (int k = 0; k < KW; ++k) {
            float part = 0.0f;
#pragma unroll
            for (int r = 0; r < kRun; ++r) part += g[r] * xv[r + k];
            s[(dt * KH + dh) * KW + k] += part;
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < K; ++i)
    if (s[i] != 0.0f) atomicAdd(acc + static_cast<int64_t>(i) * a.C + c, s[i]);
  if (sb != 0.0f) atomicAdd(acc + static_cast<int64_t>(K) * a.C + c, sb);
}

// ---------------------------------------------------------------------------
// simple kernels for other kernel sizes (one output per thread)
// ---------------------------------------------------------------------------

template <typename T, typename G, int MODE>
__global__ __launch_bounds__(256) void dwconv_simple_kernel(ConvArgs a, const G* __restrict__ in,
                                                            const T* __restrict__ wt,
                                                            const T* __restrict__ bias,
                                                            const T* __restrict__ dy,
                                                            T* __restrict__ out,
                                                            void* __restrict__ out2, int flip) {
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
        acc += ld(wc, flip ? K - 1 - tap : tap) * ld(in, r * a.C + c);
      }
    }
  }
  if (MODE == kPlain) st(out, i, acc);
  if (MODE == kGelu) st(out, i, gelu_erf(acc));
  if (MODE == kGeluSave) {
    st(out, i, gelu_erf(acc));
    st(static_cast<T*>(out2), i, acc);
  }
  if (MODE == kGeluGrad) static_cast<float*>(out2)[i] = ld(dy, i) * gelu_erf_grad(acc);
  if (MODE == kGeluGradT) st(out, i, ld(dy, i) * gelu_erf_grad(acc));
}

constexpr int kChunk = 512;

template <typename T, typename G>
__global__ __launch_bounds__(64) void dwconv_dw_simple_kernel(ConvArgs a, const T* __restrict__ x,
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
  atomicAdd(acc + static_cast<int64_t>(tap) * a.C + c, s);
}

template <typename T>
__global__ __launch_bounds__(256) void dwconv_dw_finish_kernel(const float* __restrict__ acc, int C,
                                                               int K, T* __restrict__ dw,
                                                               T* __restrict__ db) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(C) * (K + 1)) return;  // acc is [K + 1][C]
  const int tap = static_cast<int>(i / C);
  const int c = static_cast<int>(i - static_cast<int64_t>(tap) * C);
  if (tap < K) {
    if (dw != nullptr) st(dw, static_cast<int64_t>(c) * K + tap, acc[i]);
  } else if (db != nullptr) {
    st(db, c, acc[i]);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

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

bool rows_ok(const ConvArgs& a) { return (a.kw == 3 || a.kw == 5 || a.kw == 7) && a.kt <= 7 && a.kh <= 7; }
bool block_ok(const ConvArgs& a) { return a.kh == a.kw && (a.kw == 3 || a.kw == 5 || a.kw == 7); }

template <typename T, typename G, int KS, int MODE>
void launch_block(const ConvArgs& a, const G* in, const T* w, const T* b, const T* dy, T* out,
                  void* out2, int flip, hipStream_t s) {
  const int runs = (a.W + kRun - 1) / kRun;
  const int hblocks = (a.H + kBlockRows - 1) / kBlockRows;
  const int64_t items = static_cast<int64_t>(a.B) * a.T * hblocks * runs;
  const dim3 grid(static_cast<unsigned>((items + kRowWaves - 1) / kRowWaves),
                  static_cast<unsigned>((a.C + 63) / 64));
  if constexpr (std::is_same<T, bf16>::value && std::is_same<G, bf16>::value) {
    if constexpr (MODE == kPlain && KS >= 5) {
      const FwmGeom g = (a.kt == 1 || a.kt == 3) ? fwm_geometry(a) : FwmGeom{};
      if (g.R > 0 && reinterpret_cast<uintptr_t>(in) % 16 == 0 &&
          reinterpret_cast<uintptr_t>(out) % 16 == 0) {
        const dim3 mgrid(static_cast<unsigned>((a.C / kFwmCh) * g.nig));
        if (a.kt == 3)
          hipLaunchKernelGGL((dwconv_fwd_mfma_kernel<3, KS>), mgrid, dim3(64 * kFwmCh),
                             static_cast<unsigned>(g.lds), s, a, g, in, w, b, out, flip);
        else
          hipLaunchKernelGGL((dwconv_fwd_mfma_kernel<1, KS>), mgrid, dim3(64 * kFwmCh),
                             static_cast<unsigned>(g.lds), s, a, g, in, w, b, out, flip);
        return;
      }
    }
    // the dot2 kernel's wide rows are addressed with 32-bit buffer offsets
    if (KS < 5 || static_cast<int64_t>(a.B) * a.N * a.C * 2 < kBufMaxBytes) {
      hipLaunchKernelGGL((dwconv_block_dot2_kernel<KS, KS, MODE>), grid, dim3(64 * kRowWaves), 0,
                         s, a, in, w, b, dy, out, out2, flip);
      return;
    }
  }
  hipLaunchKernelGGL((dwconv_block_kernel<T, G, KS, KS, MODE>), grid, dim3(64 * kRowWaves), 0, s,
                     a, in, w, b, dy, out, out2, flip);
}

// conv of `in` (type G) with w (flip: mirrored taps), epilogue MODE
template <typename T, typename G, int MODE>
hipError_t run_conv(const ConvArgs& a, const G* in, const T* w, const T* b, const T* dy, T* out,
                    void* out2, int flip, hipStream_t s) {
  if (block_ok(a)) {
    if (a.kw == 3) launch_block<T, G, 3, MODE>(a, in, w, b, dy, out, out2, flip, s);
    else if (a.kw == 5) launch_block<T, G, 5, MODE>(a, in, w, b, dy, out, out2, flip, s);
    else launch_block<T, G, 7, MODE>(a, in, w, b, dy, out, out2, flip, s);
  } else if (rows_ok(a)) {
    const int runs = (a.W + kRun - 1) / kRun;
    const int64_t items = static_cast<int64_t>(a.B) * a.T * a.H * runs;
    const dim3 grid(static_cast<unsigned>((items + kRowWaves - 1) / kRowWaves),
                    static_cast<unsigned>((a.C + 63) / 64));
    const dim3 block(64 * kRowWaves);
    switch (a.kw) {
      case 3:
        hipLaunchKernelGGL((dwconv_rows_kernel<T, G, 3, MODE>), grid, block, 0, s, a, in, w, b, dy, out,
                           out2, flip);
        break;
      case 5:
        hipLaunchKernelGGL((dwconv_rows_kernel<T, G, 5, MODE>), grid, block, 0, s, a, in, w, b, dy, out,
                           out2, flip);
        break;
      default:
        hipLaunchKernelGGL((dwconv_rows_kernel<T, G, 7, MODE>), grid, block, 0, s, a, in, w, b, dy, out,
                           out2, flip);
        break;
    }
  } else {
    const int64_t total = static_cast<int64_t>(a.B) * a.N * a.C;
    hipLaunchKernelGGL((dwconv_simple_kernel<T, G, MODE>), dim3(static_cast<unsigned>((total + 255) / 256)),
                       dim3(256), 0, s, a, in, w, b, dy, out, out2, flip);
  }
  return hipGetLastError();
}

template <typename T, typename G, int KS>
void launch_dw_block(const ConvArgs& a, const T* x, const G* dz, float* acc, hipStream_t s) {
  const int hblocks = (a.H + kDwRows - 1) / kDwRows;
  const int strips = (hblocks + kDwStripBlocks - 1) / kDwStripBlocks;
  const int64_t items = static_cast<int64_t>(a.B) * a.T * strips;
  const dim3 grid(static_cast<unsigned>((items + kRowWaves - 1) / kRowWaves),
                  static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(a.kt));
  if constexpr (std::is_same<T, bf16>::value && std::is_same<G, bf16>::value) {
    // the matrix cores pay off from kw = 5 (3x3x3: measured slower than dot2,
    // whose rows are short)
    const DwmGeom g = KS >= 5 ? dwm_geometry(a) : DwmGeom{};
    if (g.R > 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(dz) % 16 == 0) {
      const int64_t mitems = static_cast<int64_t>(a.B) * a.T * g.bands;
      const dim3 mgrid(static_cast<unsigned>((mitems + g.ipw - 1) / g.ipw),
                       static_cast<unsigned>(a.C / kDwmCh));
      hipLaunchKernelGGL((dwconv_dw_mfma_kernel<KS, KS>), mgrid, dim3(64 * kDwmCh),
                         static_cast<unsigned>(dwm_lds_bytes(g)), s, a, g, x, dz, acc);
      return;
    }
    // the dot2 kernel addresses its rows with 32-bit buffer offsets
    if (static_cast<int64_t>(a.B) * a.N * a.C * 2 < kBufMaxBytes) {
      auto go = [&]<int R2>() {
        const int hb2 = (a.H + R2 - 1) / R2;
        const int64_t items2 =
            static_cast<int64_t>(a.B) * a.T * ((hb2 + kDwStripBlocks - 1) / kDwStripBlocks);
        const dim3 grid2(static_cast<unsigned>((items2 + kRowWaves - 1) / kRowWaves),
                         static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(a.kt));
        hipLaunchKernelGGL((dwconv_dw_block_dot2_kernel<KS, KS, R2, kDw2Run<KS>>), grid2,
                           dim3(64 * kRowWaves), 0, s, a, x, dz, acc);
      };
      // 3x3x3 rows wider than 32 voxels: 2-row blocks as well (0.61 -> 0.48 ms at
      // the 46,800-token W = 80 shape, 2.97 -> 2.72 ms at 131,072 tokens; at
      // W = 32, 4-row blocks stay 3% faster)
      if (KS == 3 && a.W > 32)
        go.template operator()<2>();
      else
        go.template operator()<kDw2Rows<KS>>();
      return;
    }
  }
  hipLaunchKernelGGL((dwconv_dw_block_kernel<T, G, KS, KS>), grid, dim3(64 * kRowWaves), 0, s, a,
                     x, dz, acc);
}

template <typename T, typename G>
void run_dw(const ConvArgs& a, const T* x, const G* dz, float* acc, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.T * a.H;
  const dim3 grid(static_cast<unsigned>((rows + kStripRows * kRowWaves - 1) / (kStripRows * kRowWaves)),
                  static_cast<unsigned>((a.C + 63) / 64));
  const dim3 block(64 * kRowWaves);
  if (block_ok(a)) {
    if (a.kw == 3) launch_dw_block<T, G, 3>(a, x, dz, acc, s);
    else if (a.kw == 5) launch_dw_block<T, G, 5>(a, x, dz, acc, s);
    else launch_dw_block<T, G, 7>(a, x, dz, acc, s);
  } else if (a.kt == 3 && a.kh == 7 && a.kw == 7) {
    hipLaunchKernelGGL((dwconv_dw_rows_kernel<T, G, 3, 7, 7>), grid, block, 0, s, a, x, dz, acc);
  } else if (a.kt == 3 && a.kh == 3 && a.kw == 3) {
    hipLaunchKernelGGL((dwconv_dw_rows_kernel<T, G, 3, 3, 3>), grid, block, 0, s, a, x, dz, acc);
  } else {
    const int K = a.kt * a.kh * a.kw;
    const dim3 g(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(K + 1),
                 static_cast<unsigned>((a.B * a.N + kChunk - 1) / kChunk));
    hipLaunchKernelGGL((dwconv_dw_simple_kernel<T, G>), g, dim3(64), 0, s, a, x, dz, acc);
  }
}

template <typename T>
hipError_t fwd_typed(const msd_dwconv3d_desc& d, const void* x, const void* w, const void* b,
                     void* y, void* z, hipStream_t s) {
  const ConvArgs a = make_args(d);
  if (d.act == 1 && z != nullptr)
    return run_conv<T, T, kGeluSave>(a, static_cast<const T*>(x), static_cast<const T*>(w),
                                     static_cast<const T*>(b), nullptr, static_cast<T*>(y), z, 0, s);
  if (d.act == 1)
    return run_conv<T, T, kGelu>(a, static_cast<const T*>(x), static_cast<const T*>(w),
                                 static_cast<const T*>(b), nullptr, static_cast<T*>(y), nullptr, 0, s);
  return run_conv<T, T, kPlain>(a, static_cast<const T*>(x), static_cast<const T*>(w),
                                static_cast<const T*>(b), nullptr, static_cast<T*>(y), nullptr, 0, s);
}

template <typename T, typename G>
hipError_t bwd_grads(const ConvArgs& a, const void* x, const void* w, const G* dz, void* dx,
                     void* dw, void* db, float* acc, hipStream_t s) {
  const int K = a.kt * a.kh * a.kw;
  if (dx != nullptr) {
    hipError_t e = run_conv<T, G, kPlain>(a, dz, static_cast<const T*>(w), nullptr, nullptr,
                                          static_cast<T*>(dx), nullptr, 1, s);
    if (e != hipSuccess) return e;
  }
  if (dw != nullptr || db != nullptr) {
    const int64_t nacc = static_cast<int64_t>(a.C) * (K + 1);
    hipLaunchKernelGGL(fill_zero_f32, dim3(fill_blocks(nacc)), dim3(256), 0, s, acc, nacc);
    run_dw<T, G>(a, static_cast<const T*>(x), dz, acc, s);
    hipLaunchKernelGGL((dwconv_dw_finish_kernel<T>), dim3(static_cast<unsigned>((nacc + 255) / 256)),
                       dim3(256), 0, s, acc, a.C, K, static_cast<T*>(dw), static_cast<T*>(db));
  }
  return hipGetLastError();
}

// dz = dy * gelu'(z) from the saved pre-activation z, 8 elements a thread
// where n allows (16-byte bf16 / 32-byte fp32 rows), grid-stride.
template <typename T, typename O>
__global__ __launch_bounds__(256) void gelu_grad_kernel(const T* __restrict__ dy,
                                                        const T* __restrict__ z,
                                                        O* __restrict__ dz, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t n8 = n / 8;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n8; i += stride) {
    T g[8], p[8];
    O r[8];
    __builtin_memcpy(g, dy + 8 * i, sizeof(g));
    __builtin_memcpy(p, z + 8 * i, sizeof(p));
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = from_f32<O>(to_f32(g[j]) * gelu_erf_grad(to_f32(p[j])));
    __builtin_memcpy(dz + 8 * i, r, sizeof(r));
  }
  for (int64_t i = 8 * n8 + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride)
    dz[i] = from_f32<O>(to_f32(dy[i]) * gelu_erf_grad(to_f32(z[i])));
}

template <typename T>
hipError_t bwd_typed(const msd_dwconv3d_desc& d, const void* x, const void* w, const void* b,
                     const void* z, const void* dy, void* dx, void* dw, void* db, void* ws,
                     hipStream_t s) {
  const ConvArgs a = make_args(d);
  const int K = a.kt * a.kh * a.kw;
  float* acc = static_cast<float*>(ws);
  const int64_t nacc = static_cast<int64_t>(a.C) * (K + 1);
  if (d.act == 1 && z != nullptr) {
    // the forward's pre-activation: dz elementwise, no recomputed convolution
    // (bf16 storage: dz rounded to bf16, as the framework's bf16 GELU backward
    // leaves it, so both gradient convs take the bf16 dot2 kernels)
    float* dz = acc + ((nacc + 63) / 64) * 64;
    const int64_t n = static_cast<int64_t>(a.B) * a.N * a.C;
    const dim3 grid(fill_blocks(n / 8 > 0 ? n / 8 : 1));
    if constexpr (std::is_same<T, bf16>::value) {
      bf16* dzb = reinterpret_cast<bf16*>(dz);
      hipLaunchKernelGGL((gelu_grad_kernel<T, bf16>), grid, dim3(256), 0, s,
                         static_cast<const T*>(dy), static_cast<const T*>(z), dzb, n);
      return bwd_grads<T, T>(a, x, w, dzb, dx, dw, db, acc, s);
    } else {
      hipLaunchKernelGGL((gelu_grad_kernel<T, float>), grid, dim3(256), 0, s,
                         static_cast<const T*>(dy), static_cast<const T*>(z), dz, n);
      return bwd_grads<T, float>(a, x, w, dz, dx, dw, db, acc, s);
    }
  }
  if (d.act == 1) {
    float* dz = acc + ((nacc + 63) / 64) * 64;
    if constexpr (std::is_same<T, bf16>::value) {
      // bf16 storage: dz rounded to bf16 as the framework's bf16 GELU backward
      // leaves it, which lets both gradient convs take the bf16 dot2 kernels
      bf16* dzb = reinterpret_cast<bf16*>(dz);
      hipError_t e = run_conv<T, T, kGeluGradT>(a, static_cast<const T*>(x),
                                                static_cast<const T*>(w), static_cast<const T*>(b),
                                                static_cast<const T*>(dy), dzb, nullptr, 0, s);
      if (e != hipSuccess) return e;
      return bwd_grads<T, T>(a, x, w, dzb, dx, dw, db, acc, s);
    } else {
      hipError_t e = run_conv<T, T, kGeluGrad>(a, static_cast<const T*>(x),
                                               static_cast<const T*>(w), static_cast<const T*>(b),
                                               static_cast<const T*>(dy), nullptr, dz, 0, s);
      if (e != hipSuccess) return e;
      return bwd_grads<T, float>(a, x, w, dz, dx, dw, db, acc, s);
    }
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
                               const void* b, void* y, void* z, hipStream_t s) {
  if (d.dtype == MSD_BF16) return fwd_typed<bf16>(d, x, w, b, y, z, s);
  return fwd_typed<float>(d, x, w, b, y, z, s);
}

hipError_t launch_dwconv3d_bwd(const msd_dwconv3d_desc& d, const void* x, const void* w,
                               const void* b, const void* z, const void* dy, void* dx, void* dw,
                               void* db, void* ws, hipStream_t s) {
  if (d.dtype == MSD_BF16) return bwd_typed<bf16>(d, x, w, b, z, dy, dx, dw, db, ws, s);
  return bwd_typed<float>(d, x, w, b, z, dy, dx, dw, db, ws, s);
}

}  // namespace msd
