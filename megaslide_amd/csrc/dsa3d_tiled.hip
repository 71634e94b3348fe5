// Tiled 3D-DSA kernels for gfx950 (bf16 storage, fp32 accumulation, head_dim 64).
//
// A workgroup of 4 waves owns one (batch, head, tile of 16 queries: 1 frame x
// 4 rows x 4 columns).  Instead of gathering 8 corner rows of K and V per tap
// (147 taps x 8 corners x 64 channels per query), it computes dense score
// tables on the matrix cores and resolves taps with table lookups:
//
//   for every z-plane touched by the tile's taps, over the (y, x) bounding
//   box of the tile's corners (split into chunks of <= 256 voxels):
//     S[q, v] = q . K[v]                         MFMA 16x16x32 bf16 -> LDS fp32
//   per (query, tap) lane: s = scale * sum_c w_c S[q, corner_c]  (trilinear)
//   softmax over each query's taps in registers (wave reductions)
//   per plane/chunk again: A[q, v] = sum_{taps, corners -> v} p * w   (LDS atomics)
//     O[q, :] += A[q, :] . V[chunk, :]           MFMA, V staged transposed in LDS
//
// The result equals the reference's grid_sample + matmul + softmax + matmul
// (infinity/video/attention.py:106-186) because trilinear sampling is linear in
// the sampled values: q . (sum_c w_c K_c) = sum_c w_c (q . K_c), and
// sum_k p_k sum_c w_c V_c = sum_v (sum_{k,c -> v} p_k w_c) V_v.
// Sampling coordinates, corner choice and weights are computed exactly as in
// the direct kernels (same fp32 op order as the reference).
//
// Precision: q, K, V are bf16 inputs (exact in the MFMA); S, O accumulate in
// fp32.  The A table enters the MFMA as a bf16 hi/lo pair (A = hi + lo), so
// its rounding error is ~2^-16 relative.
#include "common.h"
#include "dsa3d_coords.h"

namespace msd {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;

constexpr int kHD = 64;           // head_dim handled by the tiled kernels
constexpr int kTileH = 4, kTileW = 4;
constexpr int kTQ = kTileH * kTileW;  // 16 queries per tile
constexpr int kThreads = 256;     // 4 waves
constexpr int kSlots = 10;        // taps per lane: K <= 16 * kSlots = 160
constexpr int kChunkY = 16, kChunkX = 16;
constexpr int kChunkNV = kChunkY * kChunkX;   // voxels per chunk (<= 256)
constexpr int kSRow = kChunkNV + 4;           // fp32 row stride of S / A tables
constexpr int kVRow = kChunkNV + 8;           // bf16 row stride of the transposed V tile

struct TiledArgs {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* off;
  bf16* out;
  float* lse;
  int64_t qs, ks, vs;
  int64_t N;
  int B, T, H, W, nh, kt, kh, kw, K, C;
  int tiles_h, tiles_w;
  float offset_scale, softmax_scale;
  float div_x, div_y, div_z;
};

__device__ __forceinline__ bf16x8_t load_bf16x8(const bf16* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}

__device__ __forceinline__ bf16x8_t zero_bf16x8() {
  const u32x4_t z = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(bf16x8_t, z);
}

// Packed per-tap geometry kept in registers between the passes.
struct Tap {
  int yx;     // y0 | x0 << 16
  int zf;     // z0 | (hi_z << 16) | (hi_y << 17) | (hi_x << 18); z0 = -1 for an empty slot
  float fx, fy, fz;
};

__device__ __forceinline__ int tap_z0(const Tap& t) { return static_cast<int16_t>(t.zf & 0xffff); }

__global__ __launch_bounds__(kThreads) void dsa3d_fwd_tiled_kernel(TiledArgs a) {
  __shared__ float s_tab[kTQ * kSRow];               // S[q][v], then A[q][v]
  __shared__ __attribute__((aligned(16))) uint16_t s_vt[kHD * kVRow];  // V^T chunk (bf16)
  __shared__ int s_red[4][6];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int head = blockIdx.y;
  int tile = blockIdx.x;
  const int tw_i = tile % a.tiles_w;
  tile /= a.tiles_w;
  const int th_i = tile % a.tiles_h;
  tile /= a.tiles_h;
  const int t = tile % a.T;
  const int b = tile / a.T;
  const int h0 = th_i * kTileH, w0 = tw_i * kTileW;
  const int64_t sample0 = static_cast<int64_t>(b) * a.N;

  // ---- this lane's query and tap slots --------------------------------------
  const int q = wave * 4 + (lane & 3);         // query index in the tile
  const int sub = lane >> 2;                   // 0..15
  const int qh = h0 + q / kTileW, qw = w0 + q % kTileW;
  const bool q_ok = qh < a.H && qw < a.W;
  const int64_t qn = sample0 + (static_cast<int64_t>(t) * a.H + qh) * a.W + qw;

  Tap taps[kSlots];
  int zlo = 1 << 30, zhi = -1, ylo = 1 << 30, yhi = -1, xlo = 1 << 30, xhi = -1;
  {
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int kap = sub + 16 * i;
      taps[i].zf = 0xffff;  // z0 = -1
      taps[i].yx = 0;
      taps[i].fx = taps[i].fy = taps[i].fz = 0.0f;
      if (!q_ok || kap >= a.K) continue;
      const int ci = kap / (a.kh * a.kw) - a.kt / 2;
      const int cj = (kap / a.kw) % a.kh - a.kh / 2;
      const int ck = kap % a.kw - a.kw / 2;
      const bf16* op = a.off + qn * a.C + (static_cast<int64_t>(head) * a.K + kap) * 3;
      const float o0 = to_f32(op[0]) * a.offset_scale;
      const float o1 = to_f32(op[1]) * a.offset_scale;
      const float o2 = to_f32(op[2]) * a.offset_scale;
      const Axis ax = axis_sample(grid_coord(base_coord(qw, ck, a.W), o0, a.div_x), a.W);
      const Axis ay = axis_sample(grid_coord(base_coord(qh, cj, a.H), o1, a.div_y), a.H);
      const Axis az = axis_sample(grid_coord(base_coord(t, ci, a.T), o2, a.div_z), a.T);
      taps[i].yx = ay.i0 | (ax.i0 << 16);
      taps[i].zf = az.i0 | (az.hi_ok << 16) | (ay.hi_ok << 17) | (ax.hi_ok << 18);
      taps[i].fx = ax.f;
      taps[i].fy = ay.f;
      taps[i].fz = az.f;
      zlo = min(zlo, az.i0);
      zhi = max(zhi, az.i0 + (az.hi_ok ? 1 : 0));
      ylo = min(ylo, ay.i0);
      yhi = max(yhi, ay.i0 + (ay.hi_ok ? 1 : 0));
      xlo = min(xlo, ax.i0);
      xhi = max(xhi, ax.i0 + (ax.hi_ok ? 1 : 0));
    }
  }
  // block-wide bounding box of all corners
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    zlo = min(zlo, __shfl_xor(zlo, m));
    zhi = max(zhi, __shfl_xor(zhi, m));
    ylo = min(ylo, __shfl_xor(ylo, m));
    yhi = max(yhi, __shfl_xor(yhi, m));
    xlo = min(xlo, __shfl_xor(xlo, m));
    xhi = max(xhi, __shfl_xor(xhi, m));
  }
  if (lane == 0) {
    s_red[wave][0] = zlo;
    s_red[wave][1] = zhi;
    s_red[wave][2] = ylo;
    s_red[wave][3] = yhi;
    s_red[wave][4] = xlo;
    s_red[wave][5] = xhi;
  }
  __syncthreads();
  zlo = min(min(s_red[0][0], s_red[1][0]), min(s_red[2][0], s_red[3][0]));
  zhi = max(max(s_red[0][1], s_red[1][1]), max(s_red[2][1], s_red[3][1]));
  ylo = min(min(s_red[0][2], s_red[1][2]), min(s_red[2][2], s_red[3][2]));
  yhi = max(max(s_red[0][3], s_red[1][3]), max(s_red[2][3], s_red[3][3]));
  xlo = min(min(s_red[0][4], s_red[1][4]), min(s_red[2][4], s_red[3][4]));
  xhi = max(max(s_red[0][5], s_red[1][5]), max(s_red[2][5], s_red[3][5]));

  // ---- Q as the MFMA A operand: row = query lane%16, k = 8*(lane/16) + j ----
  const int mq = lane & 15;            // query row of the MFMA operand
  const int kq = 8 * (lane >> 4);      // channel offset within a 32-channel chunk
  bf16x8_t qa0 = zero_bf16x8(), qa1 = zero_bf16x8();
  {
    const int mh = h0 + mq / kTileW, mw = w0 + mq % kTileW;
    if (mh < a.H && mw < a.W) {
      const int64_t n = sample0 + (static_cast<int64_t>(t) * a.H + mh) * a.W + mw;
      const bf16* qp = a.q + n * a.qs + head * kHD;
      qa0 = load_bf16x8(qp + kq);
      qa1 = load_bf16x8(qp + 32 + kq);
    }
  }

  // ---- pass 1: scores -------------------------------------------------------
  float sacc[kSlots];
#pragma unroll
  for (int i = 0; i < kSlots; ++i) sacc[i] = 0.0f;

  for (int z = zlo; z <= zhi; ++z) {
    for (int cy0 = ylo; cy0 <= yhi; cy0 += kChunkY) {
      const int ny = min(kChunkY, yhi - cy0 + 1);
      for (int cx0 = xlo; cx0 <= xhi; cx0 += kChunkX) {
        const int nx = min(kChunkX, xhi - cx0 + 1);
        const int nv = ny * nx;
        // S = Q . K^T over the chunk, 16 voxels per MFMA block, blocks split over waves
        for (int blk = wave; blk * 16 < nv; blk += 4) {
          const int vi = blk * 16 + (lane & 15);
          bf16x8_t kb0 = zero_bf16x8(), kb1 = zero_bf16x8();
          if (vi < nv) {
            const int yy = cy0 + vi / nx, xx = cx0 + vi % nx;
            const int64_t row = sample0 + (static_cast<int64_t>(z) * a.H + yy) * a.W + xx;
            const bf16* kp = a.k + row * a.ks + head * kHD;
            kb0 = load_bf16x8(kp + kq);
            kb1 = load_bf16x8(kp + 32 + kq);
          }
          f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa0, kb0, c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa1, kb1, c, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) s_tab[(4 * (lane >> 4) + r) * kSRow + vi] = c[r];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kSlots; ++i) {
          const int z0 = tap_z0(taps[i]);
          const bool hz = (taps[i].zf >> 16) & 1;
          if (z0 != z && !(hz && z0 + 1 == z)) continue;
          const float wz = (z0 == z) ? 1.0f - taps[i].fz : taps[i].fz;
          const int y0 = taps[i].yx & 0xffff, x0 = taps[i].yx >> 16;
          const bool hy = (taps[i].zf >> 17) & 1, hx = (taps[i].zf >> 18) & 1;
          float part = 0.0f;
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) {
            const int dy = c4 >> 1, dx = c4 & 1;
            if ((dy && !hy) || (dx && !hx)) continue;
            const int yy = y0 + dy - cy0, xx = x0 + dx - cx0;
            if (yy < 0 || yy >= ny || xx < 0 || xx >= nx) continue;
            const float wyx = (dy ? taps[i].fy : 1.0f - taps[i].fy) * (dx ? taps[i].fx : 1.0f - taps[i].fx);
            part += wyx * s_tab[q * kSRow + yy * nx + xx];
          }
          sacc[i] += wz * part;
        }
        __syncthreads();
      }
    }
  }

  // ---- softmax over each query's taps (16 lanes x kSlots) -------------------
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    sacc[i] = (tap_z0(taps[i]) >= 0) ? sacc[i] * a.softmax_scale : -INFINITY;
    mx = fmaxf(mx, sacc[i]);
  }
#pragma unroll
  for (int m = 4; m <= 32; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  float den = 0.0f;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    sacc[i] = (tap_z0(taps[i]) >= 0) ? __expf(sacc[i] - mx) : 0.0f;
    den += sacc[i];
  }
#pragma unroll
  for (int m = 4; m <= 32; m <<= 1) den += __shfl_xor(den, m);
  const float inv_den = 1.0f / den;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) sacc[i] *= inv_den;  // now p
  if (a.lse != nullptr && q_ok && sub == 0) a.lse[qn * a.nh + head] = mx + logf(den);

  // ---- pass 2: O = A . V ------------------------------------------------------
  f32x4_t oacc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int nb = wave;  // this wave's 16 output channels
  for (int z = zlo; z <= zhi; ++z) {
    for (int cy0 = ylo; cy0 <= yhi; cy0 += kChunkY) {
      const int ny = min(kChunkY, yhi - cy0 + 1);
      for (int cx0 = xlo; cx0 <= xhi; cx0 += kChunkX) {
        const int nx = min(kChunkX, xhi - cx0 + 1);
        const int nv = ny * nx;
        const int nvp = (nv + 31) & ~31;
        // zero the A table, stage V^T (zero padded to nvp voxels)
        for (int e = tid; e < kTQ * nvp; e += kThreads) s_tab[(e / nvp) * kSRow + e % nvp] = 0.0f;
        for (int task = tid; task < (nvp / 2) * 8; task += kThreads) {
          const int vp = task >> 3, cg = task & 7;
          const int v0 = 2 * vp, v1 = v0 + 1;
          // 8 channels of voxels v0 and v1 as 4 dwords each (channel 2i in the low half)
          u32x4_t x0 = {0u, 0u, 0u, 0u}, x1 = {0u, 0u, 0u, 0u};
          if (v0 < nv) {
            const int yy = cy0 + v0 / nx, xx = cx0 + v0 % nx;
            const int64_t row = sample0 + (static_cast<int64_t>(z) * a.H + yy) * a.W + xx;
            __builtin_memcpy(&x0, a.v + row * a.vs + head * kHD + 8 * cg, sizeof(x0));
          }
          if (v1 < nv) {
            const int yy = cy0 + v1 / nx, xx = cx0 + v1 % nx;
            const int64_t row = sample0 + (static_cast<int64_t>(z) * a.H + yy) * a.W + xx;
            __builtin_memcpy(&x1, a.v + row * a.vs + head * kHD + 8 * cg, sizeof(x1));
          }
          // V^T rows 8cg+2i (low halves) and 8cg+2i+1 (high halves), voxels v0, v1
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t even = (x0[i] & 0xffffu) | (x1[i] << 16);
            const uint32_t odd = (x0[i] >> 16) | (x1[i] & 0xffff0000u);
            __builtin_memcpy(&s_vt[(8 * cg + 2 * i) * kVRow + v0], &even, sizeof(even));
            __builtin_memcpy(&s_vt[(8 * cg + 2 * i + 1) * kVRow + v0], &odd, sizeof(odd));
          }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kSlots; ++i) {
          const int z0 = tap_z0(taps[i]);
          const bool hz = (taps[i].zf >> 16) & 1;
          if (z0 != z && !(hz && z0 + 1 == z)) continue;
          const float pz = sacc[i] * ((z0 == z) ? 1.0f - taps[i].fz : taps[i].fz);
          const int y0 = taps[i].yx & 0xffff, x0 = taps[i].yx >> 16;
          const bool hy = (taps[i].zf >> 17) & 1, hx = (taps[i].zf >> 18) & 1;
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) {
            const int dy = c4 >> 1, dx = c4 & 1;
            if ((dy && !hy) || (dx && !hx)) continue;
            const int yy = y0 + dy - cy0, xx = x0 + dx - cx0;
            if (yy < 0 || yy >= ny || xx < 0 || xx >= nx) continue;
            const float wyx = (dy ? taps[i].fy : 1.0f - taps[i].fy) * (dx ? taps[i].fx : 1.0f - taps[i].fx);
            atomicAdd(&s_tab[q * kSRow + yy * nx + xx], pz * wyx);
          }
        }
        __syncthreads();
        for (int kc = 0; kc < nvp; kc += 32) {
          // A row as a bf16 hi/lo pair, packed two values per dword
          const float* ar = &s_tab[mq * kSRow + kc + kq];
          u32x4_t hi4, lo4;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x0 = ar[2 * i], x1 = ar[2 * i + 1];
            const uint32_t h0 = from_f32<bf16>(x0).bits, h1 = from_f32<bf16>(x1).bits;
            const uint32_t l0 = from_f32<bf16>(x0 - __uint_as_float(h0 << 16)).bits;
            const uint32_t l1 = from_f32<bf16>(x1 - __uint_as_float(h1 << 16)).bits;
            hi4[i] = h0 | (h1 << 16);
            lo4[i] = l0 | (l1 << 16);
          }
          const bf16x8_t ahi = __builtin_bit_cast(bf16x8_t, hi4);
          const bf16x8_t alo = __builtin_bit_cast(bf16x8_t, lo4);
          bf16x8_t bv;
          __builtin_memcpy(&bv, &s_vt[(16 * nb + mq) * kVRow + kc + kq], sizeof(bv));
          oacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, bv, oacc, 0, 0, 0);
          oacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bv, oacc, 0, 0, 0);
        }
        __syncthreads();
      }
    }
  }
  // oacc[r] = O[query 4*(lane/16) + r][channel 16*nb + lane%16]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int oq = 4 * (lane >> 4) + r;
    const int oh = h0 + oq / kTileW, ow = w0 + oq % kTileW;
    if (oh < a.H && ow < a.W) {
      const int64_t n = sample0 + (static_cast<int64_t>(t) * a.H + oh) * a.W + ow;
      a.out[n * (static_cast<int64_t>(a.nh) * kHD) + head * kHD + 16 * nb + mq] = from_f32<bf16>(oacc[r]);
    }
  }
}

}  // namespace

bool dsa3d_tiled_supported(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v) {
  if (d.dtype != MSD_BF16 || d.head_dim != kHD) return false;
  if (d.kt * d.kh * d.kw > 16 * kSlots) return false;
  if (d.H > 32767 || d.W > 32767 || d.T > 32767) return false;
  // 16-byte vector loads of q/k/v rows
  if ((d.q_stride % 8) || (d.k_stride % 8) || (d.v_stride % 8)) return false;
  for (const void* p : {q, k, v})
    if (reinterpret_cast<uintptr_t>(p) % 16) return false;
  return true;
}

hipError_t launch_dsa3d_fwd_tiled(const msd_dsa3d_desc& d, const void* q, const void* k,
                                  const void* v, const void* off, void* out, float* lse,
                                  hipStream_t s) {
  TiledArgs a;
  a.q = static_cast<const bf16*>(q);
  a.k = static_cast<const bf16*>(k);
  a.v = static_cast<const bf16*>(v);
  a.off = static_cast<const bf16*>(off);
  a.out = static_cast<bf16*>(out);
  a.lse = lse;
  a.qs = d.q_stride;
  a.ks = d.k_stride;
  a.vs = d.v_stride;
  a.N = static_cast<int64_t>(d.T) * d.H * d.W;
  a.B = d.B;
  a.T = d.T;
  a.H = d.H;
  a.W = d.W;
  a.nh = d.num_heads;
  a.kt = d.kt;
  a.kh = d.kh;
  a.kw = d.kw;
  a.K = d.kt * d.kh * d.kw;
  a.C = d.num_heads * a.K * 3;
  a.tiles_h = (d.H + kTileH - 1) / kTileH;
  a.tiles_w = (d.W + kTileW - 1) / kTileW;
  a.offset_scale = d.offset_scale;
  a.softmax_scale = d.softmax_scale;
  a.div_x = d.T > 1 ? static_cast<float>(d.T - 1) : 0.0f;
  a.div_y = d.H > 1 ? static_cast<float>(d.H - 1) : 0.0f;
  a.div_z = d.W > 1 ? static_cast<float>(d.W - 1) : 0.0f;
  const int64_t tiles = static_cast<int64_t>(d.B) * d.T * a.tiles_h * a.tiles_w;
  hipLaunchKernelGGL(dsa3d_fwd_tiled_kernel, dim3(static_cast<unsigned>(tiles), d.num_heads),
                     dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace msd
