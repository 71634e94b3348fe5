// Shared building blocks of the matrix-core (tiled) 3D-DSA kernels.
//
// A workgroup of 4 waves owns one (batch, head, tile of 16 queries = 1 frame x
// 4 rows x 4 columns).  Lane l of wave w serves query q = 4w + (l & 3) and the
// taps kappa = (l >> 2) + 16 i, i < kSlots.  Every tap's 2x2 (y, x) corner
// footprint is resolved against per-plane score tables
//   S[q][v] = X[q] . Y[v]   (X = q or dO rows, Y = K or V rows; MFMA, fp32 in LDS)
// built over the (y, x) bounding box of all corners of the tile, cut into
// 16 x 16 chunks whose starts are 15 voxels apart: two adjacent voxels always
// share a chunk, so each tap is assigned to exactly one chunk.
#pragma once

#include "common.h"
#include "dsa3d_coords.h"

namespace msd {
namespace tiled {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;

constexpr int kHD = 64;                 // head_dim served by the tiled kernels
constexpr int kTileH = 4, kTileW = 4;
constexpr int kTQ = kTileH * kTileW;    // queries per tile
constexpr int kThreads = 256;           // 4 waves
constexpr int kSlots = 10;              // taps per lane: windows of <= 160 taps
constexpr int kChunk = 16;              // chunk edge in y and x
constexpr int kChunkStep = 15;          // chunk start spacing (one voxel of overlap)
constexpr int kChunkNV = kChunk * kChunk;
// fp32 row stride of the tables: 260 = 4 (mod 64 banks), so the four row groups
// an MFMA result writes (rows r, r+4, r+8, r+12) and the 16 rows an operand
// read touches fall on distinct banks.
constexpr int kSRow = kChunkNV + 4;
constexpr int kVRow = kChunkNV + 8;     // bf16 row stride of a transposed K/V chunk

struct Args {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* off;
  int64_t qs, ks, vs;  // token strides of q, k, v
  int64_t N;
  int B, T, H, W, nh, kt, kh, kw, K, C;
  int tiles_h, tiles_w;
  float offset_scale, softmax_scale;
  float div_x, div_y, div_z;     // divisors of offset slots 0, 1, 2 (0 = slot dropped)
  float rdiv_x, rdiv_y, rdiv_z;  // their reciprocals (0 = slot dropped)
};

// Geometry of one tap, kept in registers between the passes.
struct Slot {
  int zc;    // z0 (bits 0-15, -1 = empty) | hz << 16 | clamp-gradient mask x,y,z << 17..19 | chunk << 20
  int idx;   // table index of corner (y0, x0) | dy_off << 9 | dx_off << 14
  float w00, w01, w10, w11;  // (y, x) bilinear weights of the corners (0 outside the volume)
  float fz;                  // weight of the upper z corner
  float fx, fy;              // fractional parts (for coordinate gradients)
};

__device__ __forceinline__ int slot_z0(const Slot& s) { return static_cast<int16_t>(s.zc & 0xffff); }
__device__ __forceinline__ bool slot_hz(const Slot& s) { return (s.zc >> 16) & 1; }
__device__ __forceinline__ int slot_chunk(const Slot& s) { return s.zc >> 20; }

struct Tile {
  int b, head, t, h0, w0;
  int64_t sample0;
  int wave, lane, q, sub;
  bool q_ok;
  int64_t qn;  // token row of this lane's query
};

__device__ __forceinline__ Tile make_tile(const Args& a) {
  Tile t;
  t.head = blockIdx.y;
  int tile = blockIdx.x;
  const int tw_i = tile % a.tiles_w;
  tile /= a.tiles_w;
  const int th_i = tile % a.tiles_h;
  tile /= a.tiles_h;
  t.t = tile % a.T;
  t.b = tile / a.T;
  t.h0 = th_i * kTileH;
  t.w0 = tw_i * kTileW;
  t.sample0 = static_cast<int64_t>(t.b) * a.N;
  t.wave = threadIdx.x >> 6;
  t.lane = threadIdx.x & 63;
  t.q = t.wave * 4 + (t.lane & 3);
  t.sub = t.lane >> 2;
  const int qh = t.h0 + t.q / kTileW, qw = t.w0 + t.q % kTileW;
  t.q_ok = qh < a.H && qw < a.W;
  t.qn = t.sample0 + (static_cast<int64_t>(t.t) * a.H + qh) * a.W + qw;
  return t;
}

// Token row of tile query m (0..15), or -1 outside the grid.
__device__ __forceinline__ int64_t tile_row(const Args& a, const Tile& t, int m) {
  const int h = t.h0 + m / kTileW, w = t.w0 + m % kTileW;
  if (h >= a.H || w >= a.W) return -1;
  return t.sample0 + (static_cast<int64_t>(t.t) * a.H + h) * a.W + w;
}

struct Box {
  int zlo, zhi, ylo, yhi, xlo, xhi;
  int ncy, ncx;  // chunk grid
};

// Tap geometry for all slots of this lane (coordinates exactly as the
// reference rounds them) and the block-wide bounding box of every corner.
__device__ __forceinline__ void setup_slots(const Args& a, const Tile& tl, Slot* sl, Box& box,
                                            int (*s_red)[6]) {
  int zlo = 1 << 30, zhi = -1, ylo = 1 << 30, yhi = -1, xlo = 1 << 30, xhi = -1;
  int y0s[kSlots], x0s[kSlots], hys[kSlots], hxs[kSlots];
  const int qh = tl.h0 + tl.q / kTileW, qw = tl.w0 + tl.q % kTileW;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const int kap = tl.sub + 16 * i;
    sl[i].zc = 0xffff;  // z0 = -1: empty
    sl[i].idx = 0;
    sl[i].w00 = sl[i].w01 = sl[i].w10 = sl[i].w11 = sl[i].fz = sl[i].fx = sl[i].fy = 0.0f;
    y0s[i] = x0s[i] = hys[i] = hxs[i] = 0;
    if (!tl.q_ok || kap >= a.K) continue;
    const int ci = kap / (a.kh * a.kw) - a.kt / 2;
    const int cj = (kap / a.kw) % a.kh - a.kh / 2;
    const int ck = kap % a.kw - a.kw / 2;
    const bf16* op = a.off + tl.qn * a.C + (static_cast<int64_t>(tl.head) * a.K + kap) * 3;
    const float o0 = to_f32(op[0]) * a.offset_scale;
    const float o1 = to_f32(op[1]) * a.offset_scale;
    const float o2 = to_f32(op[2]) * a.offset_scale;
    const Axis ax = axis_sample(grid_coord(base_coord(qw, ck, a.W), o0, a.div_x), a.W);
    const Axis ay = axis_sample(grid_coord(base_coord(qh, cj, a.H), o1, a.div_y), a.H);
    const Axis az = axis_sample(grid_coord(base_coord(tl.t, ci, a.T), o2, a.div_z), a.T);
    // clamp-gradient masks: zero where u <= 0 or u >= S-1 (grid_sample border padding)
    const int mx = (ax.u > 0.0f && ax.u < static_cast<float>(a.W - 1)) ? 1 : 0;
    const int my = (ay.u > 0.0f && ay.u < static_cast<float>(a.H - 1)) ? 1 : 0;
    const int mz = (az.u > 0.0f && az.u < static_cast<float>(a.T - 1)) ? 1 : 0;
    sl[i].zc = az.i0 | (az.hi_ok << 16) | (mx << 17) | (my << 18) | (mz << 19);
    sl[i].fx = ax.f;
    sl[i].fy = ay.f;
    sl[i].fz = az.f;
    y0s[i] = ay.i0;
    x0s[i] = ax.i0;
    hys[i] = ay.hi_ok;
    hxs[i] = ax.hi_ok;
    zlo = min(zlo, az.i0);
    zhi = max(zhi, az.i0 + (az.hi_ok ? 1 : 0));
    ylo = min(ylo, ay.i0);
    yhi = max(yhi, ay.i0 + (ay.hi_ok ? 1 : 0));
    xlo = min(xlo, ax.i0);
    xhi = max(xhi, ax.i0 + (ax.hi_ok ? 1 : 0));
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    zlo = min(zlo, __shfl_xor(zlo, m));
    zhi = max(zhi, __shfl_xor(zhi, m));
    ylo = min(ylo, __shfl_xor(ylo, m));
    yhi = max(yhi, __shfl_xor(yhi, m));
    xlo = min(xlo, __shfl_xor(xlo, m));
    xhi = max(xhi, __shfl_xor(xhi, m));
  }
  if (tl.lane == 0) {
    s_red[tl.wave][0] = zlo;
    s_red[tl.wave][1] = zhi;
    s_red[tl.wave][2] = ylo;
    s_red[tl.wave][3] = yhi;
    s_red[tl.wave][4] = xlo;
    s_red[tl.wave][5] = xhi;
  }
  __syncthreads();
  box.zlo = min(min(s_red[0][0], s_red[1][0]), min(s_red[2][0], s_red[3][0]));
  box.zhi = max(max(s_red[0][1], s_red[1][1]), max(s_red[2][1], s_red[3][1]));
  box.ylo = min(min(s_red[0][2], s_red[1][2]), min(s_red[2][2], s_red[3][2]));
  box.yhi = max(max(s_red[0][3], s_red[1][3]), max(s_red[2][3], s_red[3][3]));
  box.xlo = min(min(s_red[0][4], s_red[1][4]), min(s_red[2][4], s_red[3][4]));
  box.xhi = max(max(s_red[0][5], s_red[1][5]), max(s_red[2][5], s_red[3][5]));
  // chunk grid: starts lo, lo+15, ...; ceil((extent-1)/15) chunks (at least one)
  box.ncy = max(1, (box.yhi - box.ylo + kChunkStep - 1) / kChunkStep);
  box.ncx = max(1, (box.xhi - box.xlo + kChunkStep - 1) / kChunkStep);
  // assign every tap to the chunk holding its whole 2x2 footprint
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    if (slot_z0(sl[i]) < 0) continue;
    const int cy = min((y0s[i] - box.ylo) / kChunkStep, box.ncy - 1);
    const int cx = min((x0s[i] - box.xlo) / kChunkStep, box.ncx - 1);
    const int cy0 = box.ylo + kChunkStep * cy, cx0 = box.xlo + kChunkStep * cx;
    const int nx = min(kChunk, box.xhi - cx0 + 1);
    const int base = (y0s[i] - cy0) * nx + (x0s[i] - cx0);
    sl[i].idx = base | ((hys[i] ? nx : 0) << 9) | ((hxs[i] ? 1 : 0) << 14);
    sl[i].zc |= (cy * box.ncx + cx) << 20;
    const float fx = sl[i].fx, fy = sl[i].fy;
    sl[i].w00 = (1.0f - fy) * (1.0f - fx);
    sl[i].w01 = hxs[i] ? (1.0f - fy) * fx : 0.0f;
    sl[i].w10 = hys[i] ? fy * (1.0f - fx) : 0.0f;
    sl[i].w11 = (hys[i] && hxs[i]) ? fy * fx : 0.0f;
  }
}

struct Chunk {
  int id, cy0, cx0, ny, nx, nv, nvp;
  float rnx;  // 1/nx, for division-free voxel coordinates
};

__device__ __forceinline__ Chunk make_chunk(const Box& box, int cy, int cx) {
  Chunk c;
  c.id = cy * box.ncx + cx;
  c.cy0 = box.ylo + kChunkStep * cy;
  c.cx0 = box.xlo + kChunkStep * cx;
  c.ny = min(kChunk, box.yhi - c.cy0 + 1);
  c.nx = min(kChunk, box.xhi - c.cx0 + 1);
  c.nv = c.ny * c.nx;
  c.nvp = (c.nv + 31) & ~31;
  c.rnx = 1.0f / static_cast<float>(c.nx);
  return c;
}

// Token row of voxel vi (< nv) of chunk c in plane z.
__device__ __forceinline__ int64_t chunk_row(const Args& a, const Tile& tl, const Chunk& c, int z,
                                             int vi) {
  const int vy = static_cast<int>((static_cast<float>(vi) + 0.5f) * c.rnx);
  const int vx = vi - vy * c.nx;
  return tl.sample0 + (static_cast<int64_t>(z) * a.H + c.cy0 + vy) * a.W + c.cx0 + vx;
}

__device__ __forceinline__ bf16x8_t zero_bf16x8() {
  const u32x4_t z = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(bf16x8_t, z);
}

__device__ __forceinline__ bf16x8_t load8(const bf16* p) {
  u32x4_t r;
  __builtin_memcpy(&r, p, sizeof(r));
  return __builtin_bit_cast(bf16x8_t, r);
}

// Rows of the tile (queries m = lane % 16) as MFMA A operands, channels
// 8*(lane/16) + [0, 8) and 32 + 8*(lane/16) + [0, 8).
__device__ __forceinline__ void load_rows_operand(const Args& a, const Tile& tl, const bf16* base,
                                                  int64_t stride, bf16x8_t& lo, bf16x8_t& hi) {
  lo = hi = zero_bf16x8();
  const int64_t row = tile_row(a, tl, tl.lane & 15);
  if (row < 0) return;
  const bf16* p = base + row * stride + tl.head * kHD + 8 * (tl.lane >> 4);
  lo = load8(p);
  hi = load8(p + 32);
}

// table[m][vi] = X[m] . Y[vi] for the chunk's voxels of plane z (X as MFMA A
// operands, Y rows read from global).  Blocks of 16 voxels are split over waves.
__device__ __forceinline__ void mfma_table(const Args& a, const Tile& tl, const Chunk& c, int z,
                                           const bf16* ybase, int64_t ystride, bf16x8_t x0,
                                           bf16x8_t x1, float* table) {
  const int kq = 8 * (tl.lane >> 4);
  for (int blk = tl.wave; blk * 16 < c.nv; blk += 4) {
    const int vi = blk * 16 + (tl.lane & 15);
    bf16x8_t y0 = zero_bf16x8(), y1 = zero_bf16x8();
    if (vi < c.nv) {
      const bf16* p = ybase + chunk_row(a, tl, c, z, vi) * ystride + tl.head * kHD + kq;
      y0 = load8(p);
      y1 = load8(p + 32);
    }
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0, y0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, y1, acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) table[(4 * (tl.lane >> 4) + r) * kSRow + vi] = acc[r];
  }
}

// Chunk rows of Y (plane z) transposed into LDS: yt[channel][voxel] (bf16),
// zero padded up to nvp voxels.
__device__ __forceinline__ void stage_transposed(const Args& a, const Tile& tl, const Chunk& c,
                                                 int z, const bf16* ybase, int64_t ystride,
                                                 uint16_t* yt) {
  // lanes walk voxel pairs fastest, so a wave's dword stores hit consecutive banks
  for (int task = threadIdx.x; task < 8 * (kChunkNV / 2); task += kThreads) {
    const int cg = task >> 7, vp = task & 127;
    const int v0 = 2 * vp, v1 = v0 + 1;
    if (v0 >= c.nvp) continue;
    u32x4_t x0 = {0u, 0u, 0u, 0u}, x1 = {0u, 0u, 0u, 0u};
    if (v0 < c.nv)
      __builtin_memcpy(&x0, ybase + chunk_row(a, tl, c, z, v0) * ystride + tl.head * kHD + 8 * cg,
                       sizeof(x0));
    if (v1 < c.nv)
      __builtin_memcpy(&x1, ybase + chunk_row(a, tl, c, z, v1) * ystride + tl.head * kHD + 8 * cg,
                       sizeof(x1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t even = (x0[i] & 0xffffu) | (x1[i] << 16);
      const uint32_t odd = (x0[i] >> 16) | (x1[i] & 0xffff0000u);
      __builtin_memcpy(&yt[(8 * cg + 2 * i) * kVRow + v0], &even, sizeof(even));
      __builtin_memcpy(&yt[(8 * cg + 2 * i + 1) * kVRow + v0], &odd, sizeof(odd));
    }
  }
}

// Zero a [16][nvp] fp32 table.
__device__ __forceinline__ void zero_table(float* table, int nvp) {
  for (int task = threadIdx.x; task < kTQ * (kChunkNV / 4); task += kThreads) {
    const int row = task >> 6, c4 = (task & 63) * 4;
    if (c4 < nvp) {
      const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
      __builtin_memcpy(&table[row * kSRow + c4], &z, sizeof(z));
    }
  }
}

// Does this slot have corners on plane z of chunk c?  Returns the z weight.
__device__ __forceinline__ bool slot_hits(const Slot& s, int z, int chunk, float& wz, float& dwz) {
  const int z0 = slot_z0(s);
  if (slot_chunk(s) != chunk) return false;
  if (z0 == z) {
    wz = 1.0f - s.fz;
    dwz = -1.0f;
    return true;
  }
  if (slot_hz(s) && z0 + 1 == z) {
    wz = s.fz;
    dwz = 1.0f;
    return true;
  }
  return false;
}

// Table values at the slot's 4 (y, x) corners of the current plane.
__device__ __forceinline__ void corners4(const Slot& s, const float* row, float& t00, float& t01,
                                         float& t10, float& t11) {
  const int base = s.idx & 0x1ff, dy = (s.idx >> 9) & 0x1f, dx = (s.idx >> 14) & 1;
  t00 = row[base];
  t01 = row[base + dx];
  t10 = row[base + dy];
  t11 = row[base + dy + dx];
}

// 8 fp32 table entries -> bf16x8 MFMA operand (round to nearest even).
__device__ __forceinline__ bf16x8_t to_bf16x8(const float* p) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2_t f = {p[2 * i], p[2 * i + 1]};
    r[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
  }
  return __builtin_bit_cast(bf16x8_t, r);
}

// Same, split into hi + lo bf16 parts (value = hi + lo to ~2^-16 relative).
__device__ __forceinline__ void to_bf16x8_hilo(const float* p, bf16x8_t& hi, bf16x8_t& lo) {
  u32x4_t h, l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2_t f = {p[2 * i], p[2 * i + 1]};
    const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
    const f32x2_t back = {__uint_as_float(hb << 16), __uint_as_float(hb & 0xffff0000u)};
    const f32x2_t rem = f - back;
    h[i] = hb;
    l[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(rem, bf16x2_t));
  }
  hi = __builtin_bit_cast(bf16x8_t, h);
  lo = __builtin_bit_cast(bf16x8_t, l);
}

}  // namespace tiled
}  // namespace msd
