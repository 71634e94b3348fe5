// Shared building blocks of the matrix-core (tiled) 3D-DSA kernels.
//
// A workgroup of 8 waves owns one (batch, head, tile of FRAMES consecutive
// frames x 4 rows x 4 columns of queries).  Thread i serves group query
// q = i / SUBS (frame q / 16 of the tile, position q % 16) and the taps
// kappa = (i % SUBS) + SUBS * j, j < SLOTS.  The forward and the first backward
// kernel use FRAMES = 1, SUBS = 32, SLOTS = 5; the dK/dV/dq kernel FRAMES = 2,
// SUBS = 16, SLOTS = 10.  Every tap's 2x2 (y, x) corner
// footprint is resolved against per-plane score tables
//   S[q][v] = X[q] . Y[v]   (X = q or dO rows, Y = K or V rows; MFMA, fp32 in LDS)
// built over the (y, x) bounding box of all corners of the tile, cut into
// 16 x 16 chunks whose starts are 15 voxels apart: two adjacent voxels always
// share a chunk, so each tap is assigned to exactly one chunk.
#pragma once

#include "common.h"
#include "div_rn.h"
#include "dsa3d_coords.h"

namespace msd {
namespace tiled {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
typedef __attribute__((ext_vector_type(8))) float f32x8_t;

constexpr int kTileH = 4, kTileW = 4;
constexpr int kTQ = kTileH * kTileW;    // queries per tile
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kSubs = 32;               // lanes per query (single-frame kernels)
constexpr int kSlots = 5;               // taps per lane: windows of <= kSubs * kSlots taps
constexpr int kMaxTaps = kSubs * kSlots;
constexpr int kChunk = 16;              // chunk edge in y and x
constexpr int kChunkStep = 15;          // chunk start spacing (one voxel of overlap)
constexpr int kChunkNV = kChunk * kChunk;
constexpr int kMaxChunks = 1 << 16;     // chunk ids are kept in 16 bits
// fp32 row stride of the tables: 260 words.  The four row groups an MFMA result
// writes (rows r, r+4, r+8, r+12; 4-byte stores over 32 banks per half-wave)
// fall on distinct banks.  The operand reads (16 rows, two 16-byte reads per
// lane; 64 banks in four 16-lane passes) are 2-way conflicted in each pass, and
// no stride or row order avoids that without conflicting the result writes.
constexpr int kSRow = kChunkNV + 4;
constexpr int kVRow = kChunkNV + 8;     // bf16 row stride of a transposed K/V chunk

// Matrix-core operands per element type.  A lane's operand of one k block is
// 8 consecutive k (channels or voxels) of its row or column.  bf16 feeds one
// 16x16x32 (32x32x16) MFMA with them; fp32 feeds eight 16x16x4 (32x32x2)
// MFMAs, the j-th taking element j of every lane, so each output sums the same
// products with fp32 operands and the register layouts stay the same.
template <typename E>
struct ElemT;
template <>
struct ElemT<bf16> {
  using op = bf16x8_t;
  using word = uint16_t;                // LDS element of a transposed chunk
  static constexpr int kRow = kVRow;    // its row stride (elements)
};
template <>
struct ElemT<float> {
  using op = f32x8_t;
  using word = float;
  static constexpr int kRow = kSRow;    // 260 words, as the tables
};
template <typename E>
using op_t = typename ElemT<E>::op;
template <typename E>
using word_t = typename ElemT<E>::word;

template <typename E>
__device__ __forceinline__ op_t<E> zero_op() {
  if constexpr (sizeof(E) == 2) {
    const u32x4_t z = {0u, 0u, 0u, 0u};
    return __builtin_bit_cast(bf16x8_t, z);
  } else {
    const f32x8_t z = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    return z;
  }
}

// Bytes of one dK / dV accumulator element of the tiled backward: fp16 for
// bf16 storage (scaled per call, packed-pair atomics), fp32 otherwise.
template <typename E>
constexpr int acc_bytes() {
  return sizeof(E) == 2 ? 2 : 4;
}

// Largest |x| of an 8-element operand (a NaN element is passed over).
template <typename E>
__device__ __forceinline__ float max_abs_op(const op_t<E>& x) {
  float m = 0.0f;
  if constexpr (sizeof(E) == 2) {
    const u32x4_t b = __builtin_bit_cast(u32x4_t, x);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      m = fmaxf(m, fmaxf(fabsf(__uint_as_float(b[i] << 16)),
                         fabsf(__uint_as_float(b[i] & 0xffff0000u))));
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(x[j]));
  }
  return m;
}

// 8 consecutive elements (16 or 32 bytes) from global memory or LDS.
template <typename E, typename P>
__device__ __forceinline__ op_t<E> load_op(const P* p) {
  op_t<E> r;
  __builtin_memcpy(&r, p, sizeof(r));
  return r;
}

__device__ __forceinline__ f32x4_t mma16(const bf16x8_t& a, const bf16x8_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mma16(const f32x8_t& a, const f32x8_t& b, f32x4_t c) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
  return c;
}
__device__ __forceinline__ f32x16_t mma32(const bf16x8_t& a, const bf16x8_t& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mma32(const f32x8_t& a, const f32x8_t& b, f32x16_t c) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], c, 0, 0, 0);
  return c;
}

// Element storage of q/k/v/offsets and the outputs: bf16 or fp32 (type E of
// the kernels; every table, accumulator and reduction is fp32 or fixed point
// either way).
struct Args {
  const void* q;
  const void* k;
  const void* v;
  const void* off;
  int64_t qs, ks, vs;  // token strides of q, k, v
  int64_t N;
  int B, T, H, W, nh, kt, kh, kw, K, C;
  int tiles_h, tiles_w;
  int xcd_remap;       // tiles per XCD when tiles are spread XCD-contiguously, else 0
  int head0;           // head of blockIdx.y 0 (a launch over a group of heads)
  float offset_scale, softmax_scale;
  float div_x, div_y, div_z;     // divisors of offset slots 0, 1, 2 (0 = slot dropped)
  float rdiv_x, rdiv_y, rdiv_z;  // their reciprocals, rounded to nearest (0 = slot dropped)
  float bdiv_x, bdiv_y, bdiv_z;  // base-grid divisors max(S-1, 1) of x (W), y (H), z (T)
  float rbdiv_x, rbdiv_y, rbdiv_z;
  float r_kw, r_khkw;            // 1/kw, 1/(kh*kw): exact small-integer division
  float gsx, gsy, gsz;           // d offset per d sampling coordinate: 0.5 S rdiv offset_scale
  DropoutArgs drop;              // attention dropout on the softmax weights
  float fix_a, fix_a_inv;        // fixed-point scale of the A (= p w) tables and its inverse
  const void* ek;                // extra keys / values [B, G, D] shared by every query
  const void* ev;                //   (attention.py:160-173), tap K + g of each query
  int G;                         // extra keys per sample (0 = none, at most kMaxExtra)
  float* dlt;                    // backward with extra keys: per (token, head) fp32 Delta,
                                 //   their part, then (first backward kernel) the whole
};

constexpr int kMaxExtra = 256;   // extra keys the tiled kernels take (a table row)

// Tap records of the first backward kernel for the column-streaming dq/dK/dV
// kernel (bf16 storage).  Per (head, one-frame tile): up to K * 16 records of
// 16 bytes, counting-sorted by the tap's lower corner plane z0 into kRecBins
// bins from the tile's lowest plane, and a header of kRecHdr ints:
//   [0..5] the tile's corner box zlo, zhi, ylo, yhi, xlo, xhi; [6] bins used
//   (0: no tap; -1: the planes span more than kRecBins bins, no records);
//   [8 + b] first record of bin b (b <= bins used: [8 + bins] = count).
// Record words: y0 | x0 << 14 | query << 28 (the tile's query 0..15); fx and
// fy as 16-bit fractions (lo, hi); fz (fp32 bits); the fp16 pair (p * dropout
// factor, ds * scale / l1) of the tap, l1 = sum over the query's taps of
// |ds * scale|.  Per (head, tile) too: q and dO of the tile's 16 queries,
// transposed ([tensor][channel][query], bf16), q times l1 / 2^30 and dO times
// 1 / fix_a: the scales of the B and A tables' fixed point.
constexpr int kRecBins = 16;
constexpr int kRecHdr = 32;
struct RecArgs {
  u32x4_t* rec;    // [nh][tiles][K * 16] records
  int* hdr;        // [nh][tiles][kRecHdr]
  void* qt;        // [nh][tiles][2][HD][16] element type
  int* collist;    // [0]: count, then head * columns + column of each column
                   // left to the tile kernel
  int64_t tiles;   // one-frame tiles per head
};

// Index of the one-frame tile (b, t, th, tw) among a head's tiles.
__device__ __forceinline__ int64_t rec_tile(const Args& a, int b, int t, int th, int tw) {
  return ((static_cast<int64_t>(b) * a.T + t) * a.tiles_h + th) * a.tiles_w + tw;
}

// Geometry of one tap, kept in registers between the passes.
struct Slot {
  int zc;    // z0 (bits 0-15, -1 = empty) | hz << 16 | clamp-gradient mask x,y,z << 17..19
             // | dropped by attention dropout << 20
  int idx;   // table index of corner (y0, x0) | dy_off << 9 | dx_off << 14 | chunk << 16
  float fz;  // weight of the upper z corner
  float fx, fy;  // weights of the upper x / y corners (0 when that corner is outside)
};

// The slot's words as opaque values at this point: keeps the compiler from
// hoisting what it derives from them (keys, corner weights and addresses) out
// of a plane loop, where registers are the limit.  Costs no instruction.
__device__ __forceinline__ Slot opaque(const Slot& s) {
  Slot r = s;
  asm volatile("" : "+v"(r.zc), "+v"(r.idx), "+v"(r.fz), "+v"(r.fx), "+v"(r.fy));
  return r;
}

__device__ __forceinline__ int slot_z0(const Slot& s) { return static_cast<int16_t>(s.zc & 0xffff); }
__device__ __forceinline__ bool slot_hz(const Slot& s) { return (s.zc >> 16) & 1; }
__device__ __forceinline__ int slot_chunk(const Slot& s) {
  return static_cast<int>(static_cast<uint32_t>(s.idx) >> 16);
}
// Dropout factor of the slot's softmax weight: 1 (off), 0 (dropped) or 1/(1-p).
__device__ __forceinline__ float slot_dropout(const Slot& s, const DropoutArgs& d) {
  return d.threshold == 0 ? 1.0f : (((s.zc >> 20) & 1) ? 0.0f : d.scale);
}

struct Tile {
  int b, head, t0, t, h0, w0;  // t0: first frame of the tile; t: this lane's frame
  int64_t sample0;
  int wave, lane, q, sub;      // q: group query of this lane (table column)
  int qh, qw;                  // this lane's query position
  bool q_ok;
  int64_t qn;  // token row of this lane's query
};

// Tiles of one launch: B x ceil(T / FRAMES) x tiles_h x tiles_w.
template <int FRAMES>
inline int64_t tile_count(int B, int T, int H, int W) {
  return static_cast<int64_t>(B) * ((T + FRAMES - 1) / FRAMES) * ((H + kTileH - 1) / kTileH) *
         ((W + kTileW - 1) / kTileW);
}

// Tile `tile` of head head0 + blockIdx.y.
template <int FRAMES, int SUBS>
__device__ __forceinline__ Tile make_tile_at(const Args& a, int tile) {
  Tile t;
  t.head = a.head0 + static_cast<int>(blockIdx.y);
  // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous run of tiles so neighbouring tiles share its L2.  Frames vary
  // fastest: consecutive tiles of one (h, w) column read and accumulate into
  // nearly the same K/V planes.
  if (a.xcd_remap > 0) tile = (tile & 7) * a.xcd_remap + (tile >> 3);
  const int groups = (a.T + FRAMES - 1) / FRAMES;
  t.t0 = (tile % groups) * FRAMES;
  tile /= groups;
  const int tw_i = tile % a.tiles_w;
  tile /= a.tiles_w;
  const int th_i = tile % a.tiles_h;
  t.b = tile / a.tiles_h;
  t.h0 = th_i * kTileH;
  t.w0 = tw_i * kTileW;
  t.sample0 = static_cast<int64_t>(t.b) * a.N;
  t.wave = threadIdx.x >> 6;
  t.lane = threadIdx.x & 63;
  t.q = threadIdx.x / SUBS;
  t.sub = threadIdx.x % SUBS;
  t.t = t.t0 + t.q / kTQ;
  const int s = t.q % kTQ;
  t.qh = t.h0 + s / kTileW;
  t.qw = t.w0 + s % kTileW;
  t.q_ok = t.t < a.T && t.qh < a.H && t.qw < a.W;
  t.qn = t.sample0 + (static_cast<int64_t>(t.t) * a.H + t.qh) * a.W + t.qw;
  return t;
}

template <int FRAMES, int SUBS>
__device__ __forceinline__ Tile make_tile(const Args& a) {
  return make_tile_at<FRAMES, SUBS>(a, blockIdx.x);
}

// Token row of group query m (frame m / 16, position m % 16), or -1 outside the grid.
__device__ __forceinline__ int64_t tile_row(const Args& a, const Tile& t, int m) {
  const int tt = t.t0 + m / kTQ, s = m % kTQ;
  const int h = t.h0 + s / kTileW, w = t.w0 + s % kTileW;
  if (tt >= a.T || h >= a.H || w >= a.W) return -1;
  return t.sample0 + (static_cast<int64_t>(tt) * a.H + h) * a.W + w;
}

// Two floats as an fp16 pair in one word (round to nearest), and back.
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(lo))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(hi))) << 16);
}
__device__ __forceinline__ float h2_lo(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
}
__device__ __forceinline__ float h2_hi(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

struct Box {
  int zlo, zhi, ylo, yhi, xlo, xhi;
  int ncy, ncx;  // chunk grid
};

// Offset-free base-grid coordinate 2*(p + c)/max(S-1, 1) - 1 (attention.py:228-230).
__device__ __forceinline__ float base_coord_rn(int p, int c, float bdiv, float rbdiv) {
#pragma clang fp contract(off)
  const float pos = static_cast<float>(p) + static_cast<float>(c);
  return div_rn(2.0f * pos, bdiv, rbdiv) - 1.0f;
}

__device__ __forceinline__ float grid_coord_rn(float base, float o, float div, float rdiv) {
#pragma clang fp contract(off)
  return div > 0.0f ? base + div_rn(o, div, rdiv) : base;
}

// Tap geometry for all SLOTS slots of this lane (coordinates exactly as the
// reference rounds them) and the block-wide bounding box of every corner.
// With `dropout`, each tap's keep decision is drawn here once (bit 20 of zc).
template <typename E, int SUBS, int SLOTS, int NW = kWaves>
__device__ __forceinline__ void setup_slots(const Args& a, const Tile& tl, Slot* sl, Box& box,
                                            int (*s_red)[6], bool dropout = false) {
  int zlo = 1 << 30, zhi = -1, ylo = 1 << 30, yhi = -1, xlo = 1 << 30, xhi = -1;
  int y0s[SLOTS], x0s[SLOTS];
  const int qh = tl.qh, qw = tl.qw;
  const int khkw = a.kh * a.kw;
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) {
    const int kap = tl.sub + SUBS * i;
    sl[i].zc = 0xffff;  // z0 = -1: empty
    sl[i].idx = 0;
    sl[i].fz = sl[i].fx = sl[i].fy = 0.0f;
    y0s[i] = x0s[i] = 0;
    if (!tl.q_ok || kap >= a.K) continue;
    // kap = (ci*kh + cj)*kw + ck; (kap + 0.5) * (1/d) truncates exactly for kap < 2^16
    const int ci_ = static_cast<int>((static_cast<float>(kap) + 0.5f) * a.r_khkw);
    const int rem = kap - ci_ * khkw;
    const int cj_ = static_cast<int>((static_cast<float>(rem) + 0.5f) * a.r_kw);
    const int ck_ = rem - cj_ * a.kw;
    const int ci = ci_ - a.kt / 2, cj = cj_ - a.kh / 2, ck = ck_ - a.kw / 2;
    const E* op = static_cast<const E*>(a.off) + tl.qn * a.C +
                  (static_cast<int64_t>(tl.head) * a.K + kap) * 3;
    const float o0 = to_f32(op[0]) * a.offset_scale;
    const float o1 = to_f32(op[1]) * a.offset_scale;
    const float o2 = to_f32(op[2]) * a.offset_scale;
    const Axis ax = axis_sample(grid_coord_rn(base_coord_rn(qw, ck, a.bdiv_x, a.rbdiv_x), o0,
                                              a.div_x, a.rdiv_x), a.W);
    const Axis ay = axis_sample(grid_coord_rn(base_coord_rn(qh, cj, a.bdiv_y, a.rbdiv_y), o1,
                                              a.div_y, a.rdiv_y), a.H);
    const Axis az = axis_sample(grid_coord_rn(base_coord_rn(tl.t, ci, a.bdiv_z, a.rbdiv_z), o2,
                                              a.div_z, a.rdiv_z), a.T);
    // clamp-gradient masks: zero where u <= 0 or u >= S-1 (grid_sample border padding)
    const int mx = (ax.u > 0.0f && ax.u < static_cast<float>(a.W - 1)) ? 1 : 0;
    const int my = (ay.u > 0.0f && ay.u < static_cast<float>(a.H - 1)) ? 1 : 0;
    const int mz = (az.u > 0.0f && az.u < static_cast<float>(a.T - 1)) ? 1 : 0;
    sl[i].zc = az.i0 | (az.hi_ok << 16) | (mx << 17) | (my << 18) | (mz << 19);
    if (dropout && a.drop.threshold != 0 && dropout_factor(a.drop, tl.qn, tl.head, kap) == 0.0f)
      sl[i].zc |= 1 << 20;
    // an upper corner outside the volume only occurs with weight 0 (the
    // coordinate is clamped to S-1), so fx/fy/fz are 0 there
    sl[i].fx = ax.f;
    sl[i].fy = ay.f;
    sl[i].fz = az.f;
    y0s[i] = ay.i0;
    x0s[i] = ax.i0;
    sl[i].idx = (ay.hi_ok ? 1 : 0) | (ax.hi_ok ? 2 : 0);  // flags until the chunk is known
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
  box.zlo = s_red[0][0];
  box.zhi = s_red[0][1];
  box.ylo = s_red[0][2];
  box.yhi = s_red[0][3];
  box.xlo = s_red[0][4];
  box.xhi = s_red[0][5];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    box.zlo = min(box.zlo, s_red[w][0]);
    box.zhi = max(box.zhi, s_red[w][1]);
    box.ylo = min(box.ylo, s_red[w][2]);
    box.yhi = max(box.yhi, s_red[w][3]);
    box.xlo = min(box.xlo, s_red[w][4]);
    box.xhi = max(box.xhi, s_red[w][5]);
  }
  // the same for every lane: keep it in scalar registers
  box.zlo = __builtin_amdgcn_readfirstlane(box.zlo);
  box.zhi = __builtin_amdgcn_readfirstlane(box.zhi);
  box.ylo = __builtin_amdgcn_readfirstlane(box.ylo);
  box.yhi = __builtin_amdgcn_readfirstlane(box.yhi);
  box.xlo = __builtin_amdgcn_readfirstlane(box.xlo);
  box.xhi = __builtin_amdgcn_readfirstlane(box.xhi);
  // chunk grid: starts lo, lo+15, ...; ceil((extent-1)/15) chunks (at least one)
  box.ncy = max(1, (box.yhi - box.ylo + kChunkStep - 1) / kChunkStep);
  box.ncx = max(1, (box.xhi - box.xlo + kChunkStep - 1) / kChunkStep);
  // assign every tap to the chunk holding its whole 2x2 footprint
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) {
    if (slot_z0(sl[i]) < 0) continue;
    const bool hy = sl[i].idx & 1, hx = sl[i].idx & 2;
    const int cy = min((y0s[i] - box.ylo) / kChunkStep, box.ncy - 1);
    const int cx = min((x0s[i] - box.xlo) / kChunkStep, box.ncx - 1);
    const int cy0 = box.ylo + kChunkStep * cy, cx0 = box.xlo + kChunkStep * cx;
    const int nx = min(kChunk, box.xhi - cx0 + 1);
    const int base = (y0s[i] - cy0) * nx + (x0s[i] - cx0);
    sl[i].idx = base | ((hy ? nx : 0) << 9) | ((hx ? 1 : 0) << 14) | ((cy * box.ncx + cx) << 16);
  }
}

struct Chunk {
  int id, cy0, cx0, ny, nx, nv, nvp;
  float rnx;  // 1/nx, for division-free voxel coordinates
};

// a / n for a wave-uniform n, skipping the (scalar, multi-instruction)
// division in the common case n == 1: the whole corner box fits one chunk.
__device__ __forceinline__ int uniform_div(int a, int n) {
  if (n == 1) return a;
  return a / n;
}

__device__ __forceinline__ Chunk make_chunk(const Box& box, int id) {
  Chunk c;
  c.id = id;
  const int cy = uniform_div(id, box.ncx), cx = id - cy * box.ncx;
  c.cy0 = box.ylo + kChunkStep * cy;
  c.cx0 = box.xlo + kChunkStep * cx;
  c.ny = min(kChunk, box.yhi - c.cy0 + 1);
  c.nx = min(kChunk, box.xhi - c.cx0 + 1);
  c.nv = c.ny * c.nx;
  c.nvp = (c.nv + 31) & ~31;
  // hardware reciprocal (1 ulp): (vi + 0.5) / nx is at least 1/32 away from an
  // integer for vi < 256, nx <= 16, so the truncation below stays exact
  c.rnx = __builtin_amdgcn_rcpf(static_cast<float>(c.nx));
  return c;
}

// Walk over the (plane, chunk) pairs of a box, chunk-major: every plane of
// chunk 0, then of chunk 1, ...  A tap's corners lie in one chunk and its two
// planes are consecutive steps, and the chunk geometry is rebuilt only when the
// walk moves to the next chunk (usually never: most boxes are one chunk).
struct Walk {
  Chunk c;
  int z;
};

__device__ __forceinline__ Walk walk_begin(const Box& box) {
  Walk w;
  w.c = make_chunk(box, 0);
  w.z = box.zlo;
  return w;
}

__device__ __forceinline__ Walk walk_next(const Box& box, const Walk& w) {
  Walk n = w;
  if (w.z < box.zhi) {
    n.z = w.z + 1;
  } else {
    n.c = make_chunk(box, w.c.id + 1);
    n.z = box.zlo;
  }
  return n;
}

// Token row of voxel vi (< nv) of chunk c in plane z.
__device__ __forceinline__ int64_t chunk_row(const Args& a, const Tile& tl, const Chunk& c, int z,
                                             int vi) {
  const int vy = static_cast<int>((static_cast<float>(vi) + 0.5f) * c.rnx);
  const int vx = vi - vy * c.nx;
  return tl.sample0 + (static_cast<int64_t>(z) * a.H + c.cy0 + vy) * a.W + c.cx0 + vx;
}

// Rows of `stride` elements are addressed as a wave-uniform 64-bit base (the
// chunk's first voxel, channel `col`) plus a 32-bit per-lane byte offset, so
// loads use scalar-base addressing; the base is computed once per step.  The
// host only admits shapes where (kChunk + 1) * W rows of every operand span
// less than 2^31 bytes and strides are below 2^23 elements.
template <typename E>
__device__ __forceinline__ const char* chunk_origin(const Args& a, const Tile& tl, const Chunk& c,
                                                    int z, const E* base, int64_t stride, int col) {
  const int64_t origin = tl.sample0 + (static_cast<int64_t>(z) * a.H + c.cy0) * a.W + c.cx0;
  return reinterpret_cast<const char*>(base + origin * stride + col);
}

// Channel `lane_col` (per lane, relative to the origin's) of voxel vi.
template <typename E>
__device__ __forceinline__ const E* chunk_voxel(const char* origin, const Args& a, const Chunk& c,
                                                int64_t stride, int lane_col, int vi) {
  const int vy = static_cast<int>((static_cast<float>(vi) + 0.5f) * c.rnx);
  const uint32_t vrow = static_cast<uint32_t>(__umul24(vy, a.W)) +
                        static_cast<uint32_t>(vi - vy * c.nx);
  const uint32_t bytes =
      static_cast<uint32_t>(__umul24(vrow, static_cast<uint32_t>(stride) *
                                               static_cast<uint32_t>(sizeof(E)))) +
      static_cast<uint32_t>(lane_col) * static_cast<uint32_t>(sizeof(E));
  return reinterpret_cast<const E*>(origin + bytes);
}

__device__ __forceinline__ u32x4_t load16(const void* p) {
  u32x4_t r;
  __builtin_memcpy(&r, p, sizeof(r));
  return r;
}

// Rows of the tile (queries m = lane % 16) as MFMA A operands: x[c] holds
// channels 32*c + 8*(lane/16) + [0, 8), c < HD/32.
template <int HD, typename E>
__device__ __forceinline__ void load_rows_operand(const Args& a, const Tile& tl, const E* base,
                                                  int64_t stride, op_t<E> (&x)[HD / 32]) {
#pragma unroll
  for (int c = 0; c < HD / 32; ++c) x[c] = zero_op<E>();
  const int64_t row = tile_row(a, tl, tl.lane & 15);
  if (row < 0) return;
  const E* p = base + row * stride + tl.head * HD + 8 * (tl.lane >> 4);
#pragma unroll
  for (int c = 0; c < HD / 32; ++c) x[c] = load_op<E>(p + 32 * c);
}

// Y rows of 16-voxel block j (< 2) of this wave (block w + 8 j; a chunk has at
// most 16 blocks) as MFMA B operands: y[c] holds channels 32*c + 8*(lane/16)
// + [0, 8) of voxel 16*block + lane % 16.
template <int HD, typename E>
__device__ __forceinline__ void load_block_rows(const Args& a, const Tile& tl, const Chunk& c,
                                                const char* origin, int64_t ystride, int j,
                                                op_t<E> (&y)[HD / 32]) {
  const int vi = (tl.wave + kWaves * j) * 16 + (tl.lane & 15);
#pragma unroll
  for (int cc = 0; cc < HD / 32; ++cc) y[cc] = zero_op<E>();
  if (vi < c.nv) {
    const E* p = chunk_voxel<E>(origin, a, c, ystride, 8 * (tl.lane >> 4), vi);
#pragma unroll
    for (int cc = 0; cc < HD / 32; ++cc) y[cc] = load_op<E>(p + 32 * cc);
  }
}

// The chunk's rows of head tl.head in plane z (wave-uniform origin).
template <int HD, typename E>
__device__ __forceinline__ const char* head_origin(const Args& a, const Tile& tl, const Chunk& c,
                                                   int z, const E* ybase, int64_t ystride) {
  return chunk_origin(a, tl, c, z, ybase, ystride, tl.head * HD);
}

// table[m][vi] = X[m] . Y[vi] for the voxels vi of block j of this wave.
template <int HD, typename E>
__device__ __forceinline__ void store_table_block(const Tile& tl, const Chunk& c,
                                                  const op_t<E> (&x)[HD / 32],
                                                  const op_t<E> (&y)[HD / 32], int j,
                                                  float* table) {
  const int blk = tl.wave + kWaves * j;
  if (blk * 16 >= c.nv) return;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int cc = 0; cc < HD / 32; ++cc) acc = mma16(x[cc], y[cc], acc);
  const int vi = blk * 16 + (tl.lane & 15);
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) table[(4 * (tl.lane >> 4) + rr) * kSRow + vi] = acc[rr];
}

// Both blocks of the wave, loaded together: all loads are issued before any
// is used.
template <int HD, typename E>
struct TableRows {
  op_t<E> y[2][HD / 32];  // [block][channels 32*c + kq]
};

template <int HD, typename E>
__device__ __forceinline__ void load_table_rows(const Args& a, const Tile& tl, const Chunk& c,
                                                int z, const E* ybase, int64_t ystride,
                                                TableRows<HD, E>& r) {
  const char* origin = head_origin<HD, E>(a, tl, c, z, ybase, ystride);
#pragma unroll
  for (int j = 0; j < 2; ++j) load_block_rows<HD, E>(a, tl, c, origin, ystride, j, r.y[j]);
}

template <int HD, typename E>
__device__ __forceinline__ void store_table(const Tile& tl, const Chunk& c,
                                            const op_t<E> (&x)[HD / 32], const TableRows<HD, E>& r,
                                            float* table) {
#pragma unroll
  for (int j = 0; j < 2; ++j) store_table_block<HD, E>(tl, c, x, r.y[j], j, table);
}

// Chunk rows of Y (plane z), channels col0 + [0, CW), transposed into LDS:
// yt[channel][voxel] (row stride ElemT<E>::kRow), padded up to nvp voxels
// with zeros or, with kPadCopies, copies of voxel nv - 1 (loads of every
// lane, no zeroing; the tables hold 0 for those voxels: 3% faster in the
// forward, 2-3% slower in the dq/dK/dV kernel), by the first NT = 512 threads
// of the workgroup.  Thread t moves
// voxels 2 p + {0, 1} of channel groups q0 + 4 g (8 channels each, g < CW /
// 32), p = 16 (t >> 6) + (t & 15), q0 = (t >> 4) & 3: a wave's lanes cover 4
// adjacent channel groups of 16 voxel pairs, so a load touches 16 rows, 32
// channels of each (64 rows of 8 channels took 4% longer in the forward, 32
// rows of 16 channels 1.5%).  Its loads are issued first.
//
// LDS banks, as measured on gfx950: a 4-byte access is served per half-wave
// over 32 banks of 4 bytes; a 16-byte read over 64 banks in four passes of 16
// lanes, pass (l >> 5, parity of the bits of (l >> 2) & 7).  In the plain bf16
// layout (rows of 132 words) the two channel groups of a half-wave write the
// same 16 banks (2-way), and the MFMA operand read (lane 16 g + m: row m, 8
// voxels from 8 g) meets 2-way conflicts in every pass.  The swizzled layout
// (kSwz, rows of kVRowSwz elements = 136 words) keeps voxel v of channel ch at
// column v ^ vt_swz(ch), 32 columns apart when bit 2 ^ bit 3 of ch is set:
// both access patterns are then conflict-free.  Readers XOR their k offset the
// same way (a k block of 32 voxels maps onto a k block).
template <int NT, int CW, typename E>
struct StageRows {
  static_assert(NT == 512, "the staging map covers 128 voxel pairs x 4 groups per pass");
  static constexpr int G = CW / 32;
  static_assert(G * 32 == CW, "channel groups must split evenly over the staging threads");
  op_t<E> x[G][2];  // [channel group][voxel]
};

// The thread index is read opaquely, so the map is recomputed where used
// rather than kept live across a plane loop (where the dq/dK/dV kernel would
// spill it, and every spill reload waits for the outstanding atomics).
__device__ __forceinline__ int stage_tid() {
  int t = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int stage_pair() {
  const int t = stage_tid();
  return 16 * ((t >> 6) & 7) + (t & 15);
}
__device__ __forceinline__ int stage_group0() {
  return (stage_tid() >> 4) & 3;
}

template <int NT, int CW, typename E, bool kPadCopies = false>
__device__ __forceinline__ void load_stage_rows(const Args& a, const Tile& tl, const Chunk& c,
                                                int z, const E* ybase, int64_t ystride,
                                                int col0, StageRows<NT, CW, E>& r) {
  constexpr int G = StageRows<NT, CW, E>::G;
  const int q0 = stage_group0(), v0 = 2 * stage_pair();
  if constexpr (kPadCopies) {
    // threads past NT (a larger workgroup) or past the padded chunk do not
    // stage (store_stage skips them too)
    if (threadIdx.x >= NT || v0 >= c.nvp) return;
    const char* origin = chunk_origin(a, tl, c, z, ybase, ystride, col0);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const E* p = chunk_voxel<E>(origin, a, c, ystride, 8 * q0, min(v0 + e, c.nv - 1));
#pragma unroll
      for (int g = 0; g < G; ++g) r.x[g][e] = load_op<E>(p + 32 * g);
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) r.x[g][0] = r.x[g][1] = zero_op<E>();
    if (threadIdx.x >= NT) return;  // a larger workgroup: the other threads do not stage
    const char* origin = chunk_origin(a, tl, c, z, ybase, ystride, col0);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      if (v0 + e < c.nv) {
        const E* p = chunk_voxel<E>(origin, a, c, ystride, 8 * q0, v0 + e);
#pragma unroll
        for (int g = 0; g < G; ++g) r.x[g][e] = load_op<E>(p + 32 * g);
      }
    }
  }
}

// Row stride (elements) and column swizzle of the swizzled bf16 layout.
constexpr int kVRowSwz = 272;
__device__ __forceinline__ int vt_swz(int ch) {
  return 32 * (((ch >> 2) ^ (ch >> 3)) & 1);
}

template <int NT, int CW, typename E, bool kSwz = false>
__device__ __forceinline__ void store_stage(const Chunk& c, const StageRows<NT, CW, E>& r,
                                            word_t<E>* yt) {
  constexpr int G = StageRows<NT, CW, E>::G;
  static_assert(!kSwz || sizeof(E) == 2, "the swizzled layout is the bf16 one");
  constexpr int R = kSwz ? kVRowSwz : ElemT<E>::kRow;
  const int q0 = stage_group0(), v0 = 2 * stage_pair();
  if (threadIdx.x >= NT || v0 >= c.nvp) return;
  // channels 8 (q0 + 4 g) + 2 i (+1): bit 3 is bit 0 of q0, bit 2 is bit 1 of i
  const int vs_lo = kSwz ? v0 ^ vt_swz(8 * q0) : v0;
  const int vs_hi = kSwz ? v0 ^ vt_swz(8 * q0 + 4) : v0;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int ch0 = 8 * (q0 + 4 * g);
    if constexpr (sizeof(E) == 2) {
      const u32x4_t x0 = __builtin_bit_cast(u32x4_t, r.x[g][0]);
      const u32x4_t x1 = __builtin_bit_cast(u32x4_t, r.x[g][1]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // even: the low halves of both voxels, odd: the high halves (v_perm_b32)
        const uint32_t even = __builtin_amdgcn_perm(x1[i], x0[i], 0x05040100u);
        const uint32_t odd = __builtin_amdgcn_perm(x1[i], x0[i], 0x07060302u);
        const int vs = i < 2 ? vs_lo : vs_hi;
        __builtin_memcpy(&yt[(ch0 + 2 * i) * R + vs], &even, sizeof(even));
        __builtin_memcpy(&yt[(ch0 + 2 * i + 1) * R + vs], &odd, sizeof(odd));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const f32x2_t pr = {r.x[g][0][i], r.x[g][1][i]};
        __builtin_memcpy(&yt[(ch0 + i) * R + v0], &pr, sizeof(pr));
      }
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

// Step key of (chunk, plane z): chunk << 16 | z.  A slot's key is that of its
// lower plane z0 (an empty slot's z0 field 0xffff matches no plane), so the
// distance d = step key - slot key is 0 on the lower plane and 1 on the upper
// one (a tap's planes are consecutive steps of its chunk); one subtraction
// replaces the chunk and plane compares.
__device__ __forceinline__ uint32_t step_key(int chunk, int z) {
  return (static_cast<uint32_t>(chunk) << 16) | static_cast<uint32_t>(z);
}
__device__ __forceinline__ uint32_t slot_key(const Slot& s) {
  return (static_cast<uint32_t>(s.idx) & 0xffff0000u) | (static_cast<uint32_t>(s.zc) & 0xffffu);
}

// Does this slot have corners on the step's plane?  Returns the z weight.
__device__ __forceinline__ bool slot_hits(const Slot& s, uint32_t key, float& wz, float& dwz) {
  const uint32_t d = key - slot_key(s);
  if (d > static_cast<uint32_t>(slot_hz(s))) return false;
  wz = d == 0 ? 1.0f - s.fz : s.fz;
  dwz = d == 0 ? -1.0f : 1.0f;
  return true;
}

// Branch-free form of slot_hits: the z weight (0 when the slot has no corners
// on the step's plane), its z derivative sign (0 likewise) and the hit flag.
__device__ __forceinline__ bool slot_weight(const Slot& s, uint32_t key, float& wz, float& dwz) {
  const uint32_t d = key - slot_key(s);
  const bool hit = d <= static_cast<uint32_t>(slot_hz(s));
  wz = hit ? (d == 0 ? 1.0f - s.fz : s.fz) : 0.0f;
  dwz = hit ? (d == 0 ? -1.0f : 1.0f) : 0.0f;
  return hit;
}

// Table values at the slot's 4 (y, x) corners of the current plane.  An upper
// corner row outside the volume (dy = 0, weight fy = 0) reads the lower row
// again.  Each row's two x corners are one paired read of entries base and
// base + 1; for an upper x corner outside the volume (weight fx = 0) entry
// base + 1 belongs to another voxel, so its value is replaced by 0 (one
// select): grid_sample skips out-of-volume corners, and a non-finite score of
// that other voxel must not reach this tap as 0 * inf.  Every index is at most
// kChunkNV, inside a table row even for a slot of another chunk (whose values
// are then discarded).
__device__ __forceinline__ void corners4(const Slot& s, const float* row, float& t00, float& t01,
                                         float& t10, float& t11) {
  const int base = s.idx & 0x1ff, dy = (s.idx >> 9) & 0x1f;
  const bool hx = (s.idx >> 14) & 1;
  t00 = row[base];
  const float r01 = row[base + 1];
  t10 = row[base + dy];
  const float r11 = row[base + dy + 1];
  t01 = hx ? r01 : 0.0f;
  t11 = hx ? r11 : 0.0f;
}

// Zeroes NB whole tables (pad columns included).
template <int NB>
__device__ __forceinline__ void zero_tables_all(float* tables) {
  constexpr int n4 = NB * kTQ * kSRow / 4;
  for (int e = threadIdx.x; e < n4; e += blockDim.x) {
    const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
    __builtin_memcpy(&tables[4 * e], &z, sizeof(z));
  }
}

// Bilinear (y, x) interpolation of 4 corner values and its two partial
// derivatives: val = lerp_y(top, bot), d/dfx and d/dfy.
struct Bilerp {
  float val, dx, dy;
};

__device__ __forceinline__ Bilerp bilerp(const Slot& s, float t00, float t01, float t10, float t11) {
  const float dtop = t01 - t00, dbot = t11 - t10;
  const float top = __builtin_fmaf(s.fx, dtop, t00);
  const float bot = __builtin_fmaf(s.fx, dbot, t10);
  Bilerp r;
  r.dy = bot - top;
  r.val = __builtin_fmaf(s.fy, r.dy, top);
  r.dx = __builtin_fmaf(s.fy, dbot - dtop, dtop);
  return r;
}

// Scatter tables (A = p w, B = ds scale w) accumulate in int32 fixed point:
// LDS integer atomics run ~30x faster than fp32 ones on gfx950, and integer
// sums are exact and order-independent.  A query's entries of A sum to at most
// sum_k p_k f_k, where f_k is the tap's dropout factor (1 without dropout; 0 or
// 1/(1-p) with it), i.e. to at most F = 1/(1-p).  A therefore uses the scale
// fix_a = 2^30 / 2^ceil(log2 F) (2^30 without dropout), which bounds every
// entry and partial sum by 2^30 and keeps the inverse scale a power of two.  B
// uses 2^30 / sum_k |ds_k scale| per query, which bounds every entry and every
// partial sum by 2^30.
constexpr float kFixA = 1073741824.0f;          // 2^30
constexpr float kFixAInv = 1.0f / 1073741824.0f;

// fix_a of a call with dropout factor `scale` (DropoutArgs::scale) when
// dropout is on.
inline float fix_a_scale(const DropoutArgs& d) {
  if (d.threshold == 0) return kFixA;
  int e = 0;
  const float m = std::frexp(d.scale, &e);  // scale = m 2^e, m in [0.5, 1)
  return std::ldexp(1.0f, 30 - (m == 0.5f ? e - 1 : e));
}

// Truncating conversion: one instruction; its error (< 2^-30 of the scale)
// is far below the rounding the tables get before the MFMA (bf16: 2^-9; fp32:
// 2^-24).
__device__ __forceinline__ int to_fix(float x) { return static_cast<int>(x); }

// 8 fixed-point table entries -> MFMA operand, still in fixed-point units: the
// power-of-two scale is taken off the MFMA result instead (exact).
template <typename E>
__device__ __forceinline__ op_t<E> fix_to_op(const int* p) {
  if constexpr (sizeof(E) == 2) {
    u32x4_t r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2_t f = {static_cast<float>(p[2 * i]), static_cast<float>(p[2 * i + 1])};
      r[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
    }
    return __builtin_bit_cast(bf16x8_t, r);
  } else {
    f32x8_t r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<float>(p[i]);
    return r;
  }
}

// 8 floats -> MFMA operand (rounded to bf16 for bf16 storage).
template <typename E>
__device__ __forceinline__ op_t<E> f32_to_op(const float* p) {
  if constexpr (sizeof(E) == 2) {
    u32x4_t r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2_t f = {p[2 * i], p[2 * i + 1]};
      r[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
    }
    return __builtin_bit_cast(bf16x8_t, r);
  } else {
    f32x8_t r;
    __builtin_memcpy(&r, p, sizeof(r));
    return r;
  }
}

// MFMA B operands of 16 extra-key rows (block eb of 16): y[c] holds channels
// 32 c + 8 (lane / 16) + [0, 8) of extra key 16 eb + lane % 16 of the tile's
// sample and head; rows past G are zero.
template <int HD, typename E>
__device__ __forceinline__ void load_extra_rows(const Args& a, const Tile& tl, const void* base,
                                                int eb, op_t<E> (&y)[HD / 32]) {
#pragma unroll
  for (int c = 0; c < HD / 32; ++c) y[c] = zero_op<E>();
  const int g = 16 * eb + (tl.lane & 15);
  if (g >= a.G) return;
  const int D = a.nh * HD;
  const E* p = static_cast<const E*>(base) + (static_cast<int64_t>(tl.b) * a.G + g) * D +
               tl.head * HD + 8 * (tl.lane >> 4);
#pragma unroll
  for (int c = 0; c < HD / 32; ++c) y[c] = load_op<E>(p + 32 * c);
}

// Extra-key rows (key or value) of the tile's head, channels [0, HD), keys
// g0 + [0, ng) transposed into yt[channel][g - g0] (row stride `row`
// elements), zero for keys past G: thread item e moves 8 channels of one key.
template <int HD, typename E>
__device__ __forceinline__ void stage_extra_t(const Args& a, const Tile& tl, const void* base,
                                              int g0, int ng, int row, word_t<E>* yt, int nthreads) {
  const int D = a.nh * HD;
  for (int e = threadIdx.x; e < ng * (HD / 8); e += nthreads) {
    const int gi = e / (HD / 8), cg = e % (HD / 8), g = g0 + gi;
    op_t<E> x = zero_op<E>();
    if (g < a.G)
      x = load_op<E>(static_cast<const E*>(base) + (static_cast<int64_t>(tl.b) * a.G + g) * D +
                     tl.head * HD + 8 * cg);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (sizeof(E) == 2) {
        const u32x4_t xb = __builtin_bit_cast(u32x4_t, x);
        yt[(8 * cg + i) * row + gi] =
            static_cast<uint16_t>((i & 1) ? (xb[i / 2] >> 16) : (xb[i / 2] & 0xffffu));
      } else {
        yt[(8 * cg + i) * row + gi] = x[i];
      }
    }
  }
}

// 8 floats as bf16x8, split into hi + lo bf16 parts (value = hi + lo to ~2^-16
// relative).
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

// A operand that must keep ~fp32 precision against a B operand of type E: the
// values themselves for fp32, a bf16 hi + lo pair (two MFMAs) for bf16.
template <typename E>
struct PreciseOp;
template <>
struct PreciseOp<bf16> {
  bf16x8_t hi, lo;
};
template <>
struct PreciseOp<float> {
  f32x8_t v;
};

template <typename E>
__device__ __forceinline__ PreciseOp<E> precise_op(const float (&p)[8]) {
  PreciseOp<E> r;
  if constexpr (sizeof(E) == 2) {
    to_bf16x8_hilo(p, r.hi, r.lo);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) r.v[i] = p[i];
  }
  return r;
}

__device__ __forceinline__ f32x4_t mma16(const PreciseOp<bf16>& a, const bf16x8_t& b, f32x4_t c) {
  return mma16(a.lo, b, mma16(a.hi, b, c));
}
__device__ __forceinline__ f32x4_t mma16(const PreciseOp<float>& a, const f32x8_t& b, f32x4_t c) {
  return mma16(a.v, b, c);
}

}  // namespace tiled
}  // namespace msd
