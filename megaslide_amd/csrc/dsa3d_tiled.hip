// Matrix-core (tiled) 3D-DSA forward and backward for gfx950: bf16 or fp32
// storage, fp32 accumulation, head_dim 32, 64, 96 or 128.
//
// One workgroup = one (batch, head, tile of 16 queries).  Instead of gathering
// the 8 corner rows of K and V for each of a query's taps, it builds dense
// tables on the matrix cores over the bounding box of the tile's corners, one
// z-plane (and 16x16 chunk) at a time:
//   pass 1:  S[q][v] = q . K[v]  (MFMA)  ->  per tap s = scale * sum_c w_c S[q][c]
//   softmax over each query's taps in registers (wave reductions)
//   pass 2:  A[q][v] = sum over taps/corners landing on v of p * w  (LDS atomics)
//            O[q] += A[q] . V  (MFMA, V chunk staged transposed in LDS)
// This equals the reference's grid_sample + matmul + softmax + matmul
// (infinity/video/attention.py:106-186) because trilinear sampling is linear in
// the sampled rows.  Coordinates and corner choice round exactly as the fp32
// reference does (div_rn, dsa3d_coords.h).
#include <algorithm>
#include <type_traits>

#include "dsa3d_tiled_common.h"

namespace msd {

namespace {

using namespace tiled;

// The S (pass 1) and A (pass 2) tables are double-buffered where that keeps
// the workgroups per CU: a step's table is written while the other buffer may
// still be read for the previous step, so pass 1 needs one barrier per step and
// pass 2 two (instead of two and three).  bf16 head_dim 96 keeps one buffer:
// two would drop it to one workgroup per CU (measured 30% slower).  bf16
// head_dim 128 without extra keys stages V^T in two 64-channel rounds per
// step, which leaves room for two workgroups per CU; with extra keys it, and
// every fp32 head, stages too much V^T for two and runs one, with the
// register cap raised to match.
constexpr int kLdsBytes = 160 * 1024;
constexpr int kTabBytes = kTQ * kSRow * 4;

template <int HD, typename E, bool XK>
constexpr bool fwd_half_v() {
  return !XK && ((sizeof(E) == 2 && HD == 128) || (sizeof(E) == 4 && HD == 64));
}

// bf16 V^T chunks take the swizzled (bank-conflict-free) layout.
template <typename E>
constexpr int fwd_vt_row() {
  return sizeof(E) == 2 ? kVRowSwz : ElemT<E>::kRow;
}

template <int HD, typename E, bool XK = false>
constexpr int fwd_vt_bytes() {
  return (fwd_half_v<HD, E, XK>() ? HD / 2 : HD) * fwd_vt_row<E>() *
         static_cast<int>(sizeof(word_t<E>));
}

template <int HD, typename E, bool XK = false>
constexpr int fwd_table_bufs() {
  constexpr int vt = fwd_vt_bytes<HD, E, XK>();
  if (2 * (2 * kTabBytes + vt) <= kLdsBytes) return 2;  // two workgroups per CU
  if (2 * (kTabBytes + vt) <= kLdsBytes) return 1;      // two workgroups per CU
  return 2 * kTabBytes + vt <= kLdsBytes ? 2 : 1;       // one workgroup per CU
}

// Minimum waves per SIMD: 4 when two 512-thread workgroups fit in a CU's LDS
// (bf16; the fp32 operands need more than 128 registers).
template <int HD, typename E, bool XK = false>
constexpr int fwd_min_waves() {
  if constexpr (sizeof(E) == 4 && !fwd_half_v<HD, E, XK>()) return 2;
  return 2 * (fwd_table_bufs<HD, E, XK>() * kTabBytes + fwd_vt_bytes<HD, E, XK>()) <= kLdsBytes
             ? 4
             : 2;
}

// Slot words as used in the forward's plane loops: at head_dim 96 (128
// registers at 4 waves/SIMD) opaque, which stops the hoisting that spilled
// (10% faster); elsewhere the hoisted keys and weights are cheaper (5%).
template <int HD>
__device__ __forceinline__ Slot fwd_slot(const Slot& s) {
  if constexpr (HD == 96) return opaque(s);
  return s;
}

// XK: the call has extra keys (a.G > 0); without them the kernel compiles to
// the plain tap path.
template <int HD, typename E, bool XK>
__global__ __launch_bounds__(kThreads, (fwd_min_waves<HD, E, XK>())) void dsa3d_fwd_tiled_kernel(
    Args a, E* __restrict__ out, float* __restrict__ lse) {
  constexpr int NB = fwd_table_bufs<HD, E, XK>();
  constexpr int VR = fwd_vt_row<E>();
  constexpr bool kHV = fwd_half_v<HD, E, XK>();  // V^T in two 64-channel rounds
  constexpr int VC = kHV ? HD / 2 : HD;           // V^T channels staged at once
  __shared__ __attribute__((aligned(16))) float s_tab[NB][kTQ * kSRow];  // S, then A
  __shared__ __attribute__((aligned(16))) word_t<E> s_vt[VC * VR];      // V^T chunk
  __shared__ int s_red[kWaves][6];
  // per query: 1, or NaN when a score is not finite (its output is NaN then, as
  // softmax makes it in the reference; the fixed-point weights alone would drop it)
  __shared__ float s_qnan[kTQ];

  const Tile tl = make_tile<1, kSubs>(a);
  // the tile's q rows load while the slots are set up
  op_t<E> qx[HD / 32];
  load_rows_operand<HD, E>(a, tl, static_cast<const E*>(a.q), a.qs, qx);
  // finite tables before the first step (the paired corner reads may read an
  // entry no step has written yet); the setup's barrier orders this before
  // the first table store
  zero_tables_all<NB>(&s_tab[0][0]);
  Slot sl[kSlots];
  Box box;
  setup_slots<E, kSubs, kSlots>(a, tl, sl, box, s_red, true);
  const int nchunks = box.ncy * box.ncx;
  const int nit = (box.zhi - box.zlo + 1) * nchunks;
  const E* const kp = static_cast<const E*>(a.k);
  const E* const vp = static_cast<const E*>(a.v);

  // ---- pass 1: scores -------------------------------------------------------
  // K rows of the next (plane, chunk) are loaded while the current one is used
  float sc[kSlots];
#pragma unroll
  for (int i = 0; i < kSlots; ++i) sc[i] = 0.0f;
  TableRows<HD, E> rows;
  Walk w = walk_begin(box);
  if (nit > 0) load_table_rows<HD, E>(a, tl, w.c, w.z, kp, a.ks, rows);
  for (int it = 0; it < nit; ++it) {
    const Walk wn = walk_next(box, w);
    const Chunk& c = w.c;
    const int z = w.z;
    // buffer it % NB was last read for step it - NB, before the previous barrier
    float* tab = s_tab[it % NB];
    store_table<HD, E>(tl, c, qx, rows, tab);
    if (it + 1 < nit) load_table_rows<HD, E>(a, tl, wn.c, wn.z, kp, a.ks, rows);
    __syncthreads();
    // only the lanes whose tap has corners on this step read them; a slot that
    // no lane of the wave hits (about a third of them) is skipped
    const float* my_row = &tab[tl.q * kSRow];
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const Slot si = fwd_slot<HD>(sl[i]);
      float wz, dwz;
      if (!slot_hits(si, step_key(c.id, z), wz, dwz)) continue;
      float t0, t1, t2, t3;
      corners4(si, my_row, t0, t1, t2, t3);
      sc[i] = __builtin_fmaf(wz, bilerp(si, t0, t1, t2, t3).val, sc[i]);
    }
    if constexpr (NB == 1) __syncthreads();  // the next step overwrites the table
    w = wn;
  }

  // ---- extra keys (attention.py:160-173): S_e[q][g] = q . ek_g (MFMA) into the
  // first table, read back by the lanes of each query: lane `sub` takes keys
  // sub + 32 j ------------------------------------------------------------------
  constexpr int EPL = XK ? kMaxExtra / kSubs : 1;
  const int G = XK ? a.G : 0, Gp = (G + 31) & ~31;
  float se[EPL];
  if constexpr (XK) {
    __syncthreads();  // every pass-1 read of the tables is done
    for (int eb = tl.wave; eb < Gp / 16; eb += kWaves) {
      op_t<E> y[HD / 32];
      load_extra_rows<HD, E>(a, tl, a.ek, eb, y);
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int cc = 0; cc < HD / 32; ++cc) acc = mma16(qx[cc], y[cc], acc);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        s_tab[0][(4 * (tl.lane >> 4) + rr) * kSRow + 16 * eb + (tl.lane & 15)] = acc[rr];
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int g = tl.sub + kSubs * j;
    se[j] = XK && g < G ? s_tab[0][tl.q * kSRow + g] * a.softmax_scale : -INFINITY;
  }

  // ---- softmax over each query's taps (32 lanes x kSlots) and extra keys ----
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    sc[i] = slot_z0(sl[i]) >= 0 ? sc[i] * a.softmax_scale : -INFINITY;
    mx = fmaxf(mx, sc[i]);
  }
  if constexpr (XK) {
#pragma unroll
    for (int j = 0; j < EPL; ++j) mx = fmaxf(mx, se[j]);
  }
#pragma unroll
  for (int m = 1; m < kSubs; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  float den = 0.0f;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    sc[i] = slot_z0(sl[i]) >= 0 ? __expf(sc[i] - mx) : 0.0f;
    den += sc[i];
  }
  if constexpr (XK) {
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      se[j] = tl.sub + kSubs * j < G ? __expf(se[j] - mx) : 0.0f;
      den += se[j];
    }
  }
#pragma unroll
  for (int m = 1; m < kSubs; m <<= 1) den += __shfl_xor(den, m);
  const float inv_den = 1.0f / den;
#pragma unroll
  for (int i = 0; i < kSlots; ++i)
    sc[i] *= inv_den * slot_dropout(sl[i], a.drop) * a.fix_a;  // p (dropped), fixed-point units
  {
    // the query index from the wave (a scalar) and the lane id: a per-lane
    // index kept across the plane loops spilled
    const unsigned tid = 64u * static_cast<unsigned>(__builtin_amdgcn_readfirstlane(tl.wave)) +
                         __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    if (tid % kSubs == 0) s_qnan[tid / kSubs] = den == den ? 1.0f : __builtin_nanf("");
  }
  if (lse != nullptr && tl.sub == 0 && !kHV) {
    if (tl.q_ok) lse[tl.qn * a.nh + tl.head] = mx + logf(den);
  } else if (lse != nullptr && tl.sub == 0) {
    // V^T in rounds (bf16 head_dim 128, fp32 64): the query's token row rebuilt
    // from the wave (a scalar) and the lane id (kept across the plane loop, it
    // spilled)
    const unsigned tid = 64u * static_cast<unsigned>(__builtin_amdgcn_readfirstlane(tl.wave)) +
                         __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int64_t qn = tile_row(a, tl, static_cast<int>(tid / kSubs));
    if (qn >= 0) lse[qn * a.nh + tl.head] = mx + logf(den);
  }

  // ---- output.  The waves form CG channel groups of KP waves; wave w of group
  // g takes the k-steps w % KP, + KP, ... of a table for the TPW channel tiles of
  // group g: one A operand feeds TPW independent MFMAs, and the KP partial O
  // are summed once at the end.  hd 64 and 128: one group of 8 waves (fp32
  // hd 128: two groups of 4, for registers).  hd 96: six single-tile groups
  // (waves 6, 7 idle), which stays within 128 registers and measured faster
  // than groups of several tiles.
  constexpr int CT = HD / 16, CG = HD == 96 ? CT : (sizeof(E) == 4 && HD == 128 ? 2 : 1);
  constexpr int TPW = CT / CG, KP = HD == 96 ? 1 : kWaves / CG;
  static_assert(TPW * CG == CT && CG * KP <= kWaves, "channel tiles split over the waves");
  const int mq = tl.lane & 15, kq = 8 * (tl.lane >> 4);
  // bf16 V^T chunks are stored swizzled (row 16 t + mq: channel bits 2, 3 = those of mq)
  constexpr bool kSwz = sizeof(E) == 2;
  const int sw = kSwz ? vt_swz(mq) : 0;
  const int cg = tl.wave / KP, kph = tl.wave % KP;
  const bool av_wave = tl.wave < CG * KP;
  f32x4_t oacc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) oacc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (XK) {
    // extra keys: O += P_e . EV with P_e = p f (fixed-point units, as floats)
    // in place of S_e (each entry is read and written by its own lane) and EV
    // staged transposed in the V^T buffer
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int g = tl.sub + kSubs * j;
      if (g < Gp)
        s_tab[0][tl.q * kSRow + g] =
            g < G ? se[j] * inv_den * a.fix_a *
                        (a.drop.threshold == 0
                             ? 1.0f
                             : dropout_factor(a.drop, tl.qn, tl.head, a.K + g))
                  : 0.0f;
    }
    stage_extra_t<HD, E>(a, tl, a.ev, 0, Gp, VR, s_vt, kThreads);
    __syncthreads();
    for (int kc = 32 * kph; av_wave && kc < Gp; kc += 32 * KP) {
      const op_t<E> av = f32_to_op<E>(&s_tab[0][mq * kSRow + kc + kq]);
#pragma unroll
      for (int t = 0; t < TPW; ++t)
        oacc[t] = mma16(av, load_op<E>(&s_vt[(16 * (cg * TPW + t) + mq) * VR + kc + kq]), oacc[t]);
    }
  }

  // ---- pass 2: O += A . V over the taps --------------------------------------
  if constexpr (kHV) {
    // channels [0, 64) then [64, 128) of each step's V^T through one buffer;
    // wave w takes channel tile w % 4 of each round and the k-steps w / 4,
    // + 2, ...; the two partial O are summed at the end
    constexpr int RT = VC / 16, KPH = kWaves / RT;
    const int tt = tl.wave % RT, kh2 = tl.wave / RT;
    f32x4_t oh[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
    StageRows<kThreads, VC, E> vh;
    w = walk_begin(box);
    if (nit > 0)
      load_stage_rows<kThreads, VC, E, true>(a, tl, w.c, w.z, vp, a.vs, tl.head * HD, vh);
    __syncthreads();  // pass-1 reads of both buffers are done
    zero_table(s_tab[0], kChunkNV);
    for (int it = 0; it < nit; ++it) {
      const Walk wn = walk_next(box, w);
      const Chunk& c = w.c;
      const int z = w.z;
      int* const s_atab = reinterpret_cast<int*>(s_tab[it % NB]);
      int* row = &s_atab[tl.q * kSRow];
      __syncthreads();  // the previous step's MFMAs are done with V^T; this buffer is zeroed
      store_stage<kThreads, VC, E, kSwz>(c, vh, s_vt);
      load_stage_rows<kThreads, VC, E, true>(a, tl, c, z, vp, a.vs, tl.head * HD + VC, vh);
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        const Slot si = fwd_slot<HD>(sl[i]);
        float wz, dwz;
        if (!slot_hits(si, step_key(c.id, z), wz, dwz)) continue;
        const float pz = sc[i] * wz;
        const float gx = 1.0f - si.fx, gy = 1.0f - si.fy;
        const int base = si.idx & 0x1ff, dy = (si.idx >> 9) & 0x1f;
        atomicAdd(&row[base], to_fix(pz * (gy * gx)));
        atomicAdd(&row[base + 1], to_fix(pz * (gy * si.fx)));
        atomicAdd(&row[base + dy], to_fix(pz * (si.fy * gx)));
        atomicAdd(&row[base + dy + 1], to_fix(pz * (si.fy * si.fx)));
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        if (r == 1) {
          __syncthreads();  // every wave is done with the first round's V^T
          store_stage<kThreads, VC, E, kSwz>(c, vh, s_vt);
          if (it + 1 < nit)
            load_stage_rows<kThreads, VC, E, true>(a, tl, wn.c, wn.z, vp, a.vs, tl.head * HD, vh);
          __syncthreads();
        }
        for (int kc = 32 * kh2; kc < c.nvp; kc += 32 * KPH) {
          const op_t<E> av = fix_to_op<E>(&s_atab[mq * kSRow + kc + kq]);
          oh[r] = mma16(av, load_op<E>(&s_vt[(16 * tt + mq) * VR + ((kc + kq) ^ sw)]), oh[r]);
        }
      }
      if constexpr (NB == 1) __syncthreads();
      if (it + 1 < nit) zero_table(s_tab[(it + 1) % NB], kChunkNV);
      w = wn;
    }
    __syncthreads();
    // oh[r][i] = partial O[query 4 (lane / 16) + i][channel 16 (4 r + tt) + lane % 16]
    // of k phase kh2, through the (free) V^T buffer: red[k phase][16][HD]
    float* red = reinterpret_cast<float*>(s_vt);
    static_assert(KPH * kTQ * HD * 4 <= fwd_vt_bytes<HD, E, XK>(), "partials fit the V^T buffer");
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[(kh2 * kTQ + 4 * (tl.lane >> 4) + i) * HD + 16 * (RT * r + tt) + mq] = oh[r][i];
    __syncthreads();
    for (int e = threadIdx.x; e < kTQ * HD; e += kThreads) {
      float o = 0.0f;
#pragma unroll
      for (int kp = 0; kp < KPH; ++kp) o += red[kp * kTQ * HD + e];
      const int m = e / HD, ch = e - m * HD;
      const int64_t n = tile_row(a, tl, m);
      if (n >= 0)
        out[n * (static_cast<int64_t>(a.nh) * HD) + tl.head * HD + ch] =
            from_f32<E>(o * a.fix_a_inv * s_qnan[m]);
    }
    return;
  }
  StageRows<kThreads, HD, E> vr;
  w = walk_begin(box);
  if (nit > 0) load_stage_rows<kThreads, HD, E, true>(a, tl, w.c, w.z, vp, a.vs, tl.head * HD, vr);
  __syncthreads();  // pass-1 reads of both buffers are done
  zero_table(s_tab[0], kChunkNV);
  for (int it = 0; it < nit; ++it) {
    const Walk wn = walk_next(box, w);
    const Chunk& c = w.c;
    const int z = w.z;
    // A in fixed point (scale fix_a), buffer it % NB: zeroed during the previous step
    int* const s_atab = reinterpret_cast<int*>(s_tab[it % NB]);
    int* row = &s_atab[tl.q * kSRow];
    __syncthreads();  // the previous step's MFMAs are done with V^T; this buffer is zeroed
    store_stage<kThreads, HD, E, kSwz>(c, vr, s_vt);
    if (it + 1 < nit)
      load_stage_rows<kThreads, HD, E, true>(a, tl, wn.c, wn.z, vp, a.vs, tl.head * HD, vr);
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const Slot si = fwd_slot<HD>(sl[i]);
      float wz, dwz;
      if (!slot_hits(si, step_key(c.id, z), wz, dwz)) continue;
      const float pz = sc[i] * wz;
      const float gx = 1.0f - si.fx, gy = 1.0f - si.fy;
      const int base = si.idx & 0x1ff, dy = (si.idx >> 9) & 0x1f;
      // an upper corner outside the volume has weight 0, so all four adds run
      // without branches: a y corner (offset 0) adds 0 to the lower one, an x
      // corner adds 0 to the next entry (at most column kChunkNV, inside the
      // row), and the x pair keeps one address with immediate offsets
      atomicAdd(&row[base], to_fix(pz * (gy * gx)));
      atomicAdd(&row[base + 1], to_fix(pz * (gy * si.fx)));
      atomicAdd(&row[base + dy], to_fix(pz * (si.fy * gx)));
      atomicAdd(&row[base + dy + 1], to_fix(pz * (si.fy * si.fx)));
    }
    __syncthreads();
    for (int kc = 32 * kph; av_wave && kc < c.nvp; kc += 32 * KP) {
      const op_t<E> av = fix_to_op<E>(&s_atab[mq * kSRow + kc + kq]);
#pragma unroll
      for (int t = 0; t < TPW; ++t)
        oacc[t] = mma16(av, load_op<E>(&s_vt[(16 * (cg * TPW + t) + mq) * VR + ((kc + kq) ^ sw)]),
                        oacc[t]);
    }
    // the next buffer was last read for step it + 1 - NB, before the barrier
    // above (with one buffer: this step, so wait for every wave's MFMAs first)
    if constexpr (NB == 1) __syncthreads();
    if (it + 1 < nit) zero_table(s_tab[(it + 1) % NB], kChunkNV);
    w = wn;
  }
  __syncthreads();
  // oacc[t][r] = wave partial of O[query 4*(lane/16) + r][channel 16*(cg*TPW +
  // t) + lane%16] in fixed-point units of A.  The V^T buffer (free after the
  // barrier above) takes the KP partials of every channel; every thread then
  // sums KP for its outputs, consecutive threads on consecutive channels.
  float* red = reinterpret_cast<float*>(s_vt);  // [k phase][16][HD]
  static_assert(kHV || KP * kTQ * HD * 4 <= fwd_vt_bytes<HD, E, XK>(),
                "partials fit the V^T buffer");
  if (av_wave) {
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[(kph * kTQ + 4 * (tl.lane >> 4) + r) * HD + 16 * (cg * TPW + t) + mq] = oacc[t][r];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kTQ * HD; e += kThreads) {
    float o = 0.0f;
#pragma unroll
    for (int kp = 0; kp < KP; ++kp) o += red[kp * kTQ * HD + e];
    const int m = e / HD, ch = e - m * HD;
    const int64_t n = tile_row(a, tl, m);
    if (n >= 0)
      out[n * (static_cast<int64_t>(a.nh) * HD) + tl.head * HD + ch] =
          from_f32<E>(o * a.fix_a_inv * s_qnan[m]);
  }
}

// 32 x 16 block vb of a transposed [voxel][query] fixed-point table (row stride
// `row`, queries from column col0) as the A operand of the 32x32 MFMA: lane l
// holds voxel 32*vb + l%32, queries col0 + 8*(l/32) + j, in fixed-point units
// (the per-query scales ride on the other operand).
template <typename E>
__device__ __forceinline__ op_t<E> table_t_rows(const int* table_t, int row, int col0, int vb,
                                                int lane) {
  return fix_to_op<E>(&table_t[(32 * vb + (lane & 31)) * row + col0 + 8 * (lane >> 5)]);
}

// Zero block after each first-backward table: covers a slot's largest corner
// index dy + dx = 32 (floats; a multiple of 4 keeps the next table 16-byte
// aligned).
constexpr int kP1Zero = 36;
constexpr int kP1Tab = kTQ * kSRow + kP1Zero;

// First backward kernel (one frame, 16 queries): pass 1 of the backward.  It
// rebuilds S and dP = dO V^T per plane, accumulates per tap s, dp and their
// coordinate derivatives, then writes the offset gradients and, for the second
// kernel, p times its dropout factor and ds * softmax_scale of every tap (fp32,
// [token][head][tap]).
// Waves per SIMD of the first backward kernel.  bf16 fits 128 registers, so
// two workgroups share a CU and each hides the other's latencies (barriers,
// table loads): q and dO then stay in LDS and K/V rows are loaded at the step
// (at head_dim 128 in two 64-channel halves per table block).  fp32 keeps q/dO
// in registers and prefetches the next step's rows, at one workgroup per CU.
template <int HD, typename E>
constexpr int p1_min_waves() {
  return sizeof(E) == 2 || HD == 64 ? 4 : 2;
}

// AE: bytes of one dK / dV accumulator element (4 = fp32 rows, 2 = scaled fp16).
// REC: also write the tap records, tile header and transposed q / dO of the
// column-streaming kernel (bf16 storage).
template <int HD, typename E, int AE, bool REC = false>
__global__ __launch_bounds__(kThreads, (p1_min_waves<HD, E>())) void dsa3d_bwd_p1_kernel(
    Args a, const E* __restrict__ out, const E* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ dlse, E* __restrict__ doff,
    float* __restrict__ p_ws, float* __restrict__ b_ws, void* __restrict__ dk_acc,
    void* __restrict__ dv_acc, int64_t acc_ks, int64_t acc_vs, RecArgs rc) {
  static_assert(!REC || (sizeof(E) == 2 && p1_min_waves<HD, E>() == 4),
                "records come from the bf16 kernel that stages q and dO in LDS");
  // S and dP tables, double-buffered (one barrier per plane).  A buffer is
  // [S rows | zeros | dP rows | zeros]: a slot that misses the step reads the
  // zero block instead of its corners, so its values are 0 with no select, and
  // dP sits a constant kP1Tab floats past S (immediate offsets on the reads).
  __shared__ __attribute__((aligned(16))) float s_tb[2][2 * kP1Tab];
  __shared__ int s_red[kWaves][6];
  // record bins (REC): counts, then starts
  __shared__ int s_bin[REC ? 2 * kRecBins : 1];
  if (REC && threadIdx.x < kRecBins) s_bin[threadIdx.x] = 0;  // ordered by the setup's barrier
  constexpr bool kTwoWg = p1_min_waves<HD, E>() == 4;
  // [query][channel] row of the staged q and dO (elements): HD / 2 + 8 words makes
  // the MFMA operand reads (lane l: query l % 16, 8 channels from 8 (l / 16))
  // bank-conflict-free on gfx950 (64 banks, 16-lane passes for 16-byte reads)
  constexpr int XR = HD + 16;
  __shared__ __attribute__((aligned(16))) word_t<E> s_x[kTwoWg ? 2 * kTQ * XR : 1];

  const Tile tl = make_tile<1, kSubs>(a);
  const int D = a.nh * HD;
  // The tile's q and dO rows (staged in LDS, or held as MFMA operands) are
  // loaded first, so that the slot setup's arithmetic covers their latency.
  constexpr int XCPR = HD * static_cast<int>(sizeof(E)) / 16;  // 16-byte pieces of a row
  constexpr int kXItems = 2 * kTQ * XCPR, kXIPT = kTwoWg ? (kXItems + kThreads - 1) / kThreads : 1;
  uint4 xst[kXIPT];
  op_t<E> qx[HD / 32], gx[HD / 32];
  if constexpr (kTwoWg) {
    // item e: q (t = 0) or dO (t = 1) row m, 16 bytes from channel ch
#pragma unroll
    for (int j = 0; j < kXIPT; ++j) {
      const int e = threadIdx.x + kThreads * j;
      const int t = e / (kTQ * XCPR), m = (e / XCPR) % kTQ, ch = (e % XCPR) * (16 / sizeof(E));
      const int64_t row = e < kXItems ? tile_row(a, tl, m) : -1;
      xst[j] = uint4{0u, 0u, 0u, 0u};
      if (row >= 0) {
        const E* src = t == 0 ? static_cast<const E*>(a.q) + row * a.qs : dout + row * D;
        xst[j] = *reinterpret_cast<const uint4*>(src + tl.head * HD + ch);
      }
    }
  } else {
    load_rows_operand<HD, E>(a, tl, static_cast<const E*>(a.q), a.qs, qx);
    load_rows_operand<HD, E>(a, tl, dout, D, gx);
  }
  Slot sl[kSlots];
  Box box;
  setup_slots<E, kSubs, kSlots>(a, tl, sl, box, s_red, true);
  const int nchunks = box.ncy * box.ncx;
  const int nit = (box.zhi - box.zlo + 1) * nchunks;
  const E* const kp = static_cast<const E*>(a.k);
  const E* const vp = static_cast<const E*>(a.v);
  for (int e = threadIdx.x; e < 2 * 2 * kP1Zero; e += kThreads)
    s_tb[e / (2 * kP1Zero)][((e / kP1Zero) & 1) * kP1Tab + kTQ * kSRow + e % kP1Zero] = 0.0f;
  {
    // The second kernel adds dK and dV into accumulator rows (the fp32 outputs
    // for fp32 storage, fp32 or scaled fp16 rows for bf16): zero this tile's
    // rows of the head first (the tiles of a launch partition the (token, head)
    // pairs, and the second kernel starts after this one ends), 16 bytes a thread.
    constexpr int CPR = HD * AE / 16;
    for (int e = threadIdx.x; e < 2 * kTQ * CPR; e += kThreads) {
      const int t = e / (kTQ * CPR), m = (e / CPR) % kTQ, ch = (e % CPR) * (16 / AE);
      const int64_t row = tile_row(a, tl, m);
      if (row < 0) continue;
      const int64_t el = row * (t == 0 ? acc_ks : acc_vs) + tl.head * HD + ch;
      char* dst = static_cast<char*>(t == 0 ? dk_acc : dv_acc) + el * AE;
      *reinterpret_cast<uint4*>(dst) = uint4{0u, 0u, 0u, 0u};
    }
  }

  if constexpr (kTwoWg) {
#pragma unroll
    for (int j = 0; j < kXIPT; ++j) {
      const int e = threadIdx.x + kThreads * j;
      if (e >= kXItems) continue;
      const int t = e / (kTQ * XCPR), m = (e / XCPR) % kTQ, ch = (e % XCPR) * (16 / sizeof(E));
      *reinterpret_cast<uint4*>(&s_x[(t * kTQ + m) * XR + ch]) = xst[j];
    }
    __syncthreads();
  }
  // MFMA A operand of staged row block t (q or dO): lane l holds channels
  // 32 c + 8 (l / 16) + [0, 8) of query l % 16
  auto staged_x = [&](int t, op_t<E> (&x)[HD / 32]) {
#pragma unroll
    for (int cc = 0; cc < HD / 32; ++cc)
      x[cc] = load_op<E>(&s_x[(t * kTQ + (tl.lane & 15)) * XR + 32 * cc + 8 * (tl.lane >> 4)]);
  };

  // Delta = dO . O - dlse and lse for this lane's query.  dO . O = sum_k p_k f_k
  // dP_k over the query's taps (formed in fp32 after the plane walk) plus, with
  // extra keys, the same sum over the keys (formed by their kernel before this
  // one): neither sees the rounding of the stored output (bf16 storage), which
  // a peaked softmax would otherwise turn into ds errors as large as ds itself.
  float delta = 0.0f, lse_q = 0.0f;
  if (tl.q_ok) {
    // with extra keys: their sum of p f dP (their kernel ran first)
    if (a.G > 0) delta = a.dlt[tl.qn * a.nh + tl.head];
    lse_q = lse[tl.qn * a.nh + tl.head];
  }
  if (dlse != nullptr && tl.q_ok) delta -= dlse[tl.qn * a.nh + tl.head];
  // kept in LDS across the plane loop (registers are the limit there)
  __shared__ float s_dl[kTQ][2];
  if (tl.sub == 0) {
    s_dl[tl.q][0] = delta;
    s_dl[tl.q][1] = lse_q;
  }

  // ---- pass 1: per tap, the interpolated S and dP and their coordinate
  // derivatives (x, y within a plane; z across planes) -------------------------
  float s_[kSlots], dp_[kSlots], gxs[kSlots], gxd[kSlots], gys[kSlots], gyd[kSlots], gzs[kSlots],
      gzd[kSlots];
#pragma unroll
  for (int i = 0; i < kSlots; ++i)
    s_[i] = dp_[i] = gxs[i] = gxd[i] = gys[i] = gyd[i] = gzs[i] = gzd[i] = 0.0f;
  // K and V rows of the next (plane, chunk) are loaded while the current one is
  // used.  fp32 rows beyond head_dim 64 would spill that way: they are loaded
  // at the step, one 16-voxel block at a time.
  constexpr bool kPrefetch = !kTwoWg && (sizeof(E) == 2 || HD == 64);
  TableRows<HD, E> rk, rv;
  Walk w = walk_begin(box);
  if (kPrefetch && nit > 0) {
    load_table_rows<HD, E>(a, tl, w.c, w.z, kp, a.ks, rk);
    load_table_rows<HD, E>(a, tl, w.c, w.z, vp, a.vs, rv);
  }
  for (int it = 0; it < nit; ++it) {
    const Walk wn = walk_next(box, w);
    const Chunk& c = w.c;
    const int z = w.z;
    // buffer it & 1 was last read for step it - 2, before the previous barrier
    float* const tb = s_tb[it & 1];
    if constexpr (kPrefetch) {
      store_table<HD, E>(tl, c, qx, rk, tb);
      store_table<HD, E>(tl, c, gx, rv, tb + kP1Tab);
      if (it + 1 < nit) {
        load_table_rows<HD, E>(a, tl, wn.c, wn.z, kp, a.ks, rk);
        load_table_rows<HD, E>(a, tl, wn.c, wn.z, vp, a.vs, rv);
      }
    } else {
      const char* ko = head_origin<HD, E>(a, tl, c, z, kp, a.ks);
      const char* vo = head_origin<HD, E>(a, tl, c, z, vp, a.vs);
#pragma nounroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (kTwoWg && HD * sizeof(E) == 256) {
          // S and dP of block j over two channel halves (bf16 head_dim 128,
          // fp32 64): a half's K/V rows and q/dO operands are HD / 64
          // operands each (registers are the limit)
          constexpr int OPH = HD / 64, CH = HD / 2;
          const int blk = tl.wave + kWaves * j;
          if (blk * 16 >= c.nv) continue;  // wave-uniform: no voxel of the block
          const int vi = blk * 16 + (tl.lane & 15);
          const bool v_ok = vi < c.nv;
          const int lc = 8 * (tl.lane >> 4);
          const E* const pk = chunk_voxel<E>(ko, a, c, a.ks, lc, v_ok ? vi : 0);
          const E* const pv = chunk_voxel<E>(vo, a, c, a.vs, lc, v_ok ? vi : 0);
          f32x4_t as = {0.0f, 0.0f, 0.0f, 0.0f}, ad = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            op_t<E> yk[OPH], yv[OPH];
#pragma unroll
            for (int cc = 0; cc < OPH; ++cc) {
              yk[cc] = yv[cc] = zero_op<E>();
              if (v_ok) {
                yk[cc] = load_op<E>(pk + CH * h + 32 * cc);
                yv[cc] = load_op<E>(pv + CH * h + 32 * cc);
              }
            }
            const word_t<E>* const xq = &s_x[(tl.lane & 15) * XR + CH * h + lc];
            const word_t<E>* const xo = xq + kTQ * XR;
#pragma unroll
            for (int cc = 0; cc < OPH; ++cc) {
              as = mma16(load_op<E>(xq + 32 * cc), yk[cc], as);
              ad = mma16(load_op<E>(xo + 32 * cc), yv[cc], ad);
            }
          }
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            tb[(4 * (tl.lane >> 4) + rr) * kSRow + vi] = as[rr];
            tb[kP1Tab + (4 * (tl.lane >> 4) + rr) * kSRow + vi] = ad[rr];
          }
          continue;
        }
        load_block_rows<HD, E>(a, tl, c, ko, a.ks, j, rk.y[0]);
        load_block_rows<HD, E>(a, tl, c, vo, a.vs, j, rv.y[0]);
        if constexpr (kTwoWg) {
          op_t<E> x[HD / 32];
          staged_x(0, x);
          store_table_block<HD, E>(tl, c, x, rk.y[0], j, tb);
          staged_x(1, x);
          store_table_block<HD, E>(tl, c, x, rv.y[0], j, tb + kP1Tab);
        } else {
          store_table_block<HD, E>(tl, c, qx, rk.y[0], j, tb);
          store_table_block<HD, E>(tl, c, gx, rv.y[0], j, tb + kP1Tab);
        }
      }
    }
    __syncthreads();
    // a hit reads its 4 corners in both tables; a miss reads the zero block
    // (never stale entries, which may be non-finite) and has wz = dwz = 0.  A
    // slot that no lane of the wave hits (about a third of them) is skipped.
    const float* const r0 = &tb[tl.q * kSRow];
    const float* const zr = &tb[kTQ * kSRow];
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      float wz, dwz;
      const bool hit = slot_weight(sl[i], step_key(c.id, z), wz, dwz);
      if (__builtin_amdgcn_ballot_w64(hit) == 0) continue;
      const int base = sl[i].idx & 0x1ff, dy = (sl[i].idx >> 9) & 0x1f, dx = (sl[i].idx >> 14) & 1;
      const float* const ps = hit ? r0 + base : zr;
      const float* const pd = ps + kP1Tab;
      const Bilerp bs = bilerp(sl[i], ps[0], ps[dx], ps[dy], ps[dy + dx]);
      const Bilerp bd = bilerp(sl[i], pd[0], pd[dx], pd[dy], pd[dy + dx]);
      s_[i] = __builtin_fmaf(wz, bs.val, s_[i]);
      gxs[i] = __builtin_fmaf(wz, bs.dx, gxs[i]);
      gys[i] = __builtin_fmaf(wz, bs.dy, gys[i]);
      gzs[i] = __builtin_fmaf(dwz, bs.val, gzs[i]);
      dp_[i] = __builtin_fmaf(wz, bd.val, dp_[i]);
      gxd[i] = __builtin_fmaf(wz, bd.dx, gxd[i]);
      gyd[i] = __builtin_fmaf(wz, bd.dy, gyd[i]);
      gzd[i] = __builtin_fmaf(dwz, bd.val, gzd[i]);
    }
    w = wn;
  }

  // p = exp(scale * s - lse), ds = p (dp - Delta).  The coordinate gradient of
  // a tap is ds*scale*dS/du + p*dP/du; chain it through the clamp mask, the
  // unnormalisation (S/2), the slot divisor and offset_scale into d offsets.
  const float cxs = a.gsx, cys = a.gsy, czs = a.gsz;
  // the query's token row and the taps' offsets are recomputed here from the
  // wave (a scalar) and the lane id: kept from before the plane loop, they
  // spill (as does the thread index register)
  const int tid = 64 * __builtin_amdgcn_readfirstlane(tl.wave) +
                  static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
  const int sub = tid % kSubs;
  const int64_t qn = tile_row(a, tl, tid / kSubs);
  const int64_t tap0 = (qn * a.nh + tl.head) * a.K;
  delta = s_dl[tid / kSubs][0];  // written before the loop's first barrier
  lse_q = s_dl[tid / kSubs][1];
  // p of every tap (0 for empty slots) in place of s.  Dropout: o sums
  // pd * v_s with pd = p * factor, so dp and the V-side coordinate gradient
  // see the factor.
  float pdp = 0.0f;  // sum_k p_k f_k dP_k over this lane's taps
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const bool ok = slot_z0(sl[i]) >= 0;
    s_[i] = ok ? __expf(s_[i] * a.softmax_scale - lse_q) : 0.0f;
    pdp = __builtin_fmaf(s_[i] * slot_dropout(sl[i], a.drop), dp_[i], pdp);
  }
#pragma unroll
  for (int m = 1; m < kSubs; m <<= 1) pdp += __shfl_xor(pdp, m);
  delta += pdp;
  // the whole Delta for the extra keys' kernel that runs next (each query's
  // entry is read above and written here by this workgroup only)
  if (a.G > 0 && sub == 0 && qn >= 0) a.dlt[qn * a.nh + tl.head] = delta;
  // p * factor in place of p, ds * scale = p (f dP - Delta) scale in place of dp
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const float dfac = slot_dropout(sl[i], a.drop);
    dp_[i] = s_[i] * (dfac * dp_[i] - delta) * a.softmax_scale;
    s_[i] *= dfac;
  }
  // bf16 storage keeps one word per tap: fp16 p * factor and ds * scale / l1,
  // with l1 = sum over the query's taps of |ds * scale| kept per token and head
  // (the normalised values lie in [-1, 1], where fp16 keeps 11 bits)
  float rl1 = 1.0f, l1q = 0.0f;
  if constexpr (sizeof(E) == 2) {
    float l1 = 0.0f;
#pragma unroll
    for (int i = 0; i < kSlots; ++i) l1 += fabsf(dp_[i]);
#pragma unroll
    for (int m = 1; m < kSubs; m <<= 1) l1 += __shfl_xor(l1, m);
    rl1 = l1 > 1e-30f ? 1.0f / l1 : 0.0f;
    l1q = l1;
    if (sub == 0 && qn >= 0) b_ws[qn * a.nh + tl.head] = l1;
  }
  // Records for the column-streaming kernel (REC), counting-sorted by z0: the
  // bins' counts by LDS atomics (their return values place each record in its
  // bin), then one thread's prefix sum.  Within a bin the order is the
  // atomics' order, which no result depends on (the consumer sums integers).
  int pos[kSlots];
  const bool rec_wide = REC && !(box.zhi < box.zlo) && box.zhi - box.zlo + 1 > kRecBins;
  if constexpr (REC) {
    const int64_t trec = static_cast<int64_t>(tl.head) * rc.tiles +
                         rec_tile(a, tl.b, tl.t0, tl.h0 / kTileH, tl.w0 / kTileW);
    // the column list's count and, after the list, the 8 work counters of the
    // column-streaming kernel
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 9)
      rc.collist[threadIdx.x == 0 ? 0 : a.nh * a.B * a.tiles_h * a.tiles_w + threadIdx.x] = 0;
    const int nb = box.zhi < box.zlo ? 0 : box.zhi - box.zlo + 1;
    if (sub == 0) s_dl[tid / kSubs][0] = l1q;  // this query's l1 (delta was read above)
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      pos[i] = 0;
      if (!rec_wide && slot_z0(sl[i]) >= 0)
        pos[i] = atomicAdd(&s_bin[slot_z0(sl[i]) - box.zlo], 1);
    }
    __syncthreads();
    // exclusive prefix of the 16 counts in wave 0 (lane bb holds bin bb)
    if (threadIdx.x < 64) {
      const int bb = threadIdx.x & (kRecBins - 1);
      const int cnt = threadIdx.x < kRecBins ? s_bin[bb] : 0;
      int inc = cnt;
#pragma unroll
      for (int m = 1; m < kRecBins; m <<= 1) {
        const int o = __shfl_up(inc, m, kRecBins);
        if (bb >= m) inc += o;
      }
      int* const hdr = rc.hdr + trec * kRecHdr;
      if (threadIdx.x < kRecBins) {
        s_bin[kRecBins + bb] = inc - cnt;
        hdr[8 + bb] = inc - cnt;
        if (bb == kRecBins - 1) hdr[8 + kRecBins] = inc;
      }
      if (threadIdx.x == 0) {
        hdr[0] = box.zlo;
        hdr[1] = box.zhi;
        hdr[2] = box.ylo;
        hdr[3] = box.yhi;
        hdr[4] = box.xlo;
        hdr[5] = box.xhi;
        hdr[6] = rec_wide ? -1 : nb;
      }
    }
    __syncthreads();
  }
  // a record's corner (y0, x0) from the tap's table index in its chunk of
  // the box; one chunk column (the usual case): the box's x origin and width
  const bool one_cx = box.ncx == 1;
  const int nx1 = min(kChunk, box.xhi - box.xlo + 1);
  const float rnx1 = __builtin_amdgcn_rcpf(static_cast<float>(nx1));
  u32x4_t* const rec = REC ? rc.rec + (static_cast<int64_t>(tl.head) * rc.tiles +
                                       rec_tile(a, tl.b, tl.t0, tl.h0 / kTileH, tl.w0 / kTileW)) *
                                          (static_cast<int64_t>(a.K) * kTQ)
                           : nullptr;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    if (slot_z0(sl[i]) < 0) continue;
    const float pd = s_[i], dss = dp_[i];
    const int kap = sub + kSubs * i;
    uint32_t pair = 0;
    if constexpr (sizeof(E) == 4) {
      p_ws[tap0 + kap] = pd;
      b_ws[tap0 + kap] = dss;
    } else {
      pair = pack_h2(pd, dss * rl1);
      reinterpret_cast<uint32_t*>(p_ws)[tap0 + kap] = pair;
    }
    E* dp = doff + qn * a.C + (static_cast<int64_t>(tl.head) * a.K + kap) * 3;
    const int m = sl[i].zc >> 17;
    dp[0] = from_f32<E>((m & 1) ? (dss * gxs[i] + pd * gxd[i]) * cxs : 0.0f);
    dp[1] = from_f32<E>((m & 2) ? (dss * gys[i] + pd * gyd[i]) * cys : 0.0f);
    dp[2] = from_f32<E>((m & 4) ? (dss * gzs[i] + pd * gzd[i]) * czs : 0.0f);
    if constexpr (REC) {
      if (rec_wide) continue;
      const int idx = sl[i].idx;
      const int base = idx & 0x1ff, ch = static_cast<int>(static_cast<uint32_t>(idx) >> 16);
      int cy = ch, cx0 = box.xlo, nx = nx1;
      float rnx = rnx1;
      if (!one_cx) {
        cy = ch / box.ncx;
        cx0 = box.xlo + kChunkStep * (ch - cy * box.ncx);
        nx = min(kChunk, box.xhi - cx0 + 1);
        rnx = __builtin_amdgcn_rcpf(static_cast<float>(nx));
      }
      const int vy = static_cast<int>((static_cast<float>(base) + 0.5f) * rnx);
      const int y0 = box.ylo + kChunkStep * cy + vy, x0 = cx0 + base - vy * nx;
      const uint32_t ux = min(65535u, static_cast<uint32_t>(sl[i].fx * 65536.0f + 0.5f));
      const uint32_t uy = min(65535u, static_cast<uint32_t>(sl[i].fy * 65536.0f + 0.5f));
      u32x4_t r;
      r[0] = static_cast<uint32_t>(y0) | (static_cast<uint32_t>(x0) << 14) |
             (static_cast<uint32_t>(tid / kSubs) << 28);
      r[1] = ux | (uy << 16);
      r[2] = __float_as_uint(sl[i].fz);
      r[3] = pair;
      rec[s_bin[kRecBins + slot_z0(sl[i]) - box.zlo] + pos[i]] = r;
    }
  }
  if constexpr (REC) {
    const int64_t trec = static_cast<int64_t>(tl.head) * rc.tiles +
                         rec_tile(a, tl.b, tl.t0, tl.h0 / kTileH, tl.w0 / kTileW);
    // q and dO of the tile transposed, with the fixed-point scales of the B
    // (l1 / 2^30, per query) and A (1 / fix_a) tables: item e = (tensor,
    // channel, query half) writes 8 queries (16 bytes)
    E* const qt = static_cast<E*>(rc.qt) + trec * (2 * HD * kTQ);
    for (int e = threadIdx.x; e < 2 * HD * 2; e += kThreads) {
      const int t = e / (2 * HD), chn = (e / 2) % HD, h8 = 8 * (e & 1);
      uint16_t v8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int m = h8 + j;
        const float sc = t == 0 ? s_dl[m][0] * kFixAInv : a.fix_a_inv;
        const uint16_t raw = s_x[(t * kTQ + m) * XR + chn];
        v8[j] = from_f32<E>(__uint_as_float(static_cast<uint32_t>(raw) << 16) * sc).bits;
      }
      __builtin_memcpy(&qt[(t * HD + chn) * kTQ + h8], v8, sizeof(v8));
    }
  }
}

// Second backward kernel: dq, dK and dV for tiles of FR consecutive frames
// (16 FR queries) of one 4x4 (h, w) column, over a window of CW of the
// head's HD channels (window blockIdx.z).  Consecutive frames reach nearly the
// same planes, so one flush of the [voxel][query] tables per plane serves all
// of them: the fp32 dK/dV atomics (executed past the L2, the backward's
// dominant cost) drop accordingly.  Tap geometry is recomputed from the
// offsets; p (with its dropout factor) and ds * scale come from the first
// kernel.  The A and B tables do not depend on the channel, so a window
// narrower than the head rebuilds them per window in exchange for fewer
// registers and less LDS.
template <int FR>
struct P2Tile {
  static constexpr int Q = kTQ * FR;              // queries per tile
  static constexpr int Waves = 4 * FR;            // 16 lanes per query
  static constexpr int Threads = 64 * Waves;
  static constexpr int Subs = Threads / Q;        // lanes per query
  static constexpr int Slots = kMaxTaps / Subs;   // taps per lane
  static constexpr int Row = Q + 2;               // [voxel][query] table row (ints)
  static_assert(Subs * Slots == kMaxTaps, "the tap capacity must match the first kernel");
};
constexpr int kP2Stage = 512;  // threads that stage the K^T chunk

// [channel][query] row of the staged q / dO (elements): 16 FR + 8 bf16 (16 FR + 4
// fp32, = 36 banks at FR 2: 16 rows of 16-byte reads conflict-free).
template <typename E, int FR>
constexpr int p2_qrow() {
  return sizeof(E) == 2 ? kTQ * FR + 8 : kTQ * FR + 4;
}

// Adds a 32-voxel x 32-channel block of dK or dV (a 32x32 MFMA result; lane l
// holds channel `ch` = window channel l % 32 and, in registers 4 g + i, voxel
// 32 vb + 8 g + 4 (l / 32) + i) into fp32 rows of `acc` (token stride
// `stride`) with global fp32 atomics (executed past the L2), so one register
// across the wave covers 2 voxels x 32 contiguous channels.  s_rows gives each
// voxel's token row within the sample; the host admits N * stride < 2^30, so
// every offset is a 32-bit lane offset from a wave-uniform base.  Untouched
// voxels (exact zeros) send nothing.  (Packed bf16 atomics into bf16 outputs
// would halve the bytes, but rounding the running sum to bf16 at every add
// loses the fp32 accuracy where many tiles add into one voxel, e.g. taps
// border-clamped onto the volume's edge.)
__device__ __forceinline__ void flush_block(const Tile& tl, const f32x16_t& x, const int* s_rows,
                                            int vb, int nv, int ch, float* acc, int64_t stride) {
  char* const base = reinterpret_cast<char*>(acc + tl.sample0 * stride);
  const uint32_t st = static_cast<uint32_t>(stride);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int v0 = 32 * vb + 8 * g + 4 * (tl.lane >> 5);
    int rr[4];
    __builtin_memcpy(rr, &s_rows[v0], sizeof(rr));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float val = x[4 * g + i];
      if (v0 + i < nv && val != 0.0f)
        atomicAdd(reinterpret_cast<float*>(base + (static_cast<uint32_t>(rr[i]) * st + ch) * 4u),
                  val);
    }
  }
}

// The same block into fp16 rows, times `scale` (a power of two), with packed
// two-channel atomics: lanes l and l ^ 1 hold adjacent channels of the same
// voxels, and one swap gives the even lane both channels of voxel i and the
// odd lane both of voxel i + 1, so one atomic carries two values (they run at
// the rate of one fp32 atomic; 16 lanes cover 64 contiguous bytes of a row).
// A sum beyond the fp16 range becomes infinite, which the conversion detects.
__device__ __forceinline__ void flush_block_h16(const Tile& tl, const f32x16_t& x,
                                                const int* s_rows, int vb, int nv, int ch,
                                                void* acc, int64_t stride, float scale) {
  typedef __attribute__((ext_vector_type(2))) _Float16 h2_t;
  char* const base = static_cast<char*>(acc) + tl.sample0 * stride * 2;
  const uint32_t st = static_cast<uint32_t>(stride);
  const uint32_t che = static_cast<uint32_t>(ch & ~1);
  const bool odd = tl.lane & 1;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int v0 = 32 * vb + 8 * g + 4 * (tl.lane >> 5);
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      const float a0 = x[4 * g + i] * scale, a1 = x[4 * g + i + 1] * scale;
      const float recv = __shfl_xor(odd ? a0 : a1, 1);
      const float lo = odd ? recv : a0, hi = odd ? a1 : recv;
      const int vi = v0 + i + (odd ? 1 : 0);
      if (vi < nv && (lo != 0.0f || hi != 0.0f)) {
        const h2_t pk = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
        __builtin_amdgcn_global_atomic_fadd_v2f16(
            reinterpret_cast<h2_t*>(base + (static_cast<uint32_t>(s_rows[vi]) * st + che) * 2u),
            pk);
      }
    }
  }
}

// Accumulation modes of the second backward kernel: fp32 atomics (fp32
// storage), scaled fp16 atomics (bf16 storage), and the fp32 redo of dK / dV
// alone after an fp16 overflow (dq is already final then).
enum P2Mode { kP2F32 = 0, kP2F16 = 1, kP2Redo = 2 };

template <int HD, int CW, typename E, int FR, int MODE>
__device__ __forceinline__ void p2_tile(const Args& a, int tile, const E* __restrict__ dout,
                                        const float* __restrict__ p_ws,
                                        const float* __restrict__ b_ws, E* __restrict__ dq,
                                        void* __restrict__ dk_acc, void* __restrict__ dv_acc,
                                        int64_t acc_ks, int64_t acc_vs, int cw_base,
                                        const float* __restrict__ scales,
                                        const float* __restrict__ dqx) {
  static_assert(CW <= HD && CW % 32 == 0, "channel windows are whole 32-channel blocks");
  using G = P2Tile<FR>;
  constexpr int kP2Frames = FR, kP2Q = G::Q, kP2Subs = G::Subs, kP2Slots = G::Slots;
  constexpr int kP2Row = G::Row, NW = G::Waves, NT = G::Threads;
  constexpr int KR = ElemT<E>::kRow, QR = p2_qrow<E, FR>();
  // A^T = p w and B^T = ds scale w (fixed point), one array: a B^T entry is its
  // A^T entry plus a constant, which the LDS instructions take as an offset
  constexpr int kTab = kChunkNV * kP2Row;
  __shared__ __attribute__((aligned(16))) int s_ab[2 * kTab];
  int* const s_at = s_ab;
  int* const s_bt = s_ab + kTab;
  // K^T chunk: a 96-channel window stages it in two rounds (64 + 32 channels)
  // through one 64-channel buffer, so the whole hd-96 head fits one window
  constexpr int KW = CW == 96 ? 64 : CW;  // channels of the first round
  __shared__ __attribute__((aligned(16))) word_t<E> s_kt[KW * KR];
  // per voxel: its token row within the sample
  __shared__ __attribute__((aligned(16))) int s_rows[kChunkNV];
  __shared__ int s_red[NW][6];
  __shared__ __attribute__((aligned(16))) float s_binv[kP2Q];  // per query: 1 / fixed-point scale of B
  // the tile's q and dO rows of this window, transposed: [tensor][channel][query]
  __shared__ __attribute__((aligned(16))) word_t<E> s_qt[2][CW][QR];

  const Tile tl = make_tile_at<kP2Frames, kP2Subs>(a, tile);
  const int D = a.nh * HD;
  // first channel of the window: cw_base + CW blockIdx.z within the head
  const int cw0 = tl.head * HD + cw_base + CW * static_cast<int>(blockIdx.z);
  // p and ds * scale of this lane's taps (from the first kernel) and the q / dO
  // items it stages are loaded before the slot setup, whose arithmetic then
  // covers their latency (one workgroup per CU: nothing else would)
  // (bf16 storage: fp16 pairs of p and ds * scale / l1, and l1 per query)
  float p[kP2Slots], bsc[kP2Slots];
  const int64_t tap0 = (tl.qn * a.nh + tl.head) * a.K;
#pragma unroll
  for (int i = 0; i < kP2Slots; ++i) {
    const int kap = tl.sub + kP2Subs * i;
    const bool ok = tl.q_ok && kap < a.K;  // the slots setup_slots leaves empty
    if constexpr (sizeof(E) == 4) {
      p[i] = ok ? p_ws[tap0 + kap] : 0.0f;
      bsc[i] = ok ? b_ws[tap0 + kap] : 0.0f;
    } else {
      const uint32_t w = ok ? reinterpret_cast<const uint32_t*>(p_ws)[tap0 + kap] : 0u;
      p[i] = h2_lo(w);
      bsc[i] = h2_hi(w);
    }
  }
  const float l1_q = sizeof(E) == 2 && tl.q_ok ? b_ws[tl.qn * a.nh + tl.head] : 1.0f;
  // item e = threadIdx.x + NT j moves 8 channels of one q (tensor 0) or dO row
  constexpr int kItems = 2 * kP2Q * (CW / 8), kIPT = (kItems + NT - 1) / NT;
  op_t<E> xs[kIPT];
#pragma unroll
  for (int j = 0; j < kIPT; ++j) {
    const int e = threadIdx.x + NT * j;
    const int cg = e % (CW / 8), m = (e / (CW / 8)) % kP2Q, tensor = e / (kP2Q * (CW / 8));
    const int64_t n = e < kItems ? tile_row(a, tl, m) : -1;
    xs[j] = zero_op<E>();
    if (n >= 0) {
      const E* src = tensor == 0 ? static_cast<const E*>(a.q) + n * a.qs : dout + n * D;
      xs[j] = load_op<E>(src + cw0 + 8 * cg);
    }
  }
  Slot sl[kP2Slots];
  Box box;
  setup_slots<E, kP2Subs, kP2Slots, NW>(a, tl, sl, box, s_red);
  const int nchunks = box.ncy * box.ncx;
  const int nit = (box.zhi - box.zlo + 1) * nchunks;

  // fixed-point scale of this query's B entries: 2^30 / sum_k |ds_k scale| (of
  // the values as stored: normalised ones for bf16 storage, whose l1 then
  // joins the query's dq scale)
  float l1 = 0.0f;
#pragma unroll
  for (int i = 0; i < kP2Slots; ++i) l1 += fabsf(bsc[i]);
#pragma unroll
  for (int m = 1; m < kP2Subs; m <<= 1) l1 += __shfl_xor(l1, m);
  const bool l1_ok = l1 > 1e-30f;
  const float bscale = l1_ok ? kFixA / l1 : 0.0f;
  if (tl.sub == 0) s_binv[tl.q] = l1_ok ? l1 * kFixAInv * l1_q : 0.0f;
  // p and ds scale in fixed-point units from here on
#pragma unroll
  for (int i = 0; i < kP2Slots; ++i) {
    p[i] *= a.fix_a;
    bsc[i] *= bscale;
  }
  __syncthreads();
  // stage q and dO of the tile transposed, carrying the fixed-point scales of
  // B (per query) and A (1 / fix_a) for the dK/dV products
#pragma unroll
  for (int j = 0; j < kIPT; ++j) {
    const int e = threadIdx.x + NT * j;
    if (e >= kItems) continue;
    const int cg = e % (CW / 8), m = (e / (CW / 8)) % kP2Q, tensor = e / (kP2Q * (CW / 8));
    const op_t<E> x = xs[j];
    const float sc = tensor == 0 ? s_binv[m] : a.fix_a_inv;
    if constexpr (sizeof(E) == 2) {
      const u32x4_t xb = __builtin_bit_cast(u32x4_t, x);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x2_t f = {__uint_as_float(xb[i] << 16) * sc,
                           __uint_as_float(xb[i] & 0xffff0000u) * sc};
        const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
        s_qt[tensor][8 * cg + 2 * i][m] = static_cast<uint16_t>(h & 0xffffu);
        s_qt[tensor][8 * cg + 2 * i + 1][m] = static_cast<uint16_t>(h >> 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) s_qt[tensor][8 * cg + i][m] = x[i] * sc;
    }
  }
  __syncthreads();

  // dq (16x16x32 MFMA).  CW = 64 or 96 (and 32 at three frames): wave w takes
  // frame w / 4 and the voxel k-steps w % 4, + 4, ... for all CT channel
  // tiles (at 96 in two rounds, one per staged K^T part), so one converted B
  // operand feeds several MFMA pairs; the 4 partial dq are summed at the end.
  // Wider windows (registers): task t = (frame t / CT, channels 16*(t % CT) +
  // [0, 16)) for t = w + 8 j over all k-steps.  dK/dV (32x32x16 MFMA, one per
  // frame): task t = (channels 32*(t % NC2) + [0, 32), 32-voxel block t / NC2)
  // for t = w + 8 i.
  constexpr int CT = CW / 16, NC2 = CW / 32;
  constexpr bool DQK = CW == 64 || CW == 96 || (CW == 32 && FR == 3);  // k-split dq
  constexpr int KPQ = NW / kP2Frames;  // k phases per frame (k-split dq)
  constexpr int NDQ = DQK ? CT : (kP2Frames * CT + NW - 1) / NW;  // dq accumulators
  const int mq = tl.lane & 15, kq = 8 * (tl.lane >> 4);
  // operands of the dK/dV MFMAs are re-read from LDS where used (registers are
  // the limit here: a spill reload would wait for every outstanding atomic)
  const int oq = 8 * (tl.lane >> 5);
  f32x4_t dq_acc[NDQ];
#pragma unroll
  for (int j = 0; j < NDQ; ++j) dq_acc[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const E* const kp = static_cast<const E*>(a.k);
  // fp16 accumulation: the powers of two that scale the dK and dV partials
  const float sc_k = MODE == kP2F16 ? scales[0] : 1.0f;
  const float sc_v = MODE == kP2F16 ? scales[2] : 1.0f;
  // The step's K rows are loaded first and stored to LDS after the table
  // scatter (below)
  StageRows<kP2Stage, KW, E> kr;
  StageRows<kP2Stage, CW - KW == 0 ? 32 : CW - KW, E> kr2;  // second round (CW = 96)
  Walk w = walk_begin(box);
  for (int it = 0; it < nit; ++it) {
    const Walk wn = walk_next(box, w);
    const Chunk& c = w.c;
    const int z = w.z;
    // (the redo of dK / dV alone needs no K)
    if constexpr (MODE != kP2Redo) {
      load_stage_rows<kP2Stage, KW, E>(a, tl, c, z, kp, a.ks, cw0, kr);
      if constexpr (KW < CW)
        load_stage_rows<kP2Stage, CW - KW, E>(a, tl, c, z, kp, a.ks, cw0 + KW, kr2);
    }
    // zero the transposed A and B tables; token rows of the chunk's voxels
    for (int e = threadIdx.x; e < c.nvp * kP2Row / 4; e += NT) {
      const u32x4_t zz = {0u, 0u, 0u, 0u};
      __builtin_memcpy(&s_at[4 * e], &zz, sizeof(zz));
      __builtin_memcpy(&s_bt[4 * e], &zz, sizeof(zz));
    }
    for (int vi = threadIdx.x; vi < c.nv; vi += NT)
      s_rows[vi] = static_cast<int>(chunk_row(a, tl, c, z, vi) - tl.sample0);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kP2Slots; ++i) {
      // the slot words are re-read opaquely each step, so the corner addresses,
      // weights and keys derived from them are not hoisted out of the plane
      // loop (registers are the limit: a spill reload would wait for every
      // outstanding atomic)
      Slot si = sl[i];
      asm volatile("" : "+v"(si.zc), "+v"(si.idx), "+v"(si.fx), "+v"(si.fy));
      float wz, dwz;
      if (!slot_hits(si, step_key(c.id, z), wz, dwz)) continue;
      const float pz = p[i] * wz, bz = bsc[i] * wz;
      const float fx = si.fx, fy = si.fy, gx = 1.0f - fx, gy = 1.0f - fy;
      const float w00 = gy * gx, w01 = gy * fx, w10 = fy * gx, w11 = fy * fx;
      const int idx = si.idx;
      const int base = idx & 0x1ff, dy = (idx >> 9) & 0x1f, dx = (idx >> 14) & 1;
      int* const r00 = &s_ab[base * kP2Row + tl.q];
      int* const r01 = r00 + dx * kP2Row;
      int* const r10 = r00 + dy * kP2Row;
      int* const r11 = r10 + dx * kP2Row;
      // an upper corner outside the volume has offset 0 and weight 0: it adds 0
      // to the lower corner, so all eight adds run without branches
      atomicAdd(r00, to_fix(pz * w00));
      atomicAdd(r00 + kTab, to_fix(bz * w00));
      atomicAdd(r01, to_fix(pz * w01));
      atomicAdd(r01 + kTab, to_fix(bz * w01));
      atomicAdd(r10, to_fix(pz * w10));
      atomicAdd(r10 + kTab, to_fix(bz * w10));
      atomicAdd(r11, to_fix(pz * w11));
      atomicAdd(r11 + kTab, to_fix(bz * w11));
    }
    // the K rows are stored only now: their load waits for every atomic this
    // wave issued before it (one in-order counter), which the scatter overlaps
    if constexpr (MODE != kP2Redo) store_stage<kP2Stage, KW, E>(c, kr, s_kt);
    __syncthreads();
    // dq[q] += sum_v B[q][v] K[v]; in bf16, B as a hi/lo pair because
    // sum_v B[q][v] = 0 and K may carry a large common part
    if constexpr (MODE == kP2Redo) {
    } else if constexpr (DQK) {
      const int fq = tl.wave / KPQ;
      // the channel tiles of the staged K^T rounds: [0, KW / 16), then [KW / 16, CT)
      auto dq_round = [&](auto ct0_c, auto ct1_c) {
        constexpr int ct0 = decltype(ct0_c)::value, ct1 = decltype(ct1_c)::value;
        for (int kc = 32 * (tl.wave % KPQ); kc < c.nvp; kc += 32 * KPQ) {
          float bq[8];  // fixed-point units; the query's scale is applied to dq at the end
#pragma unroll
          for (int jj = 0; jj < 8; ++jj)
            bq[jj] = static_cast<float>(s_bt[(kc + kq + jj) * kP2Row + kTQ * fq + mq]);
          const PreciseOp<E> bp = precise_op<E>(bq);
#pragma unroll
          for (int ct = ct0; ct < ct1; ++ct)
            dq_acc[ct] = mma16(bp, load_op<E>(&s_kt[(16 * (ct - ct0) + mq) * KR + kc + kq]),
                               dq_acc[ct]);
        }
      };
      dq_round(std::integral_constant<int, 0>{}, std::integral_constant<int, KW / 16>{});
      if constexpr (KW < CW) {
        __syncthreads();  // every wave is done with the first round's K^T
        store_stage<kP2Stage, CW - KW, E>(c, kr2, s_kt);
        __syncthreads();
        dq_round(std::integral_constant<int, KW / 16>{}, std::integral_constant<int, CT>{});
      }
    } else {
#pragma unroll
      for (int j = 0; j < NDQ; ++j) {
        const int t = tl.wave + NW * j;
        if (t >= kP2Frames * CT) continue;
        const int fq = t / CT, ct = t % CT;
        for (int kc = 0; kc < c.nvp; kc += 32) {
          float bq[8];  // fixed-point units; the query's scale is applied to dq at the end
#pragma unroll
          for (int jj = 0; jj < 8; ++jj)
            bq[jj] = static_cast<float>(s_bt[(kc + kq + jj) * kP2Row + kTQ * fq + mq]);
          dq_acc[j] = mma16(precise_op<E>(bq), load_op<E>(&s_kt[(16 * ct + mq) * KR + kc + kq]),
                            dq_acc[j]);
        }
      }
    }
    // dK[v] += sum_q B[q][v] q[q];  dV[v] += sum_q A[q][v] dO[q]  (32x32 MFMA),
    // added into fp32 rows with global atomics
    for (int t = tl.wave;; t += NW) {
      const int c2 = t % NC2, vb = t / NC2;
      if (vb * 32 >= c.nv) break;
      const int och = 32 * c2 + (tl.lane & 31);
      // dK, then dV: one accumulator live at a time (registers are the limit)
      f32x16_t acc = {};
#pragma unroll
      for (int f = 0; f < kP2Frames; ++f)
        acc = mma32(table_t_rows<E>(s_bt, kP2Row, kTQ * f, vb, tl.lane),
                    load_op<E>(&s_qt[0][och][kTQ * f + oq]), acc);
      if constexpr (MODE == kP2F16)
        flush_block_h16(tl, acc, s_rows, vb, c.nv, cw0 + och, dk_acc, acc_ks, sc_k);
      else
        flush_block(tl, acc, s_rows, vb, c.nv, cw0 + och, static_cast<float*>(dk_acc), acc_ks);
      acc = f32x16_t{};
#pragma unroll
      for (int f = 0; f < kP2Frames; ++f)
        acc = mma32(table_t_rows<E>(s_at, kP2Row, kTQ * f, vb, tl.lane),
                    load_op<E>(&s_qt[1][och][kTQ * f + oq]), acc);
      if constexpr (MODE == kP2F16)
        flush_block_h16(tl, acc, s_rows, vb, c.nv, cw0 + och, dv_acc, acc_vs, sc_v);
      else
        flush_block(tl, acc, s_rows, vb, c.nv, cw0 + och, static_cast<float*>(dv_acc), acc_vs);
    }
    __syncthreads();
    w = wn;
  }
  if constexpr (MODE == kP2Redo) {
  } else if constexpr (DQK) {
    // dq_acc[ct][r] = partial dq[query 16*fq + 4*(lane/16) + r][channel 16*ct +
    // lane%16] of k phase w % 4; the A^T table (free after the loop's last
    // barrier) takes the partials, and every thread sums 4 for its outputs
    float* red = reinterpret_cast<float*>(s_ab);  // [frame][k phase][16][CW]
    static_assert(NW * kTQ * CW <= 2 * kTab, "partials fit the tables");
    const int fq = tl.wave / KPQ, kph = tl.wave % KPQ;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[((fq * KPQ + kph) * kTQ + 4 * (tl.lane >> 4) + r) * CW + 16 * ct + mq] = dq_acc[ct][r];
    __syncthreads();
    for (int e = threadIdx.x; e < kP2Q * CW; e += NT) {
      const int m = e / CW, ch = e - m * CW, f = m / kTQ, mm = m % kTQ;
      float v = 0.0f;
#pragma unroll
      for (int kp = 0; kp < KPQ; ++kp) v += red[((f * KPQ + kp) * kTQ + mm) * CW + ch];
      const int64_t n = tile_row(a, tl, m);
      if (n >= 0) {
        // the extra keys' part of dq (fp32, from their backward kernel) joins
        // before the one rounding to the element type
        dq[n * a.qs + cw0 + ch] =
            from_f32<E>(v * s_binv[m] + (a.G > 0 ? dqx[n * D + cw0 + ch] : 0.0f));
      }
    }
  } else {
    // dq_acc[j][r] = dq[query 16*fq + 4*(lane/16) + r][channel 16*ct + lane%16]
#pragma unroll
    for (int j = 0; j < NDQ; ++j) {
      const int t = tl.wave + NW * j;
      if (t >= kP2Frames * CT) continue;
      const int fq = t / CT, ct = t % CT;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = kTQ * fq + 4 * (tl.lane >> 4) + r;
        const int64_t n = tile_row(a, tl, m);
        if (n >= 0) {
          const int c = cw0 + 16 * ct + mq;
          dq[n * a.qs + c] =
              from_f32<E>(dq_acc[j][r] * s_binv[m] + (a.G > 0 ? dqx[n * D + c] : 0.0f));
        }
      }
    }
  }
}

template <int HD, int CW, typename E, int FR, int MODE>
__global__ __launch_bounds__(P2Tile<FR>::Threads) void dsa3d_bwd_p2_kernel(
    Args a, const E* __restrict__ dout, const float* __restrict__ p_ws,
    const float* __restrict__ b_ws, E* __restrict__ dq, void* __restrict__ dk_acc,
    void* __restrict__ dv_acc, int64_t acc_ks, int64_t acc_vs, int cw_base,
    const float* __restrict__ scales, const float* __restrict__ dqx) {
  p2_tile<HD, CW, E, FR, MODE>(a, blockIdx.x, dout, p_ws, b_ws, dq, dk_acc, dv_acc, acc_ks, acc_vs,
                               cw_base, scales, dqx);
}

// The tiles of the columns the column-streaming kernel left (its list: count,
// then head * columns + column), fp32 accumulation: a small grid strides over
// them (most calls have none).
template <int HD, int CW, typename E, int FR>
__global__ __launch_bounds__(P2Tile<FR>::Threads) void dsa3d_bwd_p2_list_kernel(
    Args a, const E* __restrict__ dout, const float* __restrict__ p_ws,
    const float* __restrict__ b_ws, E* __restrict__ dq, void* __restrict__ dk_acc,
    void* __restrict__ dv_acc, int64_t acc_ks, int64_t acc_vs, const int* __restrict__ list) {
  const int n = list[0];
  const int groups = (a.T + FR - 1) / FR;
  const int ncol = a.B * a.tiles_h * a.tiles_w;
#pragma nounroll
  for (int item = blockIdx.x; item < n * groups; item += gridDim.x) {
    int it = item;
    asm volatile("" : "+s"(it));  // nothing of one tile is computed ahead for the next
    const int e = list[1 + it / groups], g = it % groups;
    Args b = a;
    b.head0 = e / ncol;  // blockIdx.y is 0
    b.xcd_remap = 0;
    p2_tile<HD, CW, E, FR, kP2F32>(b, (e % ncol) * groups + g, dout, p_ws, b_ws, dq, dk_acc,
                                   dv_acc, acc_ks, acc_vs, 0, nullptr, nullptr);
    __syncthreads();  // the next tile rewrites the LDS tables
  }
}

// dK / dV again with fp32 atomics, only when the fp16 accumulation overflowed
// (*flag != 0; otherwise every workgroup returns at once): a small grid strides
// over the tiles.
template <int HD, int CW, typename E, int FR>
__global__ __launch_bounds__(P2Tile<FR>::Threads) void dsa3d_bwd_p2_redo_kernel(
    Args a, const E* __restrict__ dout, const float* __restrict__ p_ws,
    const float* __restrict__ b_ws, float* __restrict__ dk_acc, float* __restrict__ dv_acc,
    int64_t acc_ks, int64_t acc_vs, int cw_base, const int* __restrict__ flag, int tiles) {
  if (*flag == 0) return;
#pragma nounroll
  for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    int t = tile;
    asm volatile("" : "+s"(t));  // nothing of one tile is computed ahead for the next
    p2_tile<HD, CW, E, FR, kP2Redo>(a, t, dout, p_ws, b_ws, nullptr, dk_acc, dv_acc, acc_ks,
                                    acc_vs, cw_base, nullptr, nullptr);
    __syncthreads();  // the next tile rewrites the LDS tables
  }
}

// Column-streaming dq/dK/dV kernel (bf16 storage, fp32 dK/dV accumulation).
// A walk takes a 4x4 (h, w) column of one head (or both columns of a pair of
// neighbouring columns at once) through every plane of its corner box.  At
// plane z, the frames whose tiles have corners on z are live; each holds the 16
// table columns of a table slot (one column: frame t in slot t % SR; a pair:
// ring slot t % (SR / 2), table slots for the left and the right tile), and its
// taps with a corner on z come from the first kernel's records (bins z0 = z:
// lower corners, z0 = z - 1: upper).  Per plane and 16x16 chunk of the box,
// the [voxel][ring query] table of B = ds * scale * w gives dq += B K (K^T
// staged in 32-channel rounds) and dK = B^T q; the table of A = p * w then
// gives dV = A^T dO.  dK and dV are added with fp32 atomics once per plane and
// walk: tiles of FR frames flush each plane of their box once per tile, and a
// voxel lies in the boxes of about three consecutive tiles of its column (the
// window spans ~7 planes), so the atomics, executed past the L2 and the bound
// of that kernel, drop to about 40% (the frames of a column share every
// flush); a pair walk halves them again where boxes are much wider than a
// column.  A frame that starts on the last plane of its ring slot's previous
// frame takes a second pass over that plane; a column whose frames start
// earlier than that (more frames live than ring slots), whose taps span more
// planes than a tile header has bins, or with more than kS2MaxT frames is
// listed and left to the tile kernel.
// Ring and K^T staging: eight slots and 32-channel K^T rounds.  (Nine slots,
// which would take every column at the long-clip shape, where a few frames'
// corner planes span nine planes, leave LDS for 16-channel rounds only: the
// kernel then took 1.2 ms longer than the ~4% of columns it would keep from
// the tile kernel.)
// Fixed-point table words -> bf16 (hi, lo) pairs in place, hi = bf16(x) and
// lo = bf16(x - hi) (the split of precise_op), word = hi | lo << 16.
__device__ __forceinline__ u32x4_t fix_to_hilo_words(const u32x4_t& w) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const f32x2_t f = {static_cast<float>(static_cast<int>(w[2 * i])),
                       static_cast<float>(static_cast<int>(w[2 * i + 1]))};
    const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
    const f32x2_t back = {__uint_as_float(hb << 16), __uint_as_float(hb & 0xffff0000u)};
    const f32x2_t rem = f - back;
    const uint32_t lb = __builtin_bit_cast(uint32_t, __builtin_convertvector(rem, bf16x2_t));
    r[2 * i] = (hb & 0xffffu) | (lb << 16);
    r[2 * i + 1] = (hb >> 16) | (lb & 0xffff0000u);
  }
  return r;
}
// The (hi, lo) operands of eight such words.
__device__ __forceinline__ PreciseOp<bf16> hilo_op(const uint32_t (&w)[8]) {
  u32x4_t h, l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = (w[2 * i] & 0xffffu) | (w[2 * i + 1] << 16);
    l[i] = (w[2 * i] >> 16) | (w[2 * i + 1] & 0xffff0000u);
  }
  PreciseOp<bf16> r;
  r.hi = __builtin_bit_cast(bf16x8_t, h);
  r.lo = __builtin_bit_cast(bf16x8_t, l);
  return r;
}
// table_t_rows of a table of such words: the hi parts (bf16(x), what
// fix_to_op gives for the fixed-point value).
__device__ __forceinline__ bf16x8_t table_t_hi(const int* table_t, int row, int col0, int vb,
                                               int lane) {
  u32x4_t w0, w1, h;
  const int* p = &table_t[(32 * vb + (lane & 31)) * row + col0 + 8 * (lane >> 5)];
  __builtin_memcpy(&w0, p, sizeof(w0));
  __builtin_memcpy(&w1, p + 4, sizeof(w1));
  h[0] = (w0[0] & 0xffffu) | (w0[1] << 16);
  h[1] = (w0[2] & 0xffffu) | (w0[3] << 16);
  h[2] = (w1[0] & 0xffffu) | (w1[1] << 16);
  h[3] = (w1[2] & 0xffffu) | (w1[3] << 16);
  return __builtin_bit_cast(bf16x8_t, h);
}

template <int HD>
struct S2 {
  static constexpr int SR = 8;                   // ring slots (live frames)
  static constexpr int KC = 32;                  // K^T channels staged per round
  static constexpr int NR = HD / KC;             // rounds
  static constexpr int Row = SR * kTQ + 2;       // [voxel][ring query] table row (ints)
};
constexpr int kS2Waves = 16;
constexpr int kS2Threads = 64 * kS2Waves;
constexpr int kS2MaxT = 256;              // frames per column (LDS frame table)
constexpr int kS2Batch = 2;               // records a thread loads at once in the table scatter

template <int HD, typename E>
__global__ __launch_bounds__(kS2Threads) void dsa3d_bwd_p2s_kernel(
    Args a, RecArgs rc, const float* __restrict__ l1_ws, E* __restrict__ dq,
    float* __restrict__ dk_acc, float* __restrict__ dv_acc, int64_t acc_ks, int64_t acc_vs) {
  static_assert(sizeof(E) == 2, "the records carry bf16 storage's fp16 (p, ds) pairs");
  constexpr int KR = kVRowSwz;  // K^T chunks in the swizzled (bank-conflict-free) layout
  constexpr int SR = S2<HD>::SR, KC = S2<HD>::KC, NR = S2<HD>::NR, kS2Row = S2<HD>::Row;
  // The live slots' transposed q (or dO), [slot][channel][16 queries], staged in
  // the K^T buffer in parts of QC channels: the whole head up to head_dim 96
  // (the buffer grows to 24 KB, LDS 161.5 KB), two 64-channel parts at 128.
  // Rows whose channel has bit 3 set hold their two 8-query halves swapped: the
  // MFMA operand read (lane l: channel l % 32, half l / 32) then meets 16 bank
  // windows in each 16-lane pass instead of 8.
  constexpr int QC = HD <= 96 ? HD : 64, NQ = HD / QC;
  constexpr int kQSPieces = SR * 2 * QC;  // 16 bytes each
  constexpr int kQSPer = (kQSPieces + kS2Threads - 1) / kS2Threads;  // pieces per thread
  constexpr int kKtElems = SR * QC * kTQ > KC * KR ? SR * QC * kTQ : KC * KR;
  static_assert(QC * NQ == HD && QC % 32 == 0, "channel parts of whole 32-channel tiles");
  static_assert(kS2Waves == 2 * SR, "two waves hold the dq tiles of each ring slot");
  __shared__ __attribute__((aligned(16))) int s_tab[kChunkNV * kS2Row];
  __shared__ __attribute__((aligned(16))) word_t<E> s_kt[kKtElems];
  __shared__ __attribute__((aligned(16))) int s_rows[kChunkNV];
  __shared__ int s_fz[kS2MaxT][2];         // per frame: zlo, zhi (zlo > zhi: never live)
  __shared__ int s_unit;                   // the unit a workgroup takes next
  __shared__ int s_live[SR];               // frame in each slot at this plane (pass), or -1
  __shared__ int s_new[SR];                // a frame that starts on the plane its slot's frame ends
  __shared__ int s_npass;                  // 2 when some slot has such a frame
  __shared__ int64_t s_rbase[SR];          // per slot: record index of the plane's record i, less i
  __shared__ int s_rsplit[SR];             // per slot: plane records below this are upper corners
  __shared__ int s_pre[SR + 1];            // per slot: its first plane record
  __shared__ int s_red[kS2Waves][8];

  const int ncpb = a.tiles_h * a.tiles_w;  // columns per sample
  const int ncol = a.B * ncpb;
  // Work units are (head, pair of columns 2j and 2j + 1 of a row), taken by a
  // persistent grid of one workgroup per CU from 8 counters, one per XCD's
  // contiguous range of units (neighbouring columns share K rows in its L2);
  // a workgroup whose range is done helps the next ranges.  (Fixed grids where
  // some workgroups return at once, e.g. one per column where a pair takes one
  // walk, left CUs idle.)
  const int tw2 = (a.tiles_w + 1) / 2;
  const int npr = a.B * a.tiles_h * tw2;  // pairs per head
  const int nunits = npr * a.nh;
  const int per = (nunits + 7) / 8;
  int* const work = rc.collist + 1 + a.nh * ncol;
  const int64_t tstep = ncpb;  // tiles between consecutive frames of a column
  const int K16 = a.K * kTQ;
  const int D = a.nh * HD;
  const E* const kp = static_cast<const E*>(a.k);
  const E* const qtb = static_cast<const E*>(rc.qt);
  Tile tl;
  tl.wave = threadIdx.x >> 6;
  tl.lane = threadIdx.x & 63;
  tl.t0 = tl.t = 0;
  const int mq = tl.lane & 15, kq = 8 * (tl.lane >> 4), oq = 8 * (tl.lane >> 5);
  // dq tiles of this wave: slot wave / 2, channels 32 rd + 16 (wave % 2) + [0, 16)
  const int my_slot = tl.wave >> 1, my_ct = tl.wave & 1;
  f32x4_t dq_acc[NR];
#pragma unroll
  for (int rd = 0; rd < NR; ++rd) dq_acc[rd] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  StageRows<kP2Stage, KC, E> kr;
  // the current unit
  int b = 0, th = 0, twp = 0, nside = 1, hc0 = 0;
  int64_t trl = 0;  // record tile of frame 0 of the pair's left column

  // A walk takes either both columns together (wide: ring slot t % (SR / 2)
  // of frame t holds the left tile in table slot 2 (t % (SR / 2)) and the
  // right one in the next) or one column (ring slot = table slot = t % SR).
  bool wide = false;
  int side = 0;  // the column of a one-column walk
  // column (0 left, 1 right) of table slot v, and the record tile of frame t there
  auto side_of = [&](int v) { return wide ? (v & 1) : side; };
  auto tile_of = [&](int v, int t) {
    return trl + side_of(v) + static_cast<int64_t>(t) * tstep;
  };

  // ---- a walk's frames: plane ranges (s_fz), corner box, ring check ---------
  // Returns the box; bad = the walk cannot take these frames; cost = its
  // chunk steps (chunks x (planes + planes a ring slot shares, which take a
  // second pass)).
  auto setup = [&](Box& box, int& bad, int& cost) {
    const int rs = wide ? SR / 2 : SR;
    int zlo = 1 << 30, zhi = -1, ylo = 1 << 30, yhi = -1, xlo = 1 << 30, xhi = -1, nsh = 0;
    bad = a.T > kS2MaxT ? 1 : 0;
    __syncthreads();  // a previous walk has read s_fz
    for (int t = threadIdx.x; t < a.T && t < kS2MaxT; t += kS2Threads) {
      int flo = 1 << 30, fhi = -1;
      for (int sd = wide ? 0 : side; sd <= (wide ? 1 : side); ++sd) {
        const int* h = rc.hdr + (trl + sd + static_cast<int64_t>(t) * tstep) * kRecHdr;
        const int nb = h[6];
        if (nb < 0) bad = 1;
        if (nb > 0) {
          flo = min(flo, h[0]);
          fhi = max(fhi, h[1]);
          ylo = min(ylo, h[2]);
          yhi = max(yhi, h[3]);
          xlo = min(xlo, h[4]);
          xhi = max(xhi, h[5]);
        }
      }
      if (fhi >= flo) {
        s_fz[t][0] = flo;
        s_fz[t][1] = fhi;
        zlo = min(zlo, flo);
        zhi = max(zhi, fhi);
      } else {
        s_fz[t][0] = 1;
        s_fz[t][1] = 0;
      }
    }
    __syncthreads();
    // the next frame of a ring slot starts after the previous one ends, or on
    // its last plane (that plane then takes a second pass for the new frames)
    // and goes on beyond it
    for (int t = threadIdx.x; t < a.T && t < kS2MaxT; t += kS2Threads) {
      if (s_fz[t][0] > s_fz[t][1]) continue;
      for (int u = t + rs; u < a.T && u < kS2MaxT; u += rs) {
        if (s_fz[u][0] > s_fz[u][1]) continue;
        if (s_fz[u][0] < s_fz[t][1] || (s_fz[u][0] == s_fz[t][1] && s_fz[u][1] == s_fz[u][0]))
          bad = 1;
        else if (s_fz[u][0] == s_fz[t][1])
          ++nsh;
        break;
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      zlo = min(zlo, __shfl_xor(zlo, m));
      zhi = max(zhi, __shfl_xor(zhi, m));
      ylo = min(ylo, __shfl_xor(ylo, m));
      yhi = max(yhi, __shfl_xor(yhi, m));
      xlo = min(xlo, __shfl_xor(xlo, m));
      xhi = max(xhi, __shfl_xor(xhi, m));
      bad = max(bad, __shfl_xor(bad, m));
      nsh += __shfl_xor(nsh, m);
    }
    if (tl.lane == 0) {
      s_red[tl.wave][0] = zlo;
      s_red[tl.wave][1] = zhi;
      s_red[tl.wave][2] = ylo;
      s_red[tl.wave][3] = yhi;
      s_red[tl.wave][4] = xlo;
      s_red[tl.wave][5] = xhi;
      s_red[tl.wave][6] = bad;
      s_red[tl.wave][7] = nsh;
    }
    __syncthreads();
    nsh = s_red[0][7];
    box.zlo = s_red[0][0];
    box.zhi = s_red[0][1];
    box.ylo = s_red[0][2];
    box.yhi = s_red[0][3];
    box.xlo = s_red[0][4];
    box.xhi = s_red[0][5];
    bad = s_red[0][6];
#pragma unroll
    for (int w = 1; w < kS2Waves; ++w) {
      box.zlo = min(box.zlo, s_red[w][0]);
      box.zhi = max(box.zhi, s_red[w][1]);
      box.ylo = min(box.ylo, s_red[w][2]);
      box.yhi = max(box.yhi, s_red[w][3]);
      box.xlo = min(box.xlo, s_red[w][4]);
      box.xhi = max(box.xhi, s_red[w][5]);
      bad = max(bad, s_red[w][6]);
      nsh += s_red[w][7];
    }
    box.zlo = __builtin_amdgcn_readfirstlane(box.zlo);
    box.zhi = __builtin_amdgcn_readfirstlane(box.zhi);
    box.ylo = __builtin_amdgcn_readfirstlane(box.ylo);
    box.yhi = __builtin_amdgcn_readfirstlane(box.yhi);
    box.xlo = __builtin_amdgcn_readfirstlane(box.xlo);
    box.xhi = __builtin_amdgcn_readfirstlane(box.xhi);
    bad = __builtin_amdgcn_readfirstlane(bad);
    box.ncy = max(1, (box.yhi - box.ylo + kChunkStep - 1) / kChunkStep);
    box.ncx = max(1, (box.xhi - box.xlo + kChunkStep - 1) / kChunkStep);
    cost = __builtin_amdgcn_readfirstlane(
        box.zhi < box.zlo ? 0 : box.ncy * box.ncx * (box.zhi - box.zlo + 1 + nsh));
  };

  // ---- the plane walk ------------------------------------------------------
  auto walk = [&](const Box& box) {
    const int rs = wide ? SR / 2 : SR;
    const int nchunks = box.ncy * box.ncx;
    for (int z = box.zlo; z <= box.zhi; ++z) {
      // ---- live frames of this plane: per ring slot the earlier frame, and a
      // later one that starts here while the earlier one ends here -------------
      __syncthreads();  // the previous plane's dq write-out has read s_live
      if (threadIdx.x < 64) {
        // wave 0: lane l scans the frames t = l, l + 64, ... of ring slot l % rs
        // (rs divides 64); the lanes of one ring slot then reduce to its
        // earliest and latest frame live on this plane
        const int l = threadIdx.x;
        int lo = 0x7fffffff, hi = -1;
        for (int t = l; t < a.T; t += 64) {
          if (s_fz[t][0] <= z && z <= s_fz[t][1]) {
            lo = min(lo, t);
            hi = max(hi, t);
          }
        }
        for (int m = rs; m < 64; m <<= 1) {
          lo = min(lo, __shfl_xor(lo, m));
          hi = max(hi, __shfl_xor(hi, m));
        }
        const int r = l;
        const int q = wide ? (r >> 1) : r;  // ring slot of table slot r (lane q holds its range)
        lo = __shfl(lo, q & (rs - 1));
        hi = __shfl(hi, q & (rs - 1));
        bool two = false;
        if (r < SR) {
          two = hi >= 0 && hi != lo;
          s_live[r] = lo == 0x7fffffff ? -1 : lo;
          s_new[r] = two ? hi : -1;
        }
        const bool any = __builtin_amdgcn_ballot_w64(two) != 0;
        if (r == 0) s_npass = any ? 2 : 1;
      }
      __syncthreads();
      const int npass = s_npass;
      for (int pass = 0; pass < npass; ++pass) {
        if (pass == 1) {
          // the frames that start on this plane, alone (the others are done)
          __syncthreads();  // the first pass's dq write-out has read s_live
          if (threadIdx.x < SR) s_live[threadIdx.x] = s_new[threadIdx.x];
          __syncthreads();
        }
        // ---- record ranges of the pass's frames: per slot the bins z0 = z - 1
        // (upper corners on z) and z0 = z (lower), adjacent in the tile's
        // records; the plane's records are numbered slot after slot
        if (threadIdx.x < 64) {
          const int r = threadIdx.x;
          const int t = r < SR ? s_live[r] : -1;
          int first = 0, cnt = 0, nup = 0;
          int64_t tb = 0;
          if (t >= 0) {
            tb = tile_of(r, t);
            const int* h = rc.hdr + tb * kRecHdr;
            const int nb = max(h[6], 0), bl = z - h[0];
            first = h[8 + min(max(bl - 1, 0), nb)];
            nup = h[8 + min(max(bl, 0), nb)] - first;
            cnt = h[8 + min(max(bl + 1, 0), nb)] - first;
          }
          int pre = cnt;  // inclusive prefix over the slots (lanes 0..SR-1)
  #pragma unroll
          for (int m = 1; m < SR; m <<= 1) {
            const int o = __shfl_up(pre, m, 64);
            if (r >= m) pre += o;
          }
          pre -= cnt;
          if (r < SR) {
            s_pre[r] = pre;
            s_rsplit[r] = pre + nup;
            s_rbase[r] = t >= 0 ? tb * K16 + first - pre : 0;
          }
          if (r == SR - 1) s_pre[SR] = pre + cnt;
        }
        __syncthreads();
        const int nrec = s_pre[SR];

        for (int ci = 0; ci < nchunks; ++ci) {
          const Chunk c = make_chunk(box, ci);
          const int cyi = box.ncx == 1 ? ci : ci / box.ncx, cxi = ci - cyi * box.ncx;
          for (int vi = threadIdx.x; vi < c.nv; vi += kS2Threads)
            s_rows[vi] = static_cast<int>(chunk_row(a, tl, c, z, vi) - tl.sample0);

          // one record into the table: B (ds * scale * w, phase 0) or A (p * w, phase 1)
          auto scatter_one = [&](const u32x4_t& r, int slot, bool up, int phase) {
            const int y0 = static_cast<int>(r[0] & 0x3fffu);
            const int x0 = static_cast<int>((r[0] >> 14) & 0x3fffu);
            if (nchunks > 1) {
              const int ky = min((y0 - box.ylo) / kChunkStep, box.ncy - 1);
              const int kx = min((x0 - box.xlo) / kChunkStep, box.ncx - 1);
              if (ky != cyi || kx != cxi) return;
            }
            const int qq = static_cast<int>(r[0] >> 28);
            const float fz = __uint_as_float(r[2]);
            const float wz = up ? fz : 1.0f - fz;
            const float fx = static_cast<float>(r[1] & 0xffffu) * (1.0f / 65536.0f);
            const float fy = static_cast<float>(r[1] >> 16) * (1.0f / 65536.0f);
            const float v = (phase == 0 ? h2_hi(r[3]) * kFixA : h2_lo(r[3]) * a.fix_a) * wz;
            const float gx = 1.0f - fx, gy = 1.0f - fy;
            const int base = (y0 - c.cy0) * c.nx + (x0 - c.cx0);
            const int dy = fy != 0.0f ? c.nx : 0, dx = fx != 0.0f ? 1 : 0;
            int* const r00 = &s_tab[base * kS2Row + kTQ * slot + qq];
            int* const r10 = r00 + dy * kS2Row;
            atomicAdd(r00, to_fix(v * (gy * gx)));
            atomicAdd(r00 + dx * kS2Row, to_fix(v * (gy * fx)));
            atomicAdd(r10, to_fix(v * (fy * gx)));
            atomicAdd(r10 + dx * kS2Row, to_fix(v * (fy * fx)));
          };
          auto slot_of = [&](int i) {
            int j = 0;
    #pragma unroll
            for (int k = 1; k < SR; ++k) j += i >= s_pre[k] ? 1 : 0;
            return j;
          };
          auto scatter = [&](int phase) {
            for (int e = threadIdx.x; e < c.nvp * kS2Row / 4; e += kS2Threads) {
              const u32x4_t zz = {0u, 0u, 0u, 0u};
              __builtin_memcpy(&s_tab[4 * e], &zz, sizeof(zz));
            }
            __syncthreads();
            // kS2Batch records per thread and iteration, their loads issued first
            for (int i0 = threadIdx.x; i0 < nrec; i0 += kS2Batch * kS2Threads) {
              u32x4_t r[kS2Batch];
              int j[kS2Batch];
    #pragma unroll
              for (int u = 0; u < kS2Batch; ++u) {
                const int i = i0 + u * kS2Threads < nrec ? i0 + u * kS2Threads : i0;
                j[u] = slot_of(i);
                r[u] = rc.rec[s_rbase[j[u]] + i];
              }
    #pragma unroll
              for (int u = 0; u < kS2Batch; ++u) {
                const int i = i0 + u * kS2Threads;
                if (i < nrec) scatter_one(r[u], j[u], i < s_rsplit[j[u]], phase);
              }
            }
          };

          // ---- B: dq and dK -----------------------------------------------------
          // The live slots' transposed q (then dO) wait in the K^T buffer for the
          // dK (dV) products, one channel part at a time: each thread loads its
          // 16-byte pieces a phase early and stores them once that buffer is free,
          // so the products read LDS instead of waiting on global loads.
          u32x4_t qs_reg[kQSPer];
          auto qs_load = [&](int part, int qp) {  // part 0: q, 1: dO; channel part qp
    #pragma unroll
            for (int k = 0; k < kQSPer; ++k) {
              const int pc = static_cast<int>(threadIdx.x) + k * kS2Threads;
              qs_reg[k] = u32x4_t{0u, 0u, 0u, 0u};
              if (pc < kQSPieces) {
                const int v = pc / (2 * QC), t = s_live[v];
                if (t >= 0)
                  qs_reg[k] = reinterpret_cast<const u32x4_t*>(
                      qtb + tile_of(v, t) * (2 * HD * kTQ) + (part * HD + qp * QC) * kTQ)
                      [pc % (2 * QC)];
              }
            }
          };
          auto qs_store = [&]() {
    #pragma unroll
            for (int k = 0; k < kQSPer; ++k) {
              const int pc = static_cast<int>(threadIdx.x) + k * kS2Threads;
              // piece pc = half pc % 2 of row pc / 2 (bit 3 of the row: bit 4 of pc)
              if (pc < kQSPieces)
                __builtin_memcpy(&s_kt[8 * (pc ^ ((pc >> 4) & 1))], &qs_reg[k], sizeof(qs_reg[k]));
            }
          };
          // products of one channel part over the live slots, flushed per task
          auto products = [&](int qp, bool dv) {
            constexpr int C2 = QC / 32;
            for (int task = tl.wave;; task += kS2Waves) {
              const int c2 = task % C2, vb = task / C2;
              if (vb * 32 >= c.nv) break;
              const int lch = 32 * c2 + (tl.lane & 31), och = qp * QC + lch;
              f32x16_t acc = {};
    #pragma unroll
              for (int r = 0; r < SR; ++r) {
                if (s_live[r] < 0) continue;
                const op_t<E> qo =
                    load_op<E>(&s_kt[(r * QC + lch) * kTQ + (oq ^ (8 * ((lch >> 3) & 1)))]);
                acc = mma32(dv ? table_t_rows<E>(s_tab, kS2Row, kTQ * r, vb, tl.lane)
                               : table_t_hi(s_tab, kS2Row, kTQ * r, vb, tl.lane),
                            qo, acc);
              }
              flush_block(tl, acc, s_rows, vb, c.nv, hc0 + och, dv ? dv_acc : dk_acc,
                          dv ? acc_vs : acc_ks);
            }
          };
          qs_load(0, 0);
          load_stage_rows<kP2Stage, KC, E>(a, tl, c, z, kp, a.ks, hc0, kr);
          scatter(0);
          __syncthreads();
          // B in place as bf16 (hi, lo) pairs, converted once for every dq round
          // and wave (the round's K^T store below is in the same barrier interval)
          for (int e = threadIdx.x; e < c.nvp * kS2Row / 4; e += kS2Threads) {
            u32x4_t w;
            __builtin_memcpy(&w, &s_tab[4 * e], sizeof(w));
            w = fix_to_hilo_words(w);
            __builtin_memcpy(&s_tab[4 * e], &w, sizeof(w));
          }
    #pragma unroll
          for (int rd = 0; rd < NR; ++rd) {
            store_stage<kP2Stage, KC, E, true>(c, kr, s_kt);
            __syncthreads();
            if (rd + 1 < NR)
              load_stage_rows<kP2Stage, KC, E>(a, tl, c, z, kp, a.ks, hc0 + KC * (rd + 1), kr);
            if (s_live[my_slot] >= 0) {
              for (int kc = 0; kc < c.nvp; kc += 32) {
                // fixed-point units; the query's l1 / 2^30 is applied to dq at the end
                uint32_t bw[8];
    #pragma unroll
                for (int jj = 0; jj < 8; ++jj)
                  bw[jj] = static_cast<uint32_t>(
                      s_tab[(kc + kq + jj) * kS2Row + kTQ * my_slot + mq]);
                dq_acc[rd] = mma16(hilo_op(bw),
                                   load_op<E>(&s_kt[(16 * my_ct + mq) * KR + ((kc + kq) ^ vt_swz(mq))]),
                                   dq_acc[rd]);
              }
            }
            __syncthreads();  // every wave is done with this round's K^T
          }
          // dK[v] += sum over ring queries of B[q][v] q[q] (32x32 MFMA per live slot)
    #pragma unroll
          for (int qp = 0; qp < NQ; ++qp) {
            if (qp > 0) __syncthreads();  // every wave is done with the previous part
            qs_store();
            if (qp + 1 < NQ)
              qs_load(0, qp + 1);
            else
              qs_load(1, 0);
            __syncthreads();
            products(qp, false);
          }
          __syncthreads();  // every wave is done with the B table (and the staged q)

          // ---- A: dV --------------------------------------------------------------
          qs_store();
          if (NQ > 1) qs_load(1, 1);
          scatter(1);  // its first barrier orders the staged dO before the products
          __syncthreads();
    #pragma unroll
          for (int qp = 0; qp < NQ; ++qp) {
            if (qp > 0) {
              __syncthreads();  // every wave is done with the previous part
              qs_store();
              __syncthreads();
            }
            products(qp, true);
          }
          __syncthreads();  // the table and s_rows are rewritten by the next step
        }


        // ---- frames that end at this plane: their dq -------------------------
        const int tr = s_live[my_slot];
        if (tr >= 0 && s_fz[tr][1] == z) {
          const int w0 = tl.w0 + side_of(my_slot) * kTileW;
  #pragma unroll
          for (int rd = 0; rd < NR; ++rd) {
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int m = 4 * (tl.lane >> 4) + i;
              const int h = tl.h0 + m / kTileW, w = w0 + m % kTileW;
              if (h < a.H && w < a.W) {
                const int64_t n = tl.sample0 + (static_cast<int64_t>(tr) * a.H + h) * a.W + w;
                const int ch = hc0 + KC * rd + 16 * my_ct + mq;
                dq[n * a.qs + ch] =
                    from_f32<E>(dq_acc[rd][i] * l1_ws[n * a.nh + tl.head] * kFixAInv);
              }
            }
            dq_acc[rd] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
          }
        }
      }  // passes
    }
  };

  // Per unit: both columns of the pair in one walk (wide) where the ring takes
  // their frames and that walk is cheaper than one walk per column (where
  // frames span more planes than half the ring, the wide walk's shared planes
  // double its steps, and a wider box can add a chunk), else one walk per
  // column; a column that its one-column walk cannot take is left to the tile
  // kernel.
  constexpr int kNoWalk = 1 << 30;
#pragma nounroll
  for (int xq = 0; xq < 8; ++xq) {
    const int q = (static_cast<int>(blockIdx.x) + xq) & 7;
    const int ulo = q * per, uhi = min(ulo + per, nunits);
#pragma nounroll
    for (;;) {
      __syncthreads();  // every wave is done with the previous unit and s_unit
      if (threadIdx.x == 0) s_unit = ulo + atomicAdd(&work[q], 1);
      __syncthreads();
      const int u = s_unit;
      if (u >= uhi) break;
      const int hl = u / npr, pr = u % npr;
      b = pr / (a.tiles_h * tw2);
      th = (pr % (a.tiles_h * tw2)) / tw2;
      twp = pr % tw2;
      nside = 2 * twp + 1 < a.tiles_w ? 2 : 1;
      tl.head = a.head0 + hl;
      tl.b = b;
      tl.sample0 = static_cast<int64_t>(b) * a.N;
      tl.h0 = th * kTileH;
      tl.w0 = 2 * twp * kTileW;
      hc0 = tl.head * HD;
      trl = static_cast<int64_t>(tl.head) * rc.tiles + rec_tile(a, b, 0, th, 2 * twp);

      bool go_wide = false;
      if (nside == 2) {
        Box box;
        int bad, cw, c0 = 0, c1 = 0;
        wide = true;
        setup(box, bad, cw);
        if (!bad) {
          wide = false;
#pragma nounroll
          for (side = 0; side < 2; ++side) {
            int cs;
            setup(box, bad, cs);
            (side == 0 ? c0 : c1) = bad ? kNoWalk : cs;
          }
          go_wide = cw < c0 + c1 || c0 == kNoWalk || c1 == kNoWalk;
        }
      }
#pragma nounroll
      for (int job = go_wide ? 0 : 1; job <= (go_wide ? 0 : nside); ++job) {
        wide = job == 0;
        side = job == 2 ? 1 : 0;
        Box box;
        int bad, cost;
        setup(box, bad, cost);
        if (bad) {
          if (threadIdx.x == 0)
            rc.collist[1 + atomicAdd(&rc.collist[0], 1)] =
                tl.head * ncol + (b * a.tiles_h + th) * a.tiles_w + 2 * twp + side;
          continue;
        }
        if (box.zhi >= box.zlo) walk(box);
      }
    }
  }
}

// Backward of the extra keys (attention.py:160-173) for 16 consecutive tokens
// of one sample and head (4 waves, 16 lanes per query): S_e = q . ek_g and
// dP_e = dO . ev_g on the matrix cores, then per (query, key) p = exp(scale
// S_e - lse) and the dropout factor f of tap K + g.  Two launches:
//   DLT: before the first backward kernel, the keys' part of Delta, sum_g p f
//     dP_e per (token, head) in fp32, into a.dlt (the first backward kernel
//     adds the taps' part and dlse and writes the whole Delta back);
//   otherwise: after it, ds * scale = p (f dP_e - Delta) scale with that
//     Delta, written with p f ([B, nh, N, G], for the dEK / dEV reduction), and
//     dq's extra part sum_g ds_g scale ek_g (MFMA, fp32 [rows, D] dqx, which
//     the second backward kernel adds to its tap part before dq's one rounding).
constexpr int kXQ = 16;
template <int HD, typename E, bool DLT>
__global__ __launch_bounds__(256) void dsa3d_bwd_extra_kernel(
    Args a, const E* __restrict__ dout, const float* __restrict__ lse, float* __restrict__ dqx,
    E* __restrict__ ds_e, E* __restrict__ pf_e) {
  constexpr int EKR = sizeof(E) == 2 ? 40 : 36;  // 16-byte aligned transposed rows
  __shared__ __attribute__((aligned(16))) float s_s[kXQ * kSRow];   // S_e, then ds * scale
  __shared__ __attribute__((aligned(16))) float s_dp[kXQ * kSRow];  // dP_e
  __shared__ __attribute__((aligned(16))) word_t<E> s_ekt[HD * EKR];  // 32 keys of EK^T
  __shared__ float s_delta[kXQ], s_lse[kXQ];
  const int G = a.G, Gp = (G + 31) & ~31;
  const int D = a.nh * HD;
  const int b = blockIdx.x / ((a.N + kXQ - 1) / kXQ);
  const int64_t n0 = static_cast<int64_t>(blockIdx.x % ((a.N + kXQ - 1) / kXQ)) * kXQ;
  const int head = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int mq = lane & 15, kq = 8 * (lane >> 4);
  const int64_t sample0 = static_cast<int64_t>(b) * a.N;
  // Delta (the whole, from the first backward kernel) and lse of each query
  if (threadIdx.x < kXQ) {
    const int64_t n = n0 + threadIdx.x;
    const int64_t r = (sample0 + (n < a.N ? n : 0)) * a.nh + head;
    s_delta[threadIdx.x] = !DLT && n < a.N ? a.dlt[r] : 0.0f;
    s_lse[threadIdx.x] = n < a.N ? lse[r] : 0.0f;
  }
  // q and dO rows of the 16 queries as MFMA A operands (zero past N)
  op_t<E> xq[HD / 32], xo[HD / 32];
  {
    const int64_t n = n0 + mq;
#pragma unroll
    for (int c = 0; c < HD / 32; ++c) xq[c] = xo[c] = zero_op<E>();
    if (n < a.N) {
      const E* qr = static_cast<const E*>(a.q) + (sample0 + n) * a.qs + head * HD + kq;
      const E* orow = dout + (sample0 + n) * D + head * HD + kq;
#pragma unroll
      for (int c = 0; c < HD / 32; ++c) {
        xq[c] = load_op<E>(qr + 32 * c);
        xo[c] = load_op<E>(orow + 32 * c);
      }
    }
  }
  const E* const ek = static_cast<const E*>(a.ek) + static_cast<int64_t>(b) * a.G * D + head * HD;
  const E* const ev = static_cast<const E*>(a.ev) + static_cast<int64_t>(b) * a.G * D + head * HD;
  for (int eb = wave; eb < Gp / 16; eb += 4) {
    const int g = 16 * eb + mq;
    f32x4_t sacc = {0.0f, 0.0f, 0.0f, 0.0f}, dacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < HD / 32; ++c) {
      const op_t<E> yk = g < G ? load_op<E>(ek + static_cast<int64_t>(g) * D + 32 * c + kq) : zero_op<E>();
      const op_t<E> yv = g < G ? load_op<E>(ev + static_cast<int64_t>(g) * D + 32 * c + kq) : zero_op<E>();
      sacc = mma16(xq[c], yk, sacc);
      dacc = mma16(xo[c], yv, dacc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s_s[(4 * (lane >> 4) + r) * kSRow + g] = sacc[r];
      s_dp[(4 * (lane >> 4) + r) * kSRow + g] = dacc[r];
    }
  }
  __syncthreads();
  if constexpr (DLT) {
    // the keys' part of Delta: thread t takes query t / 16, keys t % 16 + 16 j
    const int qi = threadIdx.x / 16, sub = threadIdx.x % 16;
    const int64_t n = n0 + qi;
    const int64_t row = sample0 + n;
    float part = 0.0f;
    for (int g = sub; g < G; g += 16) {
      const float pe = __expf(s_s[qi * kSRow + g] * a.softmax_scale - s_lse[qi]);
      const float f = a.drop.threshold == 0 ? 1.0f : dropout_factor(a.drop, row, head, a.K + g);
      part = __builtin_fmaf(pe * f, s_dp[qi * kSRow + g], part);
    }
    part = group_sum<16>(part);
    if (sub == 0 && n < a.N) a.dlt[row * a.nh + head] = part;
    return;
  }
  // p, ds * scale per (query, key): thread t takes query t / 16, keys t % 16 + 16 j
  {
    const int qi = threadIdx.x / 16, sub = threadIdx.x % 16;
    const int64_t n = n0 + qi;
    const int64_t row = sample0 + n;
    const int64_t erow = ((static_cast<int64_t>(b) * a.nh + head) * a.N + n) * G;
    for (int g = sub; g < Gp; g += 16) {
      float dss = 0.0f;
      if (g < G && n < a.N) {
        const float pe = __expf(s_s[qi * kSRow + g] * a.softmax_scale - s_lse[qi]);
        const float f = a.drop.threshold == 0 ? 1.0f : dropout_factor(a.drop, row, head, a.K + g);
        dss = pe * (f * s_dp[qi * kSRow + g] - s_delta[qi]) * a.softmax_scale;
        ds_e[erow + g] = from_f32<E>(dss);
        pf_e[erow + g] = from_f32<E>(pe * f);
      }
      s_s[qi * kSRow + g] = dss;  // read by this thread only above
    }
  }
  // dq_e = DS_e . EK: k-steps of 32 keys, EK^T staged per step; wave w takes
  // the channel tiles w, w + 4, ...
  constexpr int CT = HD / 16, TW = (CT + 3) / 4;
  f32x4_t dqa[TW];
#pragma unroll
  for (int t = 0; t < TW; ++t) dqa[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  for (int kc = 0; kc < Gp; kc += 32) {
    __syncthreads();  // the ds table is complete (first step) / the previous step's MFMAs are done
    for (int e = threadIdx.x; e < 32 * (HD / 8); e += 256) {
      const int gi = e / (HD / 8), cg = e % (HD / 8), g = kc + gi;
      op_t<E> x = zero_op<E>();
      if (g < G) x = load_op<E>(ek + static_cast<int64_t>(g) * D + 8 * cg);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (sizeof(E) == 2) {
          const u32x4_t xb = __builtin_bit_cast(u32x4_t, x);
          s_ekt[(8 * cg + i) * EKR + gi] =
              static_cast<uint16_t>((i & 1) ? (xb[i / 2] >> 16) : (xb[i / 2] & 0xffffu));
        } else {
          s_ekt[(8 * cg + i) * EKR + gi] = x[i];
        }
      }
    }
    __syncthreads();
    float bq[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) bq[jj] = s_s[mq * kSRow + kc + kq + jj];
    const PreciseOp<E> bp = precise_op<E>(bq);
#pragma unroll
    for (int t = 0; t < TW; ++t) {
      const int ct = wave + 4 * t;
      if (ct < CT) dqa[t] = mma16(bp, load_op<E>(&s_ekt[(16 * ct + mq) * EKR + kq]), dqa[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    const int ct = wave + 4 * t;
    if (ct >= CT) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = n0 + 4 * (lane >> 4) + r;
      if (n < a.N) dqx[(sample0 + n) * D + head * HD + 16 * ct + mq] = dqa[t][r];
    }
  }
}

// dEK and dEV of the extra keys (attention.py:160-173): for one (sample,
// head), dEK[g][c] = sum_n DS_e[n][g] q[n][c] and dEV[g][c] = sum_n PF_e[n][g]
// dO[n][c] (blockIdx.z 0 / 1), DS_e = ds * scale and PF_e = p * dropout factor
// of every (query, extra key) from the first backward kernel.  A workgroup
// reduces `range` tokens (blockIdx.x) in chunks of 32 staged transposed in LDS
// (32x32 MFMAs over 16 tokens at a time, keys x channels) and adds its fp32
// partial into acc [B, G, D] with one atomic per element: a few tens of
// partials per element in all.
constexpr int kXChunk = 32;
template <int HD, typename E>
__global__ __launch_bounds__(256) void extra_grad_kernel(const E* __restrict__ ds_e,
                                                         const E* __restrict__ pf_e,
                                                         const E* __restrict__ q, int64_t qs,
                                                         const E* __restrict__ dout, int64_t N,
                                                         int nh, int G, int64_t range,
                                                         float* __restrict__ dek_acc,
                                                         float* __restrict__ dev_acc) {
  constexpr int TR = kXChunk + (sizeof(E) == 2 ? 8 : 4);  // 16-byte aligned token rows
  constexpr int MAXT = (kMaxExtra / 32) * (HD / 32) / 4;  // 32x32 tiles per wave at most
  __shared__ __attribute__((aligned(16))) word_t<E> s_x[kMaxExtra * TR];  // X^T [key][token]
  __shared__ __attribute__((aligned(16))) word_t<E> s_y[HD * TR];         // Y^T [channel][token]
  const int bh = blockIdx.y, b = bh / nh, head = bh % nh;
  const bool isv = blockIdx.z == 1;
  const int D = nh * HD, Gp = (G + 31) & ~31;
  const int MT = Gp / 32, NTL = HD / 32;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const E* const X = (isv ? pf_e : ds_e) + static_cast<int64_t>(bh) * N * G;
  const E* const Y = isv ? dout + static_cast<int64_t>(b) * N * D : q + static_cast<int64_t>(b) * N * qs;
  const int64_t ys = isv ? D : qs;
  f32x16_t acc[MAXT];
#pragma unroll
  for (int i = 0; i < MAXT; ++i) acc[i] = f32x16_t{};
  const int64_t n_begin = static_cast<int64_t>(blockIdx.x) * range;
  const int64_t n_end = n_begin + range < N ? n_begin + range : N;
  for (int64_t n0 = n_begin; n0 < n_end; n0 += kXChunk) {
    __syncthreads();  // the previous chunk's MFMAs are done with the stages
    // X rows of the chunk (keys g, 8 at a time) and Y rows (8 channels at a time),
    // transposed; tokens past the range and keys past G read zero
    for (int e = threadIdx.x; e < kXChunk * (Gp / 8); e += 256) {
      const int tok = e / (Gp / 8), g8 = 8 * (e % (Gp / 8));
      const int64_t n = n0 + tok;
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[i] = (n < n_end && g8 + i < G) ? to_f32(X[n * G + g8 + i]) : 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (sizeof(E) == 2) s_x[(g8 + i) * TR + tok] = from_f32<bf16>(v[i]).bits;
        else s_x[(g8 + i) * TR + tok] = v[i];
      }
    }
    for (int e = threadIdx.x; e < kXChunk * (HD / 8); e += 256) {
      const int tok = e / (HD / 8), c8 = 8 * (e % (HD / 8));
      const int64_t n = n0 + tok;
      op_t<E> x = zero_op<E>();
      if (n < n_end) x = load_op<E>(Y + n * ys + head * HD + c8);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (sizeof(E) == 2) {
          const u32x4_t xb = __builtin_bit_cast(u32x4_t, x);
          s_y[(c8 + i) * TR + tok] =
              static_cast<uint16_t>((i & 1) ? (xb[i / 2] >> 16) : (xb[i / 2] & 0xffffu));
        } else {
          s_y[(c8 + i) * TR + tok] = x[i];
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + 4 * i;
      if (t >= MT * NTL) continue;
      const int gb = t / NTL, cb = t % NTL;
#pragma unroll
      for (int ks = 0; ks < kXChunk; ks += 16) {
        const int k0 = ks + 8 * (lane >> 5);
        acc[i] = mma32(load_op<E>(&s_x[(32 * gb + (lane & 31)) * TR + k0]),
                       load_op<E>(&s_y[(32 * cb + (lane & 31)) * TR + k0]), acc[i]);
      }
    }
  }
  // acc[i] register r: key 32 gb + 8 (r / 4) + 4 (lane / 32) + r % 4, channel 32 cb + lane % 32
  float* const out = (isv ? dev_acc : dek_acc) + static_cast<int64_t>(b) * G * D + head * HD;
#pragma unroll
  for (int i = 0; i < MAXT; ++i) {
    const int t = wave + 4 * i;
    if (t >= MT * NTL) continue;
    const int gb = t / NTL, cb = t % NTL;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int g = 32 * gb + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
      if (g < G && acc[i][r] != 0.0f)
        atomicAdd(out + static_cast<int64_t>(g) * D + 32 * cb + (lane & 31), acc[i][r]);
    }
  }
}

}  // namespace

// Kernel arguments for a launch over `tiles` workgroups per head.
tiled::Args make_tiled_args(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v,
                            const void* off, int64_t tiles, const void* ek = nullptr,
                            const void* ev = nullptr) {
  tiled::Args a;
  a.ek = ek;
  a.ev = ev;
  a.G = d.extra_g;
  a.dlt = nullptr;
  a.q = q;
  a.k = k;
  a.v = v;
  a.off = off;
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
  a.tiles_h = (d.H + tiled::kTileH - 1) / tiled::kTileH;
  a.tiles_w = (d.W + tiled::kTileW - 1) / tiled::kTileW;
  a.xcd_remap = (tiles % 8 == 0) ? static_cast<int>(tiles / 8) : 0;
  a.head0 = 0;
  a.offset_scale = d.offset_scale;
  a.softmax_scale = d.softmax_scale;
  a.div_x = d.T > 1 ? static_cast<float>(d.T - 1) : 0.0f;
  a.div_y = d.H > 1 ? static_cast<float>(d.H - 1) : 0.0f;
  a.div_z = d.W > 1 ? static_cast<float>(d.W - 1) : 0.0f;
  a.rdiv_x = d.T > 1 ? 1.0f / static_cast<float>(d.T - 1) : 0.0f;
  a.rdiv_y = d.H > 1 ? 1.0f / static_cast<float>(d.H - 1) : 0.0f;
  a.rdiv_z = d.W > 1 ? 1.0f / static_cast<float>(d.W - 1) : 0.0f;
  a.bdiv_x = static_cast<float>(d.W > 1 ? d.W - 1 : 1);
  a.bdiv_y = static_cast<float>(d.H > 1 ? d.H - 1 : 1);
  a.bdiv_z = static_cast<float>(d.T > 1 ? d.T - 1 : 1);
  a.rbdiv_x = 1.0f / a.bdiv_x;
  a.rbdiv_y = 1.0f / a.bdiv_y;
  a.rbdiv_z = 1.0f / a.bdiv_z;
  a.r_kw = 1.0f / static_cast<float>(d.kw);
  a.r_khkw = 1.0f / static_cast<float>(d.kh * d.kw);
  // the unnormalisation (S/2), the slot divisor and offset_scale, multiplied
  // left to right in fp32
  a.gsx = 0.5f * static_cast<float>(d.W) * a.rdiv_x * a.offset_scale;
  a.gsy = 0.5f * static_cast<float>(d.H) * a.rdiv_y * a.offset_scale;
  a.gsz = 0.5f * static_cast<float>(d.T) * a.rdiv_z * a.offset_scale;
  a.drop = dropout_args(d);
  a.fix_a = tiled::fix_a_scale(a.drop);
  a.fix_a_inv = 1.0f / a.fix_a;
  return a;
}

template <int FRAMES>
int64_t tiled_tiles(const msd_dsa3d_desc& d) {
  return tiled::tile_count<FRAMES>(d.B, d.T, d.H, d.W);
}

template <int FRAMES>
dim3 tiled_grid(const msd_dsa3d_desc& d) {
  return dim3(static_cast<unsigned>(tiled_tiles<FRAMES>(d)), d.num_heads);
}

namespace {
// head sizes with compiled tiled kernels
bool tiled_head_dim(int hd) { return hd == 32 || hd == 64 || hd == 96 || hd == 128; }
}  // namespace

bool dsa3d_tiled_supported(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v) {
  if ((d.dtype != MSD_BF16 && d.dtype != MSD_F32) || !tiled_head_dim(d.head_dim)) return false;
  const int64_t eb = d.dtype == MSD_BF16 ? 2 : 4;
  if (d.kt * d.kh * d.kw > tiled::kMaxTaps || d.extra_g > tiled::kMaxExtra) return false;
  if (d.T > 32767 || d.H > 32767 || d.W > 32767) return false;
  // the chunk grid of any corner box must number fewer than kMaxChunks
  const int64_t cy = (d.H + tiled::kChunkStep - 1) / tiled::kChunkStep + 1;
  const int64_t cx = (d.W + tiled::kChunkStep - 1) / tiled::kChunkStep + 1;
  if (cy * cx >= tiled::kMaxChunks) return false;
  const int64_t tiles = static_cast<int64_t>(d.B) * d.T * ((d.H + 3) / 4) * ((d.W + 3) / 4);
  if (tiles > 0x7fffffff || d.num_heads > 65535) return false;
  // 8-element (16- or 32-byte) vector loads of q/k/v rows
  if ((d.q_stride % 8) || (d.k_stride % 8) || (d.v_stride % 8)) return false;
  // dK/dV rows of a sample are addressed with 32-bit lane offsets (elements
  // below 2^30, so bytes below 2^32 even for fp32)
  const int64_t n = static_cast<int64_t>(d.T) * d.H * d.W;
  if (n * d.k_stride >= (int64_t{1} << 30) || n * d.v_stride >= (int64_t{1} << 30)) return false;
  // K/V chunk rows are addressed as a 64-bit chunk base plus a 32-bit lane byte
  // offset (24-bit multiplies): kChunk * (W + 1) rows must span < 2^31 bytes
  for (const int64_t st : {d.k_stride, d.v_stride})
    if (st >= (int64_t{1} << 23) ||
        static_cast<int64_t>(tiled::kChunk) * (d.W + 1) * st * eb >= (int64_t{1} << 31))
      return false;
  for (const void* p : {q, k, v})
    if (reinterpret_cast<uintptr_t>(p) % 16) return false;
  return true;
}

namespace {
template <typename E>
hipError_t fwd_tiled_typed(const msd_dsa3d_desc& d, const tiled::Args& a, void* out, float* lse,
                           hipStream_t s) {
  const dim3 grid = tiled_grid<1>(d), block(tiled::kThreads);
  E* o = static_cast<E*>(out);
  auto go = [&]<int HD>() {
    if (a.G > 0)
      hipLaunchKernelGGL((dsa3d_fwd_tiled_kernel<HD, E, true>), grid, block, 0, s, a, o, lse);
    else
      hipLaunchKernelGGL((dsa3d_fwd_tiled_kernel<HD, E, false>), grid, block, 0, s, a, o, lse);
  };
  switch (d.head_dim) {
    case 32: go.template operator()<32>(); break;
    case 64: go.template operator()<64>(); break;
    case 96: go.template operator()<96>(); break;
    case 128: go.template operator()<128>(); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_dsa3d_fwd_tiled(const msd_dsa3d_desc& d, const void* q, const void* k,
                                  const void* v, const void* off, const void* ek, const void* ev,
                                  void* out, float* lse, hipStream_t s) {
  const tiled::Args a = make_tiled_args(d, q, k, v, off, tiled_tiles<1>(d), ek, ev);
  if (d.dtype == MSD_BF16) return fwd_tiled_typed<bf16>(d, a, out, lse, s);
  return fwd_tiled_typed<float>(d, a, out, lse, s);
}

// Largest power of two s with s * bound <= 2^14 (1 for a zero or non-finite
// bound; at most 2^100).
__device__ __forceinline__ float h16_pow2_scale(float bound) {
  if (!(bound > 0.0f) || !__builtin_isfinite(bound)) return 1.0f;
  int e;
  frexpf(16384.0f / bound, &e);  // 16384 / bound = f 2^e, f in [0.5, 1)
  return ldexpf(1.0f, min(e - 1, 100));
}

// Magnitudes behind the fp16 dK / dV accumulators' scales (bf16 storage), over
// an evenly spread sample of at most about kBoundRows token rows (every row of
// a smaller input): the largest |q| and |dO| element, the largest L2 norm of a
// head's slice of a dO row and of a V row (extra values included), and the
// largest |dlse|.  One thread per (sampled row, head), 16-byte loads; each
// block writes its maxima to part[blockIdx.x][kBoundsWords].
constexpr int kBoundsBlocks = 256;
constexpr int kBoundsWords = 8;
constexpr int64_t kBoundRows = 4096;
__global__ __launch_bounds__(256) void h16_bounds_kernel(
    const bf16* __restrict__ q, int64_t qs, const bf16* __restrict__ dout,
    const bf16* __restrict__ v, int64_t vs, const bf16* __restrict__ ev, int64_t erows,
    const float* __restrict__ dlse, int64_t rows, int nh, int hd, float* __restrict__ part) {
  float m[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t step = rows > kBoundRows ? rows / kBoundRows : 1;
  const int64_t nsamp = (rows + step - 1) / step;
  const int D = nh * hd;
  // (largest |x|, sum of x^2) over hd elements from p
  auto scan = [hd](const bf16* p, float& mx, float& ss) {
    for (int c = 0; c < hd; c += 8) {
      const u32x4_t x = load16(p + c);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = __uint_as_float(x[k] << 16), hi = __uint_as_float(x[k] & 0xffff0000u);
        mx = fmaxf(mx, fmaxf(fabsf(lo), fabsf(hi)));
        ss += lo * lo + hi * hi;
      }
    }
  };
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < nsamp * nh;
       i += stride) {
    const int64_t j = i / nh, r = j * step;
    const int h = static_cast<int>(i - j * nh);
    float mx = 0.0f, ss = 0.0f;
    scan(q + r * qs + h * hd, mx, ss);
    m[0] = fmaxf(m[0], mx);
    mx = ss = 0.0f;
    scan(dout + r * D + h * hd, mx, ss);
    m[1] = fmaxf(m[1], mx);
    m[2] = fmaxf(m[2], sqrtf(ss));
    mx = ss = 0.0f;
    scan(v + r * vs + h * hd, mx, ss);
    m[3] = fmaxf(m[3], sqrtf(ss));
    if (dlse != nullptr) m[4] = fmaxf(m[4], fabsf(dlse[r * nh + h]));
  }
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < erows * nh;
       i += stride) {
    float mx = 0.0f, ss = 0.0f;
    scan(ev + (i / nh) * D + (i % nh) * hd, mx, ss);
    m[3] = fmaxf(m[3], sqrtf(ss));
  }
  __shared__ float red[4][5];
#pragma unroll
  for (int k = 0; k < 5; ++k) {
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) m[k] = fmaxf(m[k], __shfl_xor(m[k], sh));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6][k] = m[k];
  }
  __syncthreads();
  if (threadIdx.x < 5)
    part[blockIdx.x * kBoundsWords + threadIdx.x] =
        fmaxf(fmaxf(red[0][threadIdx.x], red[1][threadIdx.x]),
              fmaxf(red[2][threadIdx.x], red[3][threadIdx.x]));
}

// Scales of the fp16 dK / dV accumulators.  A voxel's dV sums p w dO over the
// queries whose taps reach it, and each query's p w sum to at most the dropout
// factor F: |dV| <= n F max|dO| for n such queries.  Its dK sums B q with
// sum_v |B[q][v]| <= sum_k |ds_k scale| <= scale (2 F |dO| max|v| + |dlse_q|)
// (ds_k = p_k (f_k dO.v_k - Delta), v_k a convex combination of V rows,
// |O| <= F max|v|; |.| of dO and v is the L2 norm of the head's slice, by
// Cauchy-Schwarz), so |dK| <= n max|q| times that.  Scaling by 2^14 /
// (kH16Reach bound) keeps every partial sum below the fp16 limit (65504) for up
// to 4 kH16Reach queries' full weight on one voxel.  A sum beyond it (more such
// queries, or maxima above the sampled ones) overflows to infinity: the
// conversion flags it and dK / dV are redone in fp32, so the scales only trade
// redo probability against the values left below fp16's normal range.  They
// are powers of two (unscaling is exact).  Also clears the flag.
constexpr float kH16Reach = 1024.0f;
__global__ __launch_bounds__(256) void h16_scales_kernel(const float* __restrict__ part, int nblk,
                                                         float factor, float softmax_scale,
                                                         float* __restrict__ scales,
                                                         int* __restrict__ flag) {
  float m[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = threadIdx.x; i < nblk; i += 256)
#pragma unroll
    for (int k = 0; k < 5; ++k) m[k] = fmaxf(m[k], part[kBoundsWords * i + k]);
  __shared__ float red[4][5];
#pragma unroll
  for (int k = 0; k < 5; ++k) {
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) m[k] = fmaxf(m[k], __shfl_xor(m[k], sh));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6][k] = m[k];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float r[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) r[k] = fmaxf(fmaxf(red[0][k], red[1][k]), fmaxf(red[2][k], red[3][k]));
    const float l1 = softmax_scale * (2.0f * factor * r[2] * r[3] + r[4]);
    const float sk = h16_pow2_scale(kH16Reach * l1 * r[0]);
    const float sv = h16_pow2_scale(kH16Reach * factor * r[1]);
    scales[0] = sk;
    scales[1] = 1.0f / sk;
    scales[2] = sv;
    scales[3] = 1.0f / sv;
    *flag = 0;
  }
}

// fp16 dK (blockIdx.y 0) or dV (1) rows [rows, D] -> bf16 outputs with their
// token strides, unscaled; a non-finite value (an fp16 overflow, or a
// non-finite input) sets *flag.  8 channels per thread, grid-stride.
__global__ __launch_bounds__(256) void h16_to_bf16_kernel(const _Float16* __restrict__ hk,
                                                         const _Float16* __restrict__ hv,
                                                         bf16* __restrict__ dk,
                                                         bf16* __restrict__ dv, int64_t rows,
                                                         int D, int64_t ks, int64_t vs,
                                                         const float* __restrict__ scales,
                                                         int* __restrict__ flag) {
  typedef __attribute__((ext_vector_type(8))) _Float16 h8_t;
  const int64_t d8 = D / 8, n = rows * d8;
  const bool is_k = blockIdx.y == 0;
  const _Float16* const src0 = is_k ? hk : hv;
  bf16* const dst0 = is_k ? dk : dv;
  const int64_t st = is_k ? ks : vs;
  const float inv = scales[is_k ? 1 : 3];
  bool bad = false;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / d8, c = 8 * (i - r * d8);
    h8_t x;
    __builtin_memcpy(&x, src0 + r * D + c, sizeof(x));
    uint16_t h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = static_cast<float>(x[j]);
      bad |= !__builtin_isfinite(f);
      h[j] = from_f32<bf16>(f * inv).bits;
    }
    __builtin_memcpy(dst0 + r * st + c, h, sizeof(h));
  }
  if (__builtin_amdgcn_ballot_w64(bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(flag, 1);
}

// Zero n floats, only when *flag != 0.  Grid-stride.
__global__ __launch_bounds__(256) void fill_zero_if_flag(float* __restrict__ p, int64_t n,
                                                        const int* __restrict__ flag) {
  if (*flag == 0) return;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0.0f;
}

namespace {
// Frames per tile of the second kernel: 3 for bf16 head_dim 64, 96 and 128
// (at the 131,072-token hd-128 shape three frames in two 64-channel windows
// ran 15% faster than two frames in one window), else 2 (hd 32 would spill).
template <int HD, typename E>
constexpr int p2_frames() {
  return sizeof(E) == 2 && (HD == 64 || HD == 96 || HD == 128) ? 3 : 2;
}

// Channel window of the second backward kernel: the whole head where the LDS
// takes its K^T and q/dO stages beside the tables, else 64 channels (32 for
// fp32 head_dim 96).  bf16 head_dim 96 at three frames stages its K^T in two
// rounds (64 + 32 channels) through one buffer: one window instead of a 64-
// and a 32-channel launch, which repeated the setup, scatter and table work
// (9.8 -> 7.0 ms at the 46,800-token hd-96 shape, 15.8 -> 12.6 ms with
// offsets biased by up to 4 voxels).
template <int HD, typename E>
constexpr int p2_window() {
  if constexpr (sizeof(E) == 2) return HD == 128 ? 64 : HD;
  return HD % 64 == 0 ? 64 : 32;
}

// Buffers of one tiled backward call (workspace carved by tiled_ws).
template <typename E>
struct BwdBufs {
  float* p_ws;     // per tap: p * dropout factor (fp32 storage), or the fp16 pair
                   // (p * factor, ds * softmax_scale / l1) in one word (bf16)
  float* b_ws;     // per tap: ds * softmax_scale (fp32), or per (token, head):
                   // l1 = sum over its taps of |ds * softmax_scale| (bf16)
  void* dk_acc;    // dK / dV accumulator rows: the fp32 outputs (fp32 storage),
  void* dv_acc;    // dk32 / dv32, or scaled fp16 [rows, D] (bf16, MSD_ACCUM_F16)
  int64_t acc_ks, acc_vs;
  bool h16;       // bf16 storage with MSD_ACCUM_F16: scaled fp16 accumulator rows
  float* dk32;     // bf16 storage: fp32 [rows, D] accumulator rows (MSD_ACCUM_F32),
  float* dv32;     // or the redo's rows after an fp16 overflow (the same memory as
                   // the fp16 rows)
  float* bounds;   // bf16 storage: per-block maxima behind the fp16 scales
  float* scales;   // bf16 storage: sK, 1/sK, sV, 1/sV
  int* flag;       // bf16 storage: fp16 overflow seen
  E* ds_e;         // extra keys: ds * scale and p * factor, [B, nh, N, G]
  E* pf_e;
  float* dek_acc;  // extra keys: dEK / dEV fp32 [B, G, D] (the outputs for fp32 storage)
  float* dev_acc;
  float* dqx;      // extra keys: their part of dq, fp32 [rows, D] (null without them)
  float* dlt;      // extra keys: Delta per (token, head), fp32 [rows, nh] (null without them)
  RecArgs rec;     // column-streaming kernel's records (rec.rec null: not used)
};

// CUs of the current device (the column-streaming kernel's persistent grid),
// cached per device; 256 (MI355X) if the query fails.
int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) ==
                              hipSuccess && n > 0
                      ? n
                      : 256;
  }
  return cached[dev];
}

template <int HD, typename E>
void launch_bwd_pair(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v,
                     const void* off, const void* ek, const void* ev, const E* o, const E* go,
                     const float* lse, const float* dlse, E* gq, E* goff, const BwdBufs<E>& w,
                     hipStream_t s) {
  constexpr int CW = p2_window<HD, E>(), FR = p2_frames<HD, E>();
  tiled::Args a1 = make_tiled_args(d, q, k, v, off, tiled_tiles<1>(d), ek, ev);
  a1.dlt = w.dlt;
  const tiled::Args a2 = make_tiled_args(d, q, k, v, off, tiled_tiles<FR>(d), ek, ev);
  const dim3 g1 = tiled_grid<1>(d);
  dim3 g2 = tiled_grid<FR>(d);
  g2.z = HD / CW;
  float* const p_ws = w.p_ws;
  float* const b_ws = w.b_ws;
  void* const dk_acc = w.dk_acc;
  void* const dv_acc = w.dv_acc;
  const int64_t acc_ks = w.acc_ks, acc_vs = w.acc_vs;
  // scaled fp16 accumulation: bf16 storage with MSD_ACCUM_F16 only
  const bool h16 = sizeof(E) == 2 && w.h16;
  // bf16 with fp32 accumulation and no extra keys: the first kernel also
  // writes tap records, the column-streaming kernel takes every column it can
  // and the tile kernel the columns it flags
  if constexpr (sizeof(E) == 2) {
    if (!h16 && w.rec.rec != nullptr) {
      hipLaunchKernelGGL((dsa3d_bwd_p1_kernel<HD, E, 4, true>), g1, dim3(tiled::kThreads), 0, s,
                         a1, o, go, lse, dlse, goff, p_ws, b_ws, dk_acc, dv_acc, acc_ks, acc_vs,
                         w.rec);
      // persistent: one workgroup per CU (each takes a CU's LDS)
      hipLaunchKernelGGL((dsa3d_bwd_p2s_kernel<HD, E>), dim3(device_cus()), dim3(kS2Threads), 0,
                         s, a1, w.rec, b_ws, gq, static_cast<float*>(dk_acc),
                         static_cast<float*>(dv_acc), acc_ks, acc_vs);
      hipLaunchKernelGGL((dsa3d_bwd_p2_list_kernel<HD, CW, E, FR>), dim3(256, 1, HD / CW),
                         dim3(P2Tile<FR>::Threads), 0, s, a2, go, p_ws, b_ws, gq, dk_acc, dv_acc,
                         acc_ks, acc_vs, w.rec.collist);
      return;
    }
  }
  const dim3 gx(static_cast<unsigned>(d.B * ((a1.N + kXQ - 1) / kXQ)), d.num_heads);
  if (d.extra_g > 0)  // the keys' part of Delta, for the first backward kernel
    hipLaunchKernelGGL((dsa3d_bwd_extra_kernel<HD, E, true>), gx, dim3(256), 0, s, a1, go, lse,
                       w.dqx, w.ds_e, w.pf_e);
  if constexpr (sizeof(E) == 2) {
    if (h16)
      hipLaunchKernelGGL((dsa3d_bwd_p1_kernel<HD, E, 2>), g1, dim3(tiled::kThreads), 0, s, a1, o,
                         go, lse, dlse, goff, p_ws, b_ws, dk_acc, dv_acc, acc_ks, acc_vs, RecArgs{});
  }
  if (!h16)
    hipLaunchKernelGGL((dsa3d_bwd_p1_kernel<HD, E, 4>), g1, dim3(tiled::kThreads), 0, s, a1, o,
                       go, lse, dlse, goff, p_ws, b_ws, dk_acc, dv_acc, acc_ks, acc_vs, RecArgs{});
  if (d.extra_g > 0)
    hipLaunchKernelGGL((dsa3d_bwd_extra_kernel<HD, E, false>), gx, dim3(256), 0, s, a1, go, lse,
                       w.dqx, w.ds_e, w.pf_e);
  if constexpr (sizeof(E) == 2) {
    if (h16) {
      const float factor = a1.drop.threshold == 0 ? 1.0f : a1.drop.scale;
      hipLaunchKernelGGL(h16_bounds_kernel, dim3(kBoundsBlocks), dim3(256), 0, s,
                         static_cast<const bf16*>(q), d.q_stride, go, static_cast<const bf16*>(v),
                         d.v_stride, static_cast<const bf16*>(ev), int64_t{d.B} * d.extra_g, dlse,
                         static_cast<int64_t>(a1.N) * d.B, d.num_heads, HD, w.bounds);
      hipLaunchKernelGGL(h16_scales_kernel, dim3(1), dim3(256), 0, s, w.bounds, kBoundsBlocks,
                         factor, d.softmax_scale, w.scales, w.flag);
      hipLaunchKernelGGL((dsa3d_bwd_p2_kernel<HD, CW, E, FR, kP2F16>), g2,
                         dim3(P2Tile<FR>::Threads), 0, s, a2, go, p_ws, b_ws, gq, dk_acc, dv_acc,
                         acc_ks, acc_vs, 0, w.scales, w.dqx);
    }
  }
  if (!h16)
    hipLaunchKernelGGL((dsa3d_bwd_p2_kernel<HD, CW, E, FR, kP2F32>), g2,
                       dim3(P2Tile<FR>::Threads), 0, s, a2, go, p_ws, b_ws, gq, dk_acc, dv_acc,
                       acc_ks, acc_vs, 0, w.scales, w.dqx);
  static_assert(HD % CW == 0, "channel windows tile the head");
  if (d.extra_g > 0) {
    // dEK, dEV: about 1,024 workgroups of token ranges that are multiples of 32
    const int64_t N = static_cast<int64_t>(d.T) * d.H * d.W;
    const int64_t parts = std::max<int64_t>(1, 1024 / (2 * int64_t{d.B} * d.num_heads));
    const int64_t range = ((N + parts - 1) / parts + kXChunk - 1) / kXChunk * kXChunk;
    const dim3 grid(static_cast<unsigned>((N + range - 1) / range), d.B * d.num_heads, 2);
    hipLaunchKernelGGL((extra_grad_kernel<HD, E>), grid, dim3(256), 0, s, w.ds_e, w.pf_e,
                       static_cast<const E*>(q), d.q_stride, go, N, d.num_heads, d.extra_g, range,
                       w.dek_acc, w.dev_acc);
  }
}

// bf16 storage, after an fp16 overflow: dK and dV again into zeroed fp32 rows
// (every kernel returns at once without the flag).
template <int HD, typename E>
void launch_bwd_redo(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v,
                     const void* off, const void* ek, const void* ev, const E* go,
                     const BwdBufs<E>& w, hipStream_t s) {
  constexpr int CW = p2_window<HD, E>(), FR = p2_frames<HD, E>();
  const int64_t tiles = tiled_tiles<FR>(d);
  const tiled::Args a2 = make_tiled_args(d, q, k, v, off, tiles, ek, ev);
  const int64_t rows = static_cast<int64_t>(d.B) * d.T * d.H * d.W;
  const int64_t n = 2 * rows * d.num_heads * HD;  // dK then dV rows, contiguous
  hipLaunchKernelGGL(fill_zero_if_flag, dim3(512), dim3(256), 0, s, w.dk32, n, w.flag);
  // one workgroup per CU over all heads and windows; each strides over the tiles
  const int per = std::max(1, 256 / (d.num_heads * (HD / CW)));
  dim3 g(static_cast<unsigned>(std::min<int64_t>(per, tiles)), d.num_heads, HD / CW);
  hipLaunchKernelGGL((dsa3d_bwd_p2_redo_kernel<HD, CW, E, FR>), g, dim3(P2Tile<FR>::Threads), 0,
                     s, a2, go, w.p_ws, w.b_ws, w.dk32, w.dv32, int64_t{d.num_heads} * HD,
                     int64_t{d.num_heads} * HD, 0, w.flag, static_cast<int>(tiles));
}

// fp32 dK (blockIdx.y 0) or dV (1) accumulator [rows, D] -> bf16 with the
// output's token stride, 8 channels per thread (32-byte loads, 16-byte stores;
// D and the strides are multiples of 8), grid-stride over 64-bit indices.
// With `flag`, only when *flag != 0.
__global__ __launch_bounds__(256) void acc_to_bf16_kernel(const float* __restrict__ dk_acc,
                                                         const float* __restrict__ dv_acc,
                                                         bf16* __restrict__ dk,
                                                         bf16* __restrict__ dv, int64_t rows,
                                                         int D, int64_t ks, int64_t vs,
                                                         const int* __restrict__ flag) {
  if (flag != nullptr && *flag == 0) return;
  const int64_t d8 = D / 8, n = rows * d8;
  const bool is_k = blockIdx.y == 0;
  const float* const src0 = is_k ? dk_acc : dv_acc;
  bf16* const dst0 = is_k ? dk : dv;
  const int64_t st = is_k ? ks : vs;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / d8, c = 8 * (i - r * d8);
    f32x4_t x[2];
    __builtin_memcpy(x, src0 + r * D + c, sizeof(x));
    uint16_t h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = from_f32<bf16>(x[j / 4][j % 4]).bits;
    __builtin_memcpy(dst0 + r * st + c, h, sizeof(h));
  }
}

// Workspace layout of the tiled backward (byte offsets): the bf16 path's fp32
// accumulators (dK/dV, then dEK/dEV; fp32 storage accumulates in its outputs),
// p and ds * scale per tap, and with extra keys their ds * scale and p *
// factor per (token, head, key) in the element type, their fp32 part of dq
// and the fp32 Delta per (token, head).
// For bf16 storage the dK / dV region holds the fp32 [2, rows, D] accumulator
// rows; with MSD_ACCUM_F16 its first half serves as the fp16 [2, rows, D]
// accumulator (the fp32 rows are then only used, zeroed first, after that has
// been converted, for the redo after an overflow), and the bounds kernel's
// per-block maxima, the two scales and their inverses and the overflow flag
// follow the extra keys' buffers.
struct TiledWs {
  size_t acc, xacc, p, ds, dse, pfe, dqx, dlt, stats, scales, rec, hdr, qt, collist, bytes;
};

// Calls that take the column-streaming dq/dK/dV kernel: bf16 storage with fp32
// dK/dV accumulation and no extra keys.
bool tiled_streams(const msd_dsa3d_desc& d) {
  return d.dtype == MSD_BF16 && d.dkv_accum == MSD_ACCUM_F32 && d.extra_g == 0;
}

TiledWs tiled_ws(const msd_dsa3d_desc& d) {
  const size_t rows = static_cast<size_t>(d.B) * d.T * d.H * d.W;
  const size_t D = static_cast<size_t>(d.num_heads) * d.head_dim;
  const size_t taps = rows * d.num_heads * d.kt * d.kh * d.kw;
  const size_t G = static_cast<size_t>(d.extra_g);
  const bool bf = d.dtype == MSD_BF16;
  const size_t e = bf ? 2 : 4;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  TiledWs w;
  w.acc = 0;
  w.xacc = w.acc + (bf ? 2 * rows * D * 4 : 0);
  w.p = w.xacc + (bf ? 2 * static_cast<size_t>(d.B) * G * D * 4 : 0);
  w.ds = w.p + taps * 4;
  w.dse = up(w.ds + (bf ? rows * d.num_heads * 4 : taps * 4));
  w.pfe = up(w.dse + rows * d.num_heads * G * e);
  w.dqx = up(w.pfe + rows * d.num_heads * G * e);
  w.dlt = up(w.dqx + (G > 0 ? rows * D * 4 : 0));
  w.stats = up(w.dlt + (G > 0 ? rows * d.num_heads * 4 : 0));
  w.scales = up(w.stats + (bf ? kBoundsBlocks * kBoundsWords * 4 : 0));
  // column-streaming kernel: records, tile headers, transposed q / dO, flags
  const bool st = tiled_streams(d);
  const size_t tiles = static_cast<size_t>(d.B) * d.T * ((d.H + tiled::kTileH - 1) / tiled::kTileH) *
                       ((d.W + tiled::kTileW - 1) / tiled::kTileW) * d.num_heads;
  const size_t cols = static_cast<size_t>(d.B) * ((d.H + tiled::kTileH - 1) / tiled::kTileH) *
                      ((d.W + tiled::kTileW - 1) / tiled::kTileW) * d.num_heads;
  const size_t K = static_cast<size_t>(d.kt) * d.kh * d.kw;
  w.rec = w.hdr = w.qt = w.collist = w.bytes = w.scales + (bf ? 32 : 0);
  if (st) {
    w.rec = up(w.bytes);
    w.hdr = up(w.rec + tiles * K * tiled::kTQ * 16);
    w.qt = up(w.hdr + tiles * tiled::kRecHdr * 4);
    w.collist = up(w.qt + tiles * 2 * d.head_dim * tiled::kTQ * e);
    w.bytes = w.collist + (cols + 1 + 8) * 4;  // count, list, 8 work counters
  }
  return w;
}

template <typename E>
hipError_t bwd_tiled_typed(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v,
                           const void* off, const void* ek, const void* ev, const void* out,
                           const void* dout, const float* lse, const float* dlse, void* dq,
                           void* dk, void* dv, void* doff, void* dek, void* dev, void* ws,
                           hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(d.B) * d.T * d.H * d.W;
  const int D = d.num_heads * d.head_dim;
  const int64_t erows = static_cast<int64_t>(d.B) * d.extra_g;
  const auto* o = static_cast<const E*>(out);
  const auto* go = static_cast<const E*>(dout);
  auto* gq = static_cast<E*>(dq);
  auto* goff = static_cast<E*>(doff);
  char* const base = static_cast<char*>(ws);
  const TiledWs L = tiled_ws(d);
  // fp32 storage: dK and dV (and dEK, dEV) add up in the outputs themselves.
  // bf16 storage: dK and dV in fp32 rows, or with MSD_ACCUM_F16 in scaled fp16
  // rows (fp32 again if that overflows); dEK and dEV in fp32 accumulators;
  // converted at the end.
  constexpr bool kInPlace = sizeof(E) == 4;
  BwdBufs<E> w;
  w.h16 = !kInPlace && d.dkv_accum == MSD_ACCUM_F16;
  w.p_ws = reinterpret_cast<float*>(base + L.p);
  w.b_ws = reinterpret_cast<float*>(base + L.ds);
  w.dk32 = kInPlace ? nullptr : reinterpret_cast<float*>(base + L.acc);
  w.dv32 = kInPlace ? nullptr : w.dk32 + rows * D;
  w.dk_acc = kInPlace ? dk : w.h16 ? static_cast<void*>(base + L.acc) : w.dk32;
  w.dv_acc = kInPlace ? dv : w.h16 ? static_cast<void*>(base + L.acc + rows * D * 2) : w.dv32;
  w.acc_ks = kInPlace ? d.k_stride : D;
  w.acc_vs = kInPlace ? d.v_stride : D;
  w.bounds = kInPlace ? nullptr : reinterpret_cast<float*>(base + L.stats);
  w.scales = kInPlace ? nullptr : reinterpret_cast<float*>(base + L.scales);
  w.flag = kInPlace ? nullptr : reinterpret_cast<int*>(base + L.scales + 16);
  w.ds_e = reinterpret_cast<E*>(base + L.dse);
  w.pf_e = reinterpret_cast<E*>(base + L.pfe);
  w.dek_acc = kInPlace ? static_cast<float*>(dek) : reinterpret_cast<float*>(base + L.xacc);
  w.dev_acc = kInPlace ? static_cast<float*>(dev) : w.dek_acc + erows * D;
  w.dqx = erows > 0 ? reinterpret_cast<float*>(base + L.dqx) : nullptr;
  w.dlt = erows > 0 ? reinterpret_cast<float*>(base + L.dlt) : nullptr;
  w.rec = RecArgs{};
  if (tiled_streams(d)) {
    w.rec.rec = reinterpret_cast<tiled::u32x4_t*>(base + L.rec);
    w.rec.hdr = reinterpret_cast<int*>(base + L.hdr);
    w.rec.qt = base + L.qt;
    w.rec.collist = reinterpret_cast<int*>(base + L.collist);
    w.rec.tiles = tiled_tiles<1>(d);
  }
  if (erows > 0) {
    hipLaunchKernelGGL(fill_zero_f32, dim3(fill_blocks(erows * D)), dim3(256), 0, s, w.dek_acc,
                       erows * D);
    hipLaunchKernelGGL(fill_zero_f32, dim3(fill_blocks(erows * D)), dim3(256), 0, s, w.dev_acc,
                       erows * D);
  }
  switch (d.head_dim) {
    case 32: launch_bwd_pair<32, E>(d, q, k, v, off, ek, ev, o, go, lse, dlse, gq, goff, w, s); break;
    case 64: launch_bwd_pair<64, E>(d, q, k, v, off, ek, ev, o, go, lse, dlse, gq, goff, w, s); break;
    case 96: launch_bwd_pair<96, E>(d, q, k, v, off, ek, ev, o, go, lse, dlse, gq, goff, w, s); break;
    case 128: launch_bwd_pair<128, E>(d, q, k, v, off, ek, ev, o, go, lse, dlse, gq, goff, w, s); break;
    default: return hipErrorInvalidValue;
  }
  if constexpr (!kInPlace) {
    const dim3 cgrid(fill_blocks(rows * (D / 8)), 2);
    if (!w.h16) {
      hipLaunchKernelGGL(acc_to_bf16_kernel, cgrid, dim3(256), 0, s, w.dk32, w.dv32,
                         static_cast<bf16*>(dk), static_cast<bf16*>(dv), rows, D, d.k_stride,
                         d.v_stride, static_cast<const int*>(nullptr));
    } else {
      hipLaunchKernelGGL(h16_to_bf16_kernel, cgrid, dim3(256), 0, s,
                         static_cast<const _Float16*>(w.dk_acc), static_cast<const _Float16*>(w.dv_acc),
                         static_cast<bf16*>(dk), static_cast<bf16*>(dv), rows, D, d.k_stride,
                         d.v_stride, w.scales, w.flag);
      // after an fp16 overflow (flag set): dK and dV again in fp32
      switch (d.head_dim) {
        case 32: launch_bwd_redo<32, E>(d, q, k, v, off, ek, ev, go, w, s); break;
        case 64: launch_bwd_redo<64, E>(d, q, k, v, off, ek, ev, go, w, s); break;
        case 96: launch_bwd_redo<96, E>(d, q, k, v, off, ek, ev, go, w, s); break;
        default: launch_bwd_redo<128, E>(d, q, k, v, off, ek, ev, go, w, s); break;
      }
      // grid-stride: a small grid keeps the launch cheap when there is nothing to do
      hipLaunchKernelGGL(acc_to_bf16_kernel, dim3(std::min(cgrid.x, 1024u), 2), dim3(256), 0, s,
                         w.dk32, w.dv32, static_cast<bf16*>(dk), static_cast<bf16*>(dv), rows, D,
                         d.k_stride, d.v_stride, static_cast<const int*>(w.flag));
    }
    if (erows > 0) {
      const dim3 egrid(fill_blocks(erows * (D / 8)), 2);
      hipLaunchKernelGGL(acc_to_bf16_kernel, egrid, dim3(256), 0, s, w.dek_acc, w.dev_acc,
                         static_cast<bf16*>(dek), static_cast<bf16*>(dev), erows, D,
                         static_cast<int64_t>(D), static_cast<int64_t>(D),
                         static_cast<const int*>(nullptr));
    }
  }
  return hipGetLastError();
}
}  // namespace

// Workspace of the tiled backward (the layout of tiled_ws).
size_t dsa3d_tiled_bwd_ws_bytes(const msd_dsa3d_desc& d) {
  if ((d.dtype != MSD_BF16 && d.dtype != MSD_F32) || !tiled_head_dim(d.head_dim) ||
      d.kt * d.kh * d.kw > tiled::kMaxTaps || d.extra_g > tiled::kMaxExtra)
    return 0;
  return tiled_ws(d).bytes;
}

hipError_t launch_dsa3d_bwd_tiled(const msd_dsa3d_desc& d, const void* q, const void* k,
                                  const void* v, const void* off, const void* ek, const void* ev,
                                  const void* out, const void* dout, const float* lse,
                                  const float* dlse, void* dq, void* dk, void* dv, void* doff,
                                  void* dek, void* dev, void* ws, hipStream_t s) {
  if (d.dtype == MSD_BF16)
    return bwd_tiled_typed<bf16>(d, q, k, v, off, ek, ev, out, dout, lse, dlse, dq, dk, dv, doff,
                                 dek, dev, ws, s);
  return bwd_tiled_typed<float>(d, q, k, v, off, ek, ev, out, dout, lse, dlse, dq, dk, dv, doff,
                                dek, dev, ws, s);
}

}  // namespace msd
