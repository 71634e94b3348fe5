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
#include "dsa3d_tiled_common.h"

namespace msd {

namespace {

using namespace tiled;

// The S (pass 1) and A (pass 2) tables are double-buffered where that keeps
// the workgroups per CU: a step's table is written while the other buffer may
// still be read for the previous step, so pass 1 needs one barrier per step and
// pass 2 two (instead of two and three).  bf16 head_dim 96 keeps one buffer:
// two would drop it to one workgroup per CU (measured 30% slower).  bf16
// head_dim 128 and every fp32 head stage too much V^T for two workgroups per
// CU; they run one, with the register cap raised to match.
constexpr int kLdsBytes = 160 * 1024;
constexpr int kTabBytes = kTQ * kSRow * 4;

template <int HD, typename E>
constexpr int fwd_vt_bytes() {
  return HD * ElemT<E>::kRow * static_cast<int>(sizeof(word_t<E>));
}

template <int HD, typename E>
constexpr int fwd_table_bufs() {
  constexpr int vt = fwd_vt_bytes<HD, E>();
  if (2 * (2 * kTabBytes + vt) <= kLdsBytes) return 2;  // two workgroups per CU
  if (2 * (kTabBytes + vt) <= kLdsBytes) return 1;      // two workgroups per CU
  return 2 * kTabBytes + vt <= kLdsBytes ? 2 : 1;       // one workgroup per CU
}

// Minimum waves per SIMD: 4 when two 512-thread workgroups fit in a CU's LDS
// (bf16; the fp32 operands need more than 128 registers).
template <int HD, typename E>
constexpr int fwd_min_waves() {
  if constexpr (sizeof(E) == 4) return 2;
  return 2 * (fwd_table_bufs<HD, E>() * kTabBytes + fwd_vt_bytes<HD, E>()) <= kLdsBytes ? 4 : 2;
}

// Slot words as used in the forward's plane loops: at head_dim 96 (128
// registers at 4 waves/SIMD) opaque, which stops the hoisting that spilled
// (10% faster); elsewhere the hoisted keys and weights are cheaper (5%).
template <int HD>
__device__ __forceinline__ Slot fwd_slot(const Slot& s) {
  if constexpr (HD == 96) return opaque(s);
  return s;
}

template <int HD, typename E>
__global__ __launch_bounds__(kThreads, (fwd_min_waves<HD, E>())) void dsa3d_fwd_tiled_kernel(
    Args a, E* __restrict__ out, float* __restrict__ lse) {
  constexpr int NB = fwd_table_bufs<HD, E>();
  constexpr int VR = ElemT<E>::kRow;
  __shared__ __attribute__((aligned(16))) float s_tab[NB][kTQ * kSRow];  // S, then A
  __shared__ __attribute__((aligned(16))) word_t<E> s_vt[HD * VR];      // V^T chunk
  __shared__ int s_red[kWaves][6];

  const Tile tl = make_tile<1, kSubs>(a);
  Slot sl[kSlots];
  Box box;
  setup_slots<E, kSubs, kSlots>(a, tl, sl, box, s_red, true);
  const int nchunks = box.ncy * box.ncx;
  const int nit = (box.zhi - box.zlo + 1) * nchunks;
  const E* const kp = static_cast<const E*>(a.k);
  const E* const vp = static_cast<const E*>(a.v);

  op_t<E> qx[HD / 32];
  load_rows_operand<HD, E>(a, tl, static_cast<const E*>(a.q), a.qs, qx);

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

  // ---- softmax over each query's taps (32 lanes x kSlots) -------------------
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    sc[i] = slot_z0(sl[i]) >= 0 ? sc[i] * a.softmax_scale : -INFINITY;
    mx = fmaxf(mx, sc[i]);
  }
#pragma unroll
  for (int m = 1; m < kSubs; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  float den = 0.0f;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    sc[i] = slot_z0(sl[i]) >= 0 ? __expf(sc[i] - mx) : 0.0f;
    den += sc[i];
  }
#pragma unroll
  for (int m = 1; m < kSubs; m <<= 1) den += __shfl_xor(den, m);
  const float inv_den = 1.0f / den;
#pragma unroll
  for (int i = 0; i < kSlots; ++i)
    sc[i] *= inv_den * slot_dropout(sl[i], a.drop) * a.fix_a;  // p (dropped), fixed-point units
  if (lse != nullptr && tl.q_ok && tl.sub == 0) lse[tl.qn * a.nh + tl.head] = mx + logf(den);

  // ---- pass 2: O = A . V ------------------------------------------------------
  // The waves form CG channel groups of KP waves; wave w of group g takes the
  // voxel k-steps w % KP, + KP, ... of a step for the TPW channel tiles of
  // group g: one A operand feeds TPW independent MFMAs, and the KP partial O
  // are summed once at the end.  hd 64 and 128: one group of 8 waves (fp32
  // hd 128: two groups of 4, for registers).  hd 96: six single-tile groups
  // (waves 6, 7 idle), which stays within 128 registers and measured faster
  // than groups of several tiles.
  constexpr int CT = HD / 16, CG = HD == 96 ? CT : (sizeof(E) == 4 && HD == 128 ? 2 : 1);
  constexpr int TPW = CT / CG, KP = HD == 96 ? 1 : kWaves / CG;
  static_assert(TPW * CG == CT && CG * KP <= kWaves, "channel tiles split over the waves");
  const int mq = tl.lane & 15, kq = 8 * (tl.lane >> 4);
  const int cg = tl.wave / KP, kph = tl.wave % KP;
  const bool av_wave = tl.wave < CG * KP;
  f32x4_t oacc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) oacc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  StageRows<kThreads, HD, E> vr;
  w = walk_begin(box);
  if (nit > 0) load_stage_rows<kThreads, HD, E>(a, tl, w.c, w.z, vp, a.vs, tl.head * HD, vr);
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
    store_stage<kThreads, HD, E>(c, vr, s_vt);
    if (it + 1 < nit)
      load_stage_rows<kThreads, HD, E>(a, tl, wn.c, wn.z, vp, a.vs, tl.head * HD, vr);
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const Slot si = fwd_slot<HD>(sl[i]);
      float wz, dwz;
      if (!slot_hits(si, step_key(c.id, z), wz, dwz)) continue;
      const float pz = sc[i] * wz;
      const float gx = 1.0f - si.fx, gy = 1.0f - si.fy;
      const int base = si.idx & 0x1ff, dy = (si.idx >> 9) & 0x1f, dx = (si.idx >> 14) & 1;
      // an upper corner outside the volume has offset 0 and weight 0: it adds 0
      // to the lower corner, so all four adds run without branches
      atomicAdd(&row[base], to_fix(pz * (gy * gx)));
      atomicAdd(&row[base + dx], to_fix(pz * (gy * si.fx)));
      atomicAdd(&row[base + dy], to_fix(pz * (si.fy * gx)));
      atomicAdd(&row[base + dy + dx], to_fix(pz * (si.fy * si.fx)));
    }
    __syncthreads();
    for (int kc = 32 * kph; av_wave && kc < c.nvp; kc += 32 * KP) {
      const op_t<E> av = fix_to_op<E>(&s_atab[mq * kSRow + kc + kq]);
#pragma unroll
      for (int t = 0; t < TPW; ++t)
        oacc[t] = mma16(av, load_op<E>(&s_vt[(16 * (cg * TPW + t) + mq) * VR + kc + kq]), oacc[t]);
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
  static_assert(KP * kTQ * HD * 4 <= fwd_vt_bytes<HD, E>(), "partials fit the V^T buffer");
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
      out[n * (static_cast<int64_t>(a.nh) * HD) + tl.head * HD + ch] = from_f32<E>(o * a.fix_a_inv);
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
// Waves per SIMD of the first backward kernel.  bf16 up to head_dim 64 fits
// 128 registers, so two workgroups share a CU and each hides the other's
// latencies (barriers, table loads): q and dO then stay in LDS and K/V rows are
// loaded at the step.  Larger heads and fp32 keep q/dO in registers and
// prefetch the next step's rows, at one workgroup per CU.
template <int HD, typename E>
constexpr int p1_min_waves() {
  return sizeof(E) == 2 && HD <= 96 ? 4 : 2;
}

template <int HD, typename E>
__global__ __launch_bounds__(kThreads, (p1_min_waves<HD, E>())) void dsa3d_bwd_p1_kernel(
    Args a, const E* __restrict__ out, const E* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ dlse, E* __restrict__ doff,
    float* __restrict__ p_ws, float* __restrict__ b_ws, float* __restrict__ dk_acc,
    float* __restrict__ dv_acc, int64_t acc_ks, int64_t acc_vs) {
  // S and dP tables, double-buffered (one barrier per plane).  A buffer is
  // [S rows | zeros | dP rows | zeros]: a slot that misses the step reads the
  // zero block instead of its corners, so its values are 0 with no select, and
  // dP sits a constant kP1Tab floats past S (immediate offsets on the reads).
  __shared__ __attribute__((aligned(16))) float s_tb[2][2 * kP1Tab];
  __shared__ int s_red[kWaves][6];
  constexpr bool kTwoWg = p1_min_waves<HD, E>() == 4;
  constexpr int XR = HD + 8;  // [query][channel] row of the staged q and dO (elements)
  __shared__ __attribute__((aligned(16))) word_t<E> s_x[kTwoWg ? 2 * kTQ * XR : 1];

  const Tile tl = make_tile<1, kSubs>(a);
  const int D = a.nh * HD;
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
    // The second kernel adds dK and dV into fp32 rows (the outputs for fp32
    // storage, an accumulator for bf16): zero this tile's rows of the head first
    // (the tiles of a launch partition the (token, head) pairs, and the second
    // kernel starts after this one ends), 16 bytes a thread.
    constexpr int CPR = HD / 4;
    for (int e = threadIdx.x; e < 2 * kTQ * CPR; e += kThreads) {
      const int t = e / (kTQ * CPR), m = (e / CPR) % kTQ, ch = (e % CPR) * 4;
      const int64_t row = tile_row(a, tl, m);
      if (row < 0) continue;
      float* dst = (t == 0 ? dk_acc + row * acc_ks : dv_acc + row * acc_vs) + tl.head * HD + ch;
      *reinterpret_cast<uint4*>(dst) = uint4{0u, 0u, 0u, 0u};
    }
  }

  op_t<E> qx[HD / 32], gx[HD / 32];
  if constexpr (kTwoWg) {
    // q (t = 0) and dO (t = 1) rows of the tile's queries into LDS, 16 bytes a thread
    constexpr int CPR = HD * static_cast<int>(sizeof(E)) / 16;
    for (int e = threadIdx.x; e < 2 * kTQ * CPR; e += kThreads) {
      const int t = e / (kTQ * CPR), m = (e / CPR) % kTQ, ch = (e % CPR) * (16 / sizeof(E));
      const int64_t row = tile_row(a, tl, m);
      uint4 v = {0u, 0u, 0u, 0u};
      if (row >= 0) {
        const E* src = t == 0 ? static_cast<const E*>(a.q) + row * a.qs : dout + row * D;
        v = *reinterpret_cast<const uint4*>(src + tl.head * HD + ch);
      }
      *reinterpret_cast<uint4*>(&s_x[(t * kTQ + m) * XR + ch]) = v;
    }
    __syncthreads();
  } else {
    load_rows_operand<HD, E>(a, tl, static_cast<const E*>(a.q), a.qs, qx);
    load_rows_operand<HD, E>(a, tl, dout, D, gx);
  }
  // MFMA A operand of staged row block t (q or dO): lane l holds channels
  // 32 c + 8 (l / 16) + [0, 8) of query l % 16
  auto staged_x = [&](int t, op_t<E> (&x)[HD / 32]) {
#pragma unroll
    for (int cc = 0; cc < HD / 32; ++cc)
      x[cc] = load_op<E>(&s_x[(t * kTQ + (tl.lane & 15)) * XR + 32 * cc + 8 * (tl.lane >> 4)]);
  };

  // Delta = dO . O (- dlse) and lse for this lane's query: 32 lanes x HD/32 channels
  constexpr int CPL = HD / kSubs;
  float delta = 0.0f, lse_q = 0.0f;
  if (tl.q_ok) {
    const int64_t base = tl.qn * D + tl.head * HD + CPL * tl.sub;
#pragma unroll
    for (int j = 0; j < CPL; ++j) delta += to_f32(dout[base + j]) * to_f32(out[base + j]);
    lse_q = lse[tl.qn * a.nh + tl.head];
  }
#pragma unroll
  for (int m = 1; m < kSubs; m <<= 1) delta += __shfl_xor(delta, m);
  if (dlse != nullptr && tl.q_ok) delta -= dlse[tl.qn * a.nh + tl.head];

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
  const float cxs = 0.5f * a.W * a.rdiv_x * a.offset_scale;
  const float cys = 0.5f * a.H * a.rdiv_y * a.offset_scale;
  const float czs = 0.5f * a.T * a.rdiv_z * a.offset_scale;
  const int64_t tap0 = (tl.qn * a.nh + tl.head) * a.K;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    if (slot_z0(sl[i]) < 0) continue;
    const float pi = __expf(s_[i] * a.softmax_scale - lse_q);
    // dropout: o sums pd * v_s with pd = p * factor, so dp and the V-side
    // coordinate gradient see the factor
    const float dfac = slot_dropout(sl[i], a.drop);
    const float pd = pi * dfac;
    const float dss = pi * (dfac * dp_[i] - delta) * a.softmax_scale;
    const int kap = tl.sub + kSubs * i;
    p_ws[tap0 + kap] = pd;
    b_ws[tap0 + kap] = dss;
    E* dp = doff + tl.qn * a.C + (static_cast<int64_t>(tl.head) * a.K + kap) * 3;
    const int m = sl[i].zc >> 17;
    dp[0] = from_f32<E>((m & 1) ? (dss * gxs[i] + pd * gxd[i]) * cxs : 0.0f);
    dp[1] = from_f32<E>((m & 2) ? (dss * gys[i] + pd * gyd[i]) * cys : 0.0f);
    dp[2] = from_f32<E>((m & 4) ? (dss * gzs[i] + pd * gzd[i]) * czs : 0.0f);
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

template <int HD, int CW, typename E, int FR>
__global__ __launch_bounds__(P2Tile<FR>::Threads) void dsa3d_bwd_p2_kernel(
    Args a, const E* __restrict__ dout, const float* __restrict__ p_ws,
    const float* __restrict__ b_ws, E* __restrict__ dq, float* __restrict__ dk_acc,
    float* __restrict__ dv_acc, int64_t acc_ks, int64_t acc_vs, int cw_base) {
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
  __shared__ __attribute__((aligned(16))) word_t<E> s_kt[CW * KR];      // K^T chunk
  // per voxel: its token row within the sample
  __shared__ __attribute__((aligned(16))) int s_rows[kChunkNV];
  __shared__ int s_red[NW][6];
  __shared__ __attribute__((aligned(16))) float s_binv[kP2Q];  // per query: 1 / fixed-point scale of B
  // the tile's q and dO rows of this window, transposed: [tensor][channel][query]
  __shared__ __attribute__((aligned(16))) word_t<E> s_qt[2][CW][QR];

  const Tile tl = make_tile<kP2Frames, kP2Subs>(a);
  const int D = a.nh * HD;
  // first channel of the window: cw_base + CW blockIdx.z within the head
  const int cw0 = tl.head * HD + cw_base + CW * static_cast<int>(blockIdx.z);
  Slot sl[kP2Slots];
  Box box;
  setup_slots<E, kP2Subs, kP2Slots, NW>(a, tl, sl, box, s_red);
  const int nchunks = box.ncy * box.ncx;
  const int nit = (box.zhi - box.zlo + 1) * nchunks;

  float p[kP2Slots], bsc[kP2Slots];
  const int64_t tap0 = (tl.qn * a.nh + tl.head) * a.K;
#pragma unroll
  for (int i = 0; i < kP2Slots; ++i) {
    p[i] = bsc[i] = 0.0f;
    if (slot_z0(sl[i]) < 0) continue;
    const int kap = tl.sub + kP2Subs * i;
    p[i] = p_ws[tap0 + kap];
    bsc[i] = b_ws[tap0 + kap];
  }
  // fixed-point scale of this query's B entries: 2^30 / sum_k |ds_k scale|
  float l1 = 0.0f;
#pragma unroll
  for (int i = 0; i < kP2Slots; ++i) l1 += fabsf(bsc[i]);
#pragma unroll
  for (int m = 1; m < kP2Subs; m <<= 1) l1 += __shfl_xor(l1, m);
  const bool l1_ok = l1 > 1e-30f;
  const float bscale = l1_ok ? kFixA / l1 : 0.0f;
  if (tl.sub == 0) s_binv[tl.q] = l1_ok ? l1 * kFixAInv : 0.0f;
  // p and ds scale in fixed-point units from here on
#pragma unroll
  for (int i = 0; i < kP2Slots; ++i) {
    p[i] *= a.fix_a;
    bsc[i] *= bscale;
  }
  __syncthreads();
  // stage q and dO of the tile transposed, carrying the fixed-point scales of
  // B (per query) and A (1 / fix_a) for the dK/dV products: item e moves 8
  // channels of one row
  for (int e = threadIdx.x; e < 2 * kP2Q * (CW / 8); e += NT) {
    const int cg = e % (CW / 8), m = (e / (CW / 8)) % kP2Q, tensor = e / (kP2Q * (CW / 8));
    const int64_t n = tile_row(a, tl, m);
    op_t<E> x = zero_op<E>();
    if (n >= 0) {
      const E* src = tensor == 0 ? static_cast<const E*>(a.q) + n * a.qs : dout + n * D;
      x = load_op<E>(src + cw0 + 8 * cg);
    }
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

  // dq (16x16x32 MFMA).  CW = 64 (and 32 at three frames): wave w takes
  // frame w / 4 and the voxel k-steps w % 4, + 4, ... for all CT channel
  // tiles, so one converted B
  // operand feeds CT MFMA pairs; the 4 partial dq are summed at the end.
  // Wider windows (registers): task t = (frame t / CT, channels 16*(t % CT) +
  // [0, 16)) for t = w + 8 j over all k-steps.  dK/dV (32x32x16 MFMA, one per
  // frame): task t = (channels 32*(t % NC2) + [0, 32), 32-voxel block t / NC2)
  // for t = w + 8 i.
  constexpr int CT = CW / 16, NC2 = CW / 32;
  constexpr bool DQK = CW == 64 || (CW == 32 && FR == 3);  // k-split dq
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
  // K rows of the next (plane, chunk) are loaded while the current one is used,
  // except with three frames, whose registers are too few to keep them live
  // across the step (the kernel is atomic-bound there anyway)
  constexpr bool kPrefetchK = FR == 2;
  StageRows<kP2Stage, CW, E> kr;
  Walk w = walk_begin(box);
  if (kPrefetchK && nit > 0) load_stage_rows<kP2Stage, CW, E>(a, tl, w.c, w.z, kp, a.ks, cw0, kr);
  for (int it = 0; it < nit; ++it) {
    const Walk wn = walk_next(box, w);
    const Chunk& c = w.c;
    const int z = w.z;
    if (!kPrefetchK) load_stage_rows<kP2Stage, CW, E>(a, tl, c, z, kp, a.ks, cw0, kr);
    // zero the transposed A and B tables; token rows of the chunk's voxels
    for (int e = threadIdx.x; e < c.nvp * kP2Row / 4; e += NT) {
      const u32x4_t zz = {0u, 0u, 0u, 0u};
      __builtin_memcpy(&s_at[4 * e], &zz, sizeof(zz));
      __builtin_memcpy(&s_bt[4 * e], &zz, sizeof(zz));
    }
    for (int vi = threadIdx.x; vi < c.nv; vi += NT)
      s_rows[vi] = static_cast<int>(chunk_row(a, tl, c, z, vi) - tl.sample0);
    store_stage<kP2Stage, CW, E>(c, kr, s_kt);
    if (kPrefetchK && it + 1 < nit)
      load_stage_rows<kP2Stage, CW, E>(a, tl, wn.c, wn.z, kp, a.ks, cw0, kr);
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
    __syncthreads();
    // dq[q] += sum_v B[q][v] K[v]; in bf16, B as a hi/lo pair because
    // sum_v B[q][v] = 0 and K may carry a large common part
    if constexpr (DQK) {
      const int fq = tl.wave / KPQ;
      for (int kc = 32 * (tl.wave % KPQ); kc < c.nvp; kc += 32 * KPQ) {
        float bq[8];  // fixed-point units; the query's scale is applied to dq at the end
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          bq[jj] = static_cast<float>(s_bt[(kc + kq + jj) * kP2Row + kTQ * fq + mq]);
        const PreciseOp<E> bp = precise_op<E>(bq);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          dq_acc[ct] = mma16(bp, load_op<E>(&s_kt[(16 * ct + mq) * KR + kc + kq]), dq_acc[ct]);
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
      flush_block(tl, acc, s_rows, vb, c.nv, cw0 + och, dk_acc, acc_ks);
      acc = f32x16_t{};
#pragma unroll
      for (int f = 0; f < kP2Frames; ++f)
        acc = mma32(table_t_rows<E>(s_at, kP2Row, kTQ * f, vb, tl.lane),
                    load_op<E>(&s_qt[1][och][kTQ * f + oq]), acc);
      flush_block(tl, acc, s_rows, vb, c.nv, cw0 + och, dv_acc, acc_vs);
    }
    __syncthreads();
    w = wn;
  }
  if constexpr (DQK) {
    // dq_acc[ct][r] = partial dq[query 16*fq + 4*(lane/16) + r][channel 16*ct +
    // lane%16] of k phase w % 4; the A^T table (free after the loop's last
    // barrier) takes the partials, and every thread sums 4 for its outputs
    float* red = reinterpret_cast<float*>(s_at);  // [frame][k phase][16][CW]
    static_assert(NW * kTQ * CW <= kChunkNV * kP2Row, "partials fit the A^T table");
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
      if (n >= 0) dq[n * a.qs + cw0 + ch] = from_f32<E>(v * s_binv[m]);
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
        if (n >= 0) dq[n * a.qs + cw0 + 16 * ct + mq] = from_f32<E>(dq_acc[j][r] * s_binv[m]);
      }
    }
  }
}

}  // namespace

// Kernel arguments for a launch over `tiles` workgroups per head.
tiled::Args make_tiled_args(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v,
                            const void* off, int64_t tiles) {
  tiled::Args a;
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
  if (d.kt * d.kh * d.kw > tiled::kMaxTaps) return false;
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
  switch (d.head_dim) {
    case 32: hipLaunchKernelGGL((dsa3d_fwd_tiled_kernel<32, E>), grid, block, 0, s, a, o, lse); break;
    case 64: hipLaunchKernelGGL((dsa3d_fwd_tiled_kernel<64, E>), grid, block, 0, s, a, o, lse); break;
    case 96: hipLaunchKernelGGL((dsa3d_fwd_tiled_kernel<96, E>), grid, block, 0, s, a, o, lse); break;
    case 128: hipLaunchKernelGGL((dsa3d_fwd_tiled_kernel<128, E>), grid, block, 0, s, a, o, lse); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_dsa3d_fwd_tiled(const msd_dsa3d_desc& d, const void* q, const void* k,
                                  const void* v, const void* off, void* out, float* lse,
                                  hipStream_t s) {
  const tiled::Args a = make_tiled_args(d, q, k, v, off, tiled_tiles<1>(d));
  if (d.dtype == MSD_BF16) return fwd_tiled_typed<bf16>(d, a, out, lse, s);
  return fwd_tiled_typed<float>(d, a, out, lse, s);
}

namespace {
// Frames per tile of the second kernel: 3 for bf16 head_dim 64 and 128 (at
// the 131,072-token hd-128 shape three frames in two 64-channel windows ran
// 15% faster than two frames in one window), else 2 (bf16 hd 96 would need
// three 32-channel windows for three frames: 8% slower; hd 32 would spill).
template <int HD, typename E>
constexpr int p2_frames() {
  return sizeof(E) == 2 && (HD == 64 || HD == 96 || HD == 128) ? 3 : 2;
}

// Channel window of the second backward kernel: the whole head where the LDS
// takes its K^T and q/dO stages beside the tables, else 64 channels (32 for
// fp32 head_dim 96).  bf16 head_dim 96 at three frames runs a 64- and a
// 32-channel window (two launches): 8% faster than two frames over the whole
// head at the 46,800-token DiT-block shape.
template <int HD, typename E>
constexpr int p2_window() {
  if constexpr (sizeof(E) == 2) return p2_frames<HD, E>() == 3 && HD > 64 ? 64 : HD;
  return HD % 64 == 0 ? 64 : 32;
}

template <int HD, typename E>
void launch_bwd_pair(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v,
                     const void* off, const E* o, const E* go, const float* lse,
                     const float* dlse, E* gq, E* goff, float* p_ws, float* b_ws, float* dk_acc,
                     float* dv_acc, int64_t acc_ks, int64_t acc_vs, hipStream_t s) {
  constexpr int CW = p2_window<HD, E>(), FR = p2_frames<HD, E>();
  const tiled::Args a1 = make_tiled_args(d, q, k, v, off, tiled_tiles<1>(d));
  const tiled::Args a2 = make_tiled_args(d, q, k, v, off, tiled_tiles<FR>(d));
  const dim3 g1 = tiled_grid<1>(d);
  dim3 g2 = tiled_grid<FR>(d);
  g2.z = HD / CW;
  hipLaunchKernelGGL((dsa3d_bwd_p1_kernel<HD, E>), g1, dim3(tiled::kThreads), 0, s, a1, o, go,
                     lse, dlse, goff, p_ws, b_ws, dk_acc, dv_acc, acc_ks, acc_vs);
  hipLaunchKernelGGL((dsa3d_bwd_p2_kernel<HD, CW, E, FR>), g2, dim3(P2Tile<FR>::Threads), 0, s,
                     a2, go, p_ws, b_ws, gq, dk_acc, dv_acc, acc_ks, acc_vs, 0);
  if constexpr (HD % CW != 0) {  // bf16 head_dim 96: a 64- and a 32-channel window
    g2.z = 1;
    hipLaunchKernelGGL((dsa3d_bwd_p2_kernel<HD, HD % CW, E, FR>), g2, dim3(P2Tile<FR>::Threads), 0,
                       s, a2, go, p_ws, b_ws, gq, dk_acc, dv_acc, acc_ks, acc_vs,
                       CW * (HD / CW));
  }
}

// fp32 dK (blockIdx.y 0) or dV (1) accumulator [rows, D] -> bf16 with the
// output's token stride, 8 channels per thread (32-byte loads, 16-byte stores;
// D and the strides are multiples of 8), grid-stride over 64-bit indices.
__global__ __launch_bounds__(256) void acc_to_bf16_kernel(const float* __restrict__ dk_acc,
                                                         const float* __restrict__ dv_acc,
                                                         bf16* __restrict__ dk,
                                                         bf16* __restrict__ dv, int64_t rows,
                                                         int D, int64_t ks, int64_t vs) {
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

template <typename E>
hipError_t bwd_tiled_typed(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v,
                           const void* off, const void* out, const void* dout, const float* lse,
                           const float* dlse, void* dq, void* dk, void* dv, void* doff,
                           float* p_ws, float* b_ws, float* acc, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(d.B) * d.T * d.H * d.W;
  const int D = d.num_heads * d.head_dim;
  const auto* o = static_cast<const E*>(out);
  const auto* go = static_cast<const E*>(dout);
  auto* gq = static_cast<E*>(dq);
  auto* goff = static_cast<E*>(doff);
  // dK and dV add up in fp32: in the outputs themselves for fp32 storage, in
  // the workspace accumulator (converted once at the end) for bf16
  constexpr bool kInPlace = sizeof(E) == 4;
  float* const dk_acc = kInPlace ? static_cast<float*>(dk) : acc;
  float* const dv_acc = kInPlace ? static_cast<float*>(dv) : acc + rows * D;
  const int64_t aks = kInPlace ? d.k_stride : D, avs = kInPlace ? d.v_stride : D;
  switch (d.head_dim) {
    case 32:
      launch_bwd_pair<32, E>(d, q, k, v, off, o, go, lse, dlse, gq, goff, p_ws, b_ws, dk_acc,
                               dv_acc, aks, avs, s);
      break;
    case 64:
      launch_bwd_pair<64, E>(d, q, k, v, off, o, go, lse, dlse, gq, goff, p_ws, b_ws, dk_acc,
                               dv_acc, aks, avs, s);
      break;
    case 96:
      launch_bwd_pair<96, E>(d, q, k, v, off, o, go, lse, dlse, gq, goff, p_ws, b_ws, dk_acc,
                               dv_acc, aks, avs, s);
      break;
    case 128:
      launch_bwd_pair<128, E>(d, q, k, v, off, o, go, lse, dlse, gq, goff, p_ws, b_ws, dk_acc,
                                dv_acc, aks, avs, s);
      break;
    default:
      return hipErrorInvalidValue;
  }
  if constexpr (!kInPlace) {
    const dim3 cgrid(fill_blocks(rows * (D / 8)), 2);
    hipLaunchKernelGGL(acc_to_bf16_kernel, cgrid, dim3(256), 0, s, dk_acc, dv_acc,
                       static_cast<bf16*>(dk), static_cast<bf16*>(dv), rows, D, d.k_stride,
                       d.v_stride);
  }
  return hipGetLastError();
}
}  // namespace

// Workspace of the tiled backward: for bf16 the dK/dV fp32 accumulators
// ([token][D] each; fp32 storage accumulates in its outputs), then p and
// ds * softmax_scale of every tap (fp32 [token][head][tap] each).
size_t dsa3d_tiled_bwd_ws_bytes(const msd_dsa3d_desc& d) {
  if ((d.dtype != MSD_BF16 && d.dtype != MSD_F32) || !tiled_head_dim(d.head_dim) ||
      d.kt * d.kh * d.kw > tiled::kMaxTaps)
    return 0;
  const int64_t rows = static_cast<int64_t>(d.B) * d.T * d.H * d.W;
  const int64_t acc = d.dtype == MSD_BF16 ? 2 * rows * d.num_heads * d.head_dim : 0;
  return static_cast<size_t>(acc + 2 * rows * d.num_heads * d.kt * d.kh * d.kw) * sizeof(float);
}

hipError_t launch_dsa3d_bwd_tiled(const msd_dsa3d_desc& d, const void* q, const void* k,
                                  const void* v, const void* off, const void* out,
                                  const void* dout, const float* lse, const float* dlse, void* dq,
                                  void* dk, void* dv, void* doff, void* ws, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(d.B) * d.T * d.H * d.W;
  const int64_t taps = rows * d.num_heads * d.kt * d.kh * d.kw;
  // accumulators first: rows * D floats keep p and ds 16-byte aligned
  float* acc = static_cast<float*>(ws);
  float* p_ws = acc + (d.dtype == MSD_BF16 ? 2 * rows * d.num_heads * d.head_dim : 0);
  float* b_ws = p_ws + taps;
  if (d.dtype == MSD_BF16)
    return bwd_tiled_typed<bf16>(d, q, k, v, off, out, dout, lse, dlse, dq, dk, dv, doff, p_ws,
                                 b_ws, acc, s);
  return bwd_tiled_typed<float>(d, q, k, v, off, out, dout, lse, dlse, dq, dk, dv, doff, p_ws,
                                b_ws, acc, s);
}

}  // namespace msd
