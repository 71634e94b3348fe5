// Direct-form 3D-DSA kernels for gfx950: one 16-lane group per
// (batch, token, head), every tap's eight trilinear corners gathered from
// global memory, online softmax in registers.
//
// These are the general kernels: any head_dim <= 256, any window, fp32 or
// bf16.  They restate, for one query and head, what the reference computes
// with grid_sample + matmul + softmax + matmul (infinity/video/attention.py:
// 106-186) and autograd's backward of it:
//
//   per tap (i, j, k), kappa = (i*kh + j)*kw + k, raw offsets o = off[...]*scale
//     g_x = 2(w + k - kw/2)/max(W-1,1) - 1 + (T>1 ? o0/(T-1) : 0)   (:118-127,
//     g_y = 2(h + j - kh/2)/max(H-1,1) - 1 + (H>1 ? o1/(H-1) : 0)    :209-236;
//     g_z = 2(t + i - kt/2)/max(T-1,1) - 1 + (W>1 ? o2/(W-1) : 0)    slot 0 goes
//                                                                      to x, slot 2 to z)
//     u = ((g + 1)*S - 1)/2, clamped to [0, S-1]  (grid_sample, align_corners
//     = False, padding_mode = 'border', :262-268); corners beyond S-1 carry
//     weight 0 and are skipped.
//   s = q . sum_c w_c K_c / sqrt(hd); p = softmax(s); o = sum p sum_c w_c V_c.
//
// Backward per tap: dp = dO . v_s, ds = p (dp - Delta), Delta = sum over taps
// (and extra keys) of p f dp - dlse, formed in fp32 by a first pass over the
// taps (dO . o from the stored output would carry its rounding: for bf16
// storage that is of the size of ds itself where the softmax is peaked, and
// the reference's softmax backward sums p dp over its taps as well);
// dq += ds*scale*k_s; dK_c += w_c ds scale q; dV_c += w_c p dO (fp32 atomics
// into an fp32 accumulator); d u = sum_c dw_c/du (ds scale q.K_c + p dO.V_c),
// zeroed where u <= 0 or u >= S-1 (border clamp), times S/2 (unnormalise),
// divided by the slot's divisor and times offset_scale.
#include "common.h"
#include "dsa3d_coords.h"

namespace msd {

namespace {

constexpr int kGroup = 16;            // lanes per (token, head)
constexpr int kBlock = 256;           // threads per block
constexpr int kGroupsPerBlock = kBlock / kGroup;

struct CoreArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* off;
  int64_t qs, ks, vs;  // token strides of q, k, v (elements)
  int64_t N;           // tokens per sample
  int B, T, H, W, nh, hd, kt, kh, kw, C;
  float offset_scale, softmax_scale;
  float div_x, div_y, div_z;     // T-1, H-1, W-1: divisors of slots 0, 1, 2 (0 if that dim is 1)
  float rdiv_x, rdiv_y, rdiv_z;  // their reciprocals (0 if the dim is 1), for the gradient
  DropoutArgs drop;              // attention dropout on the softmax weights
  const void* ek;                // extra keys / values [B, G, D] (attention.py:160-173)
  const void* ev;
  int G;                         // extra keys per sample (0 = none)
};

template <typename T>
__device__ __forceinline__ void load_offsets(const T* p, float scale, float& o0, float& o1,
                                             float& o2) {
  o0 = ld(p, 0) * scale;
  o1 = ld(p, 1) * scale;
  o2 = ld(p, 2) * scale;
}

template <typename T, int CPL>
__global__ __launch_bounds__(kBlock) void dsa3d_fwd_direct_kernel(CoreArgs a, T* __restrict__ out,
                                                                   float* __restrict__ lse) {
  const int lane = threadIdx.x % kGroup;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int64_t total = static_cast<int64_t>(a.B) * a.N * a.nh;
  if (gid >= total) return;  // uniform across the 16-lane group
  const int head = static_cast<int>(gid % a.nh);
  const int64_t bn = gid / a.nh;
  const int b = static_cast<int>(bn / a.N);
  const int64_t n = bn - static_cast<int64_t>(b) * a.N;
  const int w = static_cast<int>(n % a.W);
  const int h = static_cast<int>((n / a.W) % a.H);
  const int t = static_cast<int>(n / (static_cast<int64_t>(a.W) * a.H));
  const T* __restrict__ qp = static_cast<const T*>(a.q);
  const T* __restrict__ kp = static_cast<const T*>(a.k);
  const T* __restrict__ vp = static_cast<const T*>(a.v);
  const int K = a.kt * a.kh * a.kw;
  const T* __restrict__ op = static_cast<const T*>(a.off) + bn * a.C + static_cast<int64_t>(head) * K * 3;
  const int cbase = head * a.hd + lane * CPL;
  const int64_t sample0 = static_cast<int64_t>(b) * a.N;

  float qv[CPL], acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int d = lane * CPL + j;
    qv[j] = d < a.hd ? ld(qp, bn * a.qs + cbase + j) : 0.0f;
    acc[j] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  int kap = 0;
  for (int i = 0; i < a.kt; ++i) {
    const float bz = base_coord(t, i - a.kt / 2, a.T);
    for (int jj = 0; jj < a.kh; ++jj) {
      const float by = base_coord(h, jj - a.kh / 2, a.H);
      for (int kk = 0; kk < a.kw; ++kk, ++kap) {
        const float bx = base_coord(w, kk - a.kw / 2, a.W);
        float o0, o1, o2;
        load_offsets(op + kap * 3, a.offset_scale, o0, o1, o2);
        const Axis ax = axis_sample(grid_coord(bx, o0, a.div_x), a.W);
        const Axis ay = axis_sample(grid_coord(by, o1, a.div_y), a.H);
        const Axis az = axis_sample(grid_coord(bz, o2, a.div_z), a.T);
        float ksum[CPL], vsum[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) ksum[j] = vsum[j] = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int dz = c >> 2, dy = (c >> 1) & 1, dx = c & 1;
          if ((dz && !az.hi_ok) || (dy && !ay.hi_ok) || (dx && !ax.hi_ok)) continue;
          const float wgt = (dz ? az.f : 1.0f - az.f) * (dy ? ay.f : 1.0f - ay.f) *
                            (dx ? ax.f : 1.0f - ax.f);
          const int64_t row =
              sample0 + (static_cast<int64_t>(az.i0 + dz) * a.H + (ay.i0 + dy)) * a.W + (ax.i0 + dx);
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            if (lane * CPL + j < a.hd) {
              ksum[j] += wgt * ld(kp, row * a.ks + cbase + j);
              vsum[j] += wgt * ld(vp, row * a.vs + cbase + j);
            }
          }
        }
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) part += qv[j] * ksum[j];
        const float s = group_sum<kGroup>(part) * a.softmax_scale;
        const float mn = fmaxf(m, s);
        const float corr = __expf(m - mn);
        const float e = __expf(s - mn);
        l = l * corr + e;  // the softmax normaliser counts dropped taps too
        const float ed = e * dropout_factor(a.drop, bn, head, kap);
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[j] = acc[j] * corr + ed * vsum[j];
        m = mn;
      }
    }
  }
  // extra keys shared by every query: taps K + g of the same softmax
  const T* __restrict__ ekp = static_cast<const T*>(a.ek);
  const T* __restrict__ evp = static_cast<const T*>(a.ev);
  const int D = a.nh * a.hd;
  for (int g = 0; g < a.G; ++g) {
    const int64_t erow = (static_cast<int64_t>(b) * a.G + g) * D + cbase;
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      if (lane * CPL + j < a.hd) part += qv[j] * ld(ekp, erow + j);
    const float s = group_sum<kGroup>(part) * a.softmax_scale;
    const float mn = fmaxf(m, s);
    const float corr = __expf(m - mn);
    const float e = __expf(s - mn);
    l = l * corr + e;
    const float ed = e * dropout_factor(a.drop, bn, head, K + g);
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      acc[j] = acc[j] * corr + (lane * CPL + j < a.hd ? ed * ld(evp, erow + j) : 0.0f);
    m = mn;
  }
  T* __restrict__ orow = out + bn * (static_cast<int64_t>(a.nh) * a.hd);
  const float inv = 1.0f / l;
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if (lane * CPL + j < a.hd) st(orow, cbase + j, acc[j] * inv);
  if (lse != nullptr && lane == 0) lse[bn * a.nh + head] = m + logf(l);
}

template <typename T, int CPL>
__global__ __launch_bounds__(kBlock) void dsa3d_bwd_direct_kernel(
    CoreArgs a, const T* __restrict__ out, const T* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ dlse, T* __restrict__ dq, float* __restrict__ dk_acc,
    float* __restrict__ dv_acc, T* __restrict__ doff, float* __restrict__ dek_acc,
    float* __restrict__ dev_acc) {
  (void)out;  // Delta comes from the taps, not from the stored output
  const int lane = threadIdx.x % kGroup;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int64_t total = static_cast<int64_t>(a.B) * a.N * a.nh;
  if (gid >= total) return;
  const int head = static_cast<int>(gid % a.nh);
  const int64_t bn = gid / a.nh;
  const int b = static_cast<int>(bn / a.N);
  const int64_t n = bn - static_cast<int64_t>(b) * a.N;
  const int w = static_cast<int>(n % a.W);
  const int h = static_cast<int>((n / a.W) % a.H);
  const int t = static_cast<int>(n / (static_cast<int64_t>(a.W) * a.H));
  const T* __restrict__ qp = static_cast<const T*>(a.q);
  const T* __restrict__ kp = static_cast<const T*>(a.k);
  const T* __restrict__ vp = static_cast<const T*>(a.v);
  const int K = a.kt * a.kh * a.kw;
  const int64_t obase = bn * a.C + static_cast<int64_t>(head) * K * 3;
  const T* __restrict__ op = static_cast<const T*>(a.off) + obase;
  const int D = a.nh * a.hd;
  const int cbase = head * a.hd + lane * CPL;
  const int64_t sample0 = static_cast<int64_t>(b) * a.N;

  float qv[CPL], gov[CPL], dqv[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const bool on = lane * CPL + j < a.hd;
    qv[j] = on ? ld(qp, bn * a.qs + cbase + j) : 0.0f;
    gov[j] = on ? ld(dout, bn * D + cbase + j) : 0.0f;
    dqv[j] = 0.0f;
  }
  const float lse_q = lse[bn * a.nh + head];
  const float sc = a.softmax_scale;
  const T* __restrict__ ekp = static_cast<const T*>(a.ek);
  const T* __restrict__ evp = static_cast<const T*>(a.ev);

  // s and dp of tap kap (the same gathers and rounding as the main pass below)
  auto tap_s_dp = [&](int kap, float bx, float by, float bz, float& s, float& dp) {
    float o0, o1, o2;
    load_offsets(op + kap * 3, a.offset_scale, o0, o1, o2);
    const Axis ax = axis_sample(grid_coord(bx, o0, a.div_x), a.W);
    const Axis ay = axis_sample(grid_coord(by, o1, a.div_y), a.H);
    const Axis az = axis_sample(grid_coord(bz, o2, a.div_z), a.T);
    float s_part = 0.0f, dp_part = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int dz = c >> 2, dy = (c >> 1) & 1, dx = c & 1;
      if ((dz && !az.hi_ok) || (dy && !ay.hi_ok) || (dx && !ax.hi_ok)) continue;
      const float wgt = (dz ? az.f : 1.0f - az.f) * (dy ? ay.f : 1.0f - ay.f) *
                        (dx ? ax.f : 1.0f - ax.f);
      const int64_t row =
          sample0 + (static_cast<int64_t>(az.i0 + dz) * a.H + (ay.i0 + dy)) * a.W + (ax.i0 + dx);
      float pkc = 0.0f, pvc = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (lane * CPL + j < a.hd) {
          pkc += qv[j] * ld(kp, row * a.ks + cbase + j);
          pvc += gov[j] * ld(vp, row * a.vs + cbase + j);
        }
      }
      s_part += wgt * pkc;
      dp_part += wgt * pvc;
    }
    s = group_sum<kGroup>(s_part) * sc;
    dp = group_sum<kGroup>(dp_part);
  };

  // Delta = dO . o = sum of p f dp over the taps and extra keys, in fp32
  float delta = 0.0f;
  {
    int kap = 0;
    for (int i = 0; i < a.kt; ++i) {
      const float bz = base_coord(t, i - a.kt / 2, a.T);
      for (int jj = 0; jj < a.kh; ++jj) {
        const float by = base_coord(h, jj - a.kh / 2, a.H);
        for (int kk = 0; kk < a.kw; ++kk, ++kap) {
          float s, dp;
          tap_s_dp(kap, base_coord(w, kk - a.kw / 2, a.W), by, bz, s, dp);
          delta += __expf(s - lse_q) * dropout_factor(a.drop, bn, head, kap) * dp;
        }
      }
    }
    for (int g = 0; g < a.G; ++g) {
      const int64_t erow = (static_cast<int64_t>(b) * a.G + g) * D + cbase;
      float s_part = 0.0f, dp_part = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (lane * CPL + j < a.hd) {
          s_part += qv[j] * ld(ekp, erow + j);
          dp_part += gov[j] * ld(evp, erow + j);
        }
      }
      const float s = group_sum<kGroup>(s_part) * sc;
      const float dp = group_sum<kGroup>(dp_part);
      delta += __expf(s - lse_q) * dropout_factor(a.drop, bn, head, K + g) * dp;
    }
  }
  if (dlse != nullptr) delta -= dlse[bn * a.nh + head];

  int kap = 0;
  for (int i = 0; i < a.kt; ++i) {
    const float bz = base_coord(t, i - a.kt / 2, a.T);
    for (int jj = 0; jj < a.kh; ++jj) {
      const float by = base_coord(h, jj - a.kh / 2, a.H);
      for (int kk = 0; kk < a.kw; ++kk, ++kap) {
        const float bx = base_coord(w, kk - a.kw / 2, a.W);
        float o0, o1, o2;
        load_offsets(op + kap * 3, a.offset_scale, o0, o1, o2);
        const Axis ax = axis_sample(grid_coord(bx, o0, a.div_x), a.W);
        const Axis ay = axis_sample(grid_coord(by, o1, a.div_y), a.H);
        const Axis az = axis_sample(grid_coord(bz, o2, a.div_z), a.T);
        float ksum[CPL];
        float pk[8], pv[8];
        int64_t rows[8];
#pragma unroll
        for (int j = 0; j < CPL; ++j) ksum[j] = 0.0f;
        float s_part = 0.0f, dp_part = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int dz = c >> 2, dy = (c >> 1) & 1, dx = c & 1;
          pk[c] = pv[c] = 0.0f;
          rows[c] = -1;
          if ((dz && !az.hi_ok) || (dy && !ay.hi_ok) || (dx && !ax.hi_ok)) continue;
          const float wgt = (dz ? az.f : 1.0f - az.f) * (dy ? ay.f : 1.0f - ay.f) *
                            (dx ? ax.f : 1.0f - ax.f);
          const int64_t row =
              sample0 + (static_cast<int64_t>(az.i0 + dz) * a.H + (ay.i0 + dy)) * a.W + (ax.i0 + dx);
          rows[c] = row;
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            if (lane * CPL + j < a.hd) {
              const float kv = ld(kp, row * a.ks + cbase + j);
              const float vv = ld(vp, row * a.vs + cbase + j);
              ksum[j] += wgt * kv;
              pk[c] += qv[j] * kv;
              pv[c] += gov[j] * vv;
            }
          }
          s_part += wgt * pk[c];
          dp_part += wgt * pv[c];
        }
        const float s = group_sum<kGroup>(s_part) * sc;
        const float dp = group_sum<kGroup>(dp_part);
        const float p = __expf(s - lse_q);
        // dropout: o sums pd * v_s with pd = p * factor, so dp/ds see the factor
        const float dfac = dropout_factor(a.drop, bn, head, kap);
        const float pd = p * dfac;
        const float ds = p * (dfac * dp - delta);
        const float dss = ds * sc;
#pragma unroll
        for (int j = 0; j < CPL; ++j) dqv[j] += dss * ksum[j];
        float gx = 0.0f, gy = 0.0f, gz = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          if (rows[c] < 0) continue;
          const int dz = c >> 2, dy = (c >> 1) & 1, dx = c & 1;
          const float wz = dz ? az.f : 1.0f - az.f;
          const float wy = dy ? ay.f : 1.0f - ay.f;
          const float wx = dx ? ax.f : 1.0f - ax.f;
          const float wgt = wz * wy * wx;
          const float tc = dss * pk[c] + pd * pv[c];
          gx += (dx ? 1.0f : -1.0f) * wy * wz * tc;
          gy += (dy ? 1.0f : -1.0f) * wx * wz * tc;
          gz += (dz ? 1.0f : -1.0f) * wx * wy * tc;
          const int64_t row = rows[c];
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            if (lane * CPL + j < a.hd) {
              atomicAdd(dk_acc + row * D + cbase + j, wgt * dss * qv[j]);
              atomicAdd(dv_acc + row * D + cbase + j, wgt * pd * gov[j]);
            }
          }
        }
        gx = group_sum<kGroup>(gx);
        gy = group_sum<kGroup>(gy);
        gz = group_sum<kGroup>(gz);
        if (lane == 0) {
          const float mx = (ax.u > 0.0f && ax.u < static_cast<float>(a.W - 1)) ? 0.5f * a.W : 0.0f;
          const float my = (ay.u > 0.0f && ay.u < static_cast<float>(a.H - 1)) ? 0.5f * a.H : 0.0f;
          const float mz = (az.u > 0.0f && az.u < static_cast<float>(a.T - 1)) ? 0.5f * a.T : 0.0f;
          T* __restrict__ dop = doff + obase + kap * 3;
          st(dop, 0, gx * mx * a.rdiv_x * a.offset_scale);
          st(dop, 1, gy * my * a.rdiv_y * a.offset_scale);
          st(dop, 2, gz * mz * a.rdiv_z * a.offset_scale);
        }
      }
    }
  }
  // extra keys: dq += ds scale ek_g; dEK_g += ds scale q, dEV_g += p f dO (fp32 atomics)
  for (int g = 0; g < a.G; ++g) {
    const int64_t erow = (static_cast<int64_t>(b) * a.G + g) * D + cbase;
    float ekv[CPL], s_part = 0.0f, dp_part = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const bool on = lane * CPL + j < a.hd;
      ekv[j] = on ? ld(ekp, erow + j) : 0.0f;
      s_part += qv[j] * ekv[j];
      dp_part += on ? gov[j] * ld(evp, erow + j) : 0.0f;
    }
    const float s = group_sum<kGroup>(s_part) * sc;
    const float dp = group_sum<kGroup>(dp_part);
    const float p = __expf(s - lse_q);
    const float dfac = dropout_factor(a.drop, bn, head, K + g);
    const float pd = p * dfac;
    const float dss = p * (dfac * dp - delta) * sc;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (lane * CPL + j < a.hd) {
        dqv[j] += dss * ekv[j];
        atomicAdd(dek_acc + erow + j, dss * qv[j]);
        atomicAdd(dev_acc + erow + j, pd * gov[j]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if (lane * CPL + j < a.hd) st(dq, bn * a.qs + cbase + j, dqv[j]);
}

// Accumulator [rows, D] fp32 -> dst with token stride `stride`, element type T.
template <typename T>
__global__ __launch_bounds__(256) void strided_convert_kernel(const float* __restrict__ src,
                                                              T* __restrict__ dst, int64_t rows,
                                                              int D, int64_t stride) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * D) return;
  const int64_t r = i / D;
  const int c = static_cast<int>(i - r * D);
  st(dst, r * stride + c, src[i]);
}

CoreArgs make_args(const msd_dsa3d_desc& d, const void* q, const void* k, const void* v,
                   const void* off, const void* ek, const void* ev) {
  CoreArgs a;
  a.ek = ek;
  a.ev = ev;
  a.G = d.extra_g;
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
  a.hd = d.head_dim;
  a.kt = d.kt;
  a.kh = d.kh;
  a.kw = d.kw;
  a.C = d.num_heads * d.kt * d.kh * d.kw * 3;
  a.offset_scale = d.offset_scale;
  a.softmax_scale = d.softmax_scale;
  a.div_x = d.T > 1 ? static_cast<float>(d.T - 1) : 0.0f;
  a.div_y = d.H > 1 ? static_cast<float>(d.H - 1) : 0.0f;
  a.div_z = d.W > 1 ? static_cast<float>(d.W - 1) : 0.0f;
  a.rdiv_x = d.T > 1 ? 1.0f / static_cast<float>(d.T - 1) : 0.0f;
  a.rdiv_y = d.H > 1 ? 1.0f / static_cast<float>(d.H - 1) : 0.0f;
  a.rdiv_z = d.W > 1 ? 1.0f / static_cast<float>(d.W - 1) : 0.0f;
  a.drop = dropout_args(d);
  return a;
}

template <typename F>
hipError_t dispatch_cpl(int hd, F&& f) {
  const int need = (hd + kGroup - 1) / kGroup;
  if (need <= 1) return f.template operator()<1>();
  if (need <= 2) return f.template operator()<2>();
  if (need <= 3) return f.template operator()<3>();
  if (need <= 4) return f.template operator()<4>();
  if (need <= 6) return f.template operator()<6>();
  if (need <= 8) return f.template operator()<8>();
  if (need <= 12) return f.template operator()<12>();
  return f.template operator()<16>();
}

template <typename T>
hipError_t fwd_typed(const msd_dsa3d_desc& d, const CoreArgs& a, void* out, float* lse,
                     hipStream_t s) {
  const int64_t groups = static_cast<int64_t>(a.B) * a.N * a.nh;
  const dim3 grid(static_cast<unsigned>((groups + kGroupsPerBlock - 1) / kGroupsPerBlock));
  return dispatch_cpl(d.head_dim, [&]<int CPL>() {
    hipLaunchKernelGGL((dsa3d_fwd_direct_kernel<T, CPL>), grid, dim3(kBlock), 0, s, a,
                       static_cast<T*>(out), lse);
    return hipGetLastError();
  });
}

template <typename T>
hipError_t bwd_typed(const msd_dsa3d_desc& d, const CoreArgs& a, const void* out, const void* dout,
                     const float* lse, const float* dlse, void* dq, void* dk, void* dv, void* doff,
                     void* dek, void* dev, void* ws, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.N;
  const int D = a.nh * a.hd;
  const int64_t erows = static_cast<int64_t>(a.B) * a.G;
  float* dk_acc = static_cast<float*>(ws);
  float* dv_acc = dk_acc + rows * D;
  float* dek_acc = dv_acc + rows * D;
  float* dev_acc = dek_acc + erows * D;
  const int64_t nacc = 2 * (rows + erows) * D;
  hipLaunchKernelGGL(fill_zero_f32, dim3(fill_blocks(nacc)), dim3(256), 0, s, dk_acc, nacc);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t groups = rows * a.nh;
  const dim3 grid(static_cast<unsigned>((groups + kGroupsPerBlock - 1) / kGroupsPerBlock));
  e = dispatch_cpl(d.head_dim, [&]<int CPL>() {
    hipLaunchKernelGGL((dsa3d_bwd_direct_kernel<T, CPL>), grid, dim3(kBlock), 0, s, a,
                       static_cast<const T*>(out), static_cast<const T*>(dout), lse, dlse,
                       static_cast<T*>(dq), dk_acc, dv_acc, static_cast<T*>(doff), dek_acc,
                       dev_acc);
    return hipGetLastError();
  });
  if (e != hipSuccess) return e;
  const dim3 cgrid(static_cast<unsigned>((rows * D + 255) / 256));
  hipLaunchKernelGGL((strided_convert_kernel<T>), cgrid, dim3(256), 0, s, dk_acc,
                     static_cast<T*>(dk), rows, D, a.ks);
  hipLaunchKernelGGL((strided_convert_kernel<T>), cgrid, dim3(256), 0, s, dv_acc,
                     static_cast<T*>(dv), rows, D, a.vs);
  if (erows > 0) {
    const dim3 egrid(static_cast<unsigned>((erows * D + 255) / 256));
    hipLaunchKernelGGL((strided_convert_kernel<T>), egrid, dim3(256), 0, s, dek_acc,
                       static_cast<T*>(dek), erows, D, static_cast<int64_t>(D));
    hipLaunchKernelGGL((strided_convert_kernel<T>), egrid, dim3(256), 0, s, dev_acc,
                       static_cast<T*>(dev), erows, D, static_cast<int64_t>(D));
  }
  return hipGetLastError();
}

}  // namespace

int dsa3d_max_head_dim() { return kGroup * 16; }

// The larger of the two families' needs, so a descriptor the tiled kernels
// take still runs if a pointer sends it to the direct ones: the direct
// backward's dK/dV (and extra-key) fp32 accumulators, the tiled backward's per-tap p and ds
// (the larger whenever kt * kh * kw > head_dim: every tiled head size at the
// reference 3x7x7 window).
size_t dsa3d_bwd_ws_bytes(const msd_dsa3d_desc& d) {
  const int64_t rows = static_cast<int64_t>(d.B) * d.T * d.H * d.W + int64_t{d.B} * d.extra_g;
  const size_t direct = static_cast<size_t>(2 * rows * d.num_heads * d.head_dim) * sizeof(float);
  const size_t tiled = dsa3d_tiled_bwd_ws_bytes(d);
  return direct > tiled ? direct : tiled;
}

hipError_t launch_dsa3d_fwd_direct(const msd_dsa3d_desc& d, const void* q, const void* k,
                                   const void* v, const void* off, const void* ek, const void* ev,
                                   void* out, float* lse, hipStream_t s) {
  const CoreArgs a = make_args(d, q, k, v, off, ek, ev);
  if (d.dtype == MSD_BF16) return fwd_typed<bf16>(d, a, out, lse, s);
  return fwd_typed<float>(d, a, out, lse, s);
}

hipError_t launch_dsa3d_bwd_direct(const msd_dsa3d_desc& d, const void* q, const void* k,
                                   const void* v, const void* off, const void* ek, const void* ev,
                                   const void* out, const void* dout, const float* lse,
                                   const float* dlse, void* dq, void* dk, void* dv, void* doff,
                                   void* dek, void* dev, void* ws, hipStream_t s) {
  const CoreArgs a = make_args(d, q, k, v, off, ek, ev);
  if (d.dtype == MSD_BF16)
    return bwd_typed<bf16>(d, a, out, dout, lse, dlse, dq, dk, dv, doff, dek, dev, ws, s);
  return bwd_typed<float>(d, a, out, dout, lse, dlse, dq, dk, dv, doff, dek, dev, ws, s);
}

}  // namespace msd
