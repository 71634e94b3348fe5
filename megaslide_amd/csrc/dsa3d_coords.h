// Sampling-coordinate arithmetic shared by the 3D-DSA kernels.
#pragma once

#include "common.h"

namespace msd {

// The sampling coordinate is computed op for op in fp32 as the reference does
// it, with every operation rounded on its own (no FMA contraction, true
// division): at coordinates that land exactly on a voxel the trilinear
// gradient is discontinuous, so the corner choice must round identically.
//   base: 2*(p + c) / max(S-1, 1) - 1          (attention.py:228-230)
//   grid: base + (o * offset_scale) / (dim-1)  (:106, :118-127)
//   u   : ((grid + 1) * S - 1) / 2             (grid_sample, align_corners=False)

// Base grid value of one axis, in fp32 and in the reference's op order.
__device__ __forceinline__ float base_coord(int p, int c, int S) {
#pragma clang fp contract(off)
  const float pos = static_cast<float>(p) + static_cast<float>(c);
  return 2.0f * pos / static_cast<float>(S > 1 ? S - 1 : 1) - 1.0f;
}

// grid value: base + offset / divisor (divisor 0 means the slot is dropped).
__device__ __forceinline__ float grid_coord(float base, float o, float divisor) {
#pragma clang fp contract(off)
  return divisor > 0.0f ? base + o / divisor : base;
}

struct Axis {
  int i0;      // lower corner index (0 <= i0 <= S-1)
  bool hi_ok;  // upper corner i0+1 inside the volume
  float f;     // weight of the upper corner
  float u;     // unnormalised, unclamped coordinate (for the clamp gradient)
};

__device__ __forceinline__ Axis axis_sample(float g, int S) {
#pragma clang fp contract(off)
  Axis a;
  a.u = ((g + 1.0f) * static_cast<float>(S) - 1.0f) * 0.5f;
  // fmaxf returns the non-NaN operand, so a NaN coordinate lands on 0.
  const float c = fminf(fmaxf(a.u, 0.0f), static_cast<float>(S - 1));
  const float fl = floorf(c);
  a.i0 = min(max(static_cast<int>(fl), 0), S - 1);
  a.f = c - fl;
  a.hi_ok = (a.i0 + 1) < S;
  return a;
}

}  // namespace msd
