// Correctly rounded fp32 division by a divisor with a precomputed reciprocal.
// Host- and device-compilable so the CPU tests check this exact source.
#pragma once

#ifndef MSD_HD
#if defined(__HIPCC__)
#define MSD_HD __host__ __device__
#else
#define MSD_HD
#endif
#endif

namespace msd {

// a / b rounded to nearest, from rb = RN(1/b): the product a*rb is within an ulp
// of the quotient, and one fused residual step (Markstein's correction) rounds
// it correctly.  Three instructions instead of the ten of a full IEEE divide.
MSD_HD inline float div_rn(float a, float b, float rb) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  const float q = a * rb;
  const float r = __builtin_fmaf(-b, q, a);
  return __builtin_fmaf(r, rb, q);
}

}  // namespace msd
