// Attention-dropout keep mask from a counter-based generator: Philox4x32-10
// (J. K. Salmon, M. A. Moraes, R. O. Dror, D. E. Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11).  Host- and device-compilable so the
// CPU tests check this exact source against the published known-answer vectors.
//
// The reference drops softmax weights with nn.Dropout (infinity/video/
// attention.py:80, :180).  PyTorch's random stream cannot be reproduced here;
// the kernels draw tap k of global token row r and head m from counter
// (k, r mod 2^32, (r >> 32) << 16 | m, offset) under key (seed lo, seed hi):
// the tap is dropped when the first output word is below `threshold`
// (floor(p * 2^32)) and kept weights are multiplied by `scale` = 1 / (1 - p)
// (fp32), as nn.Dropout scales them.  threshold == 0 means no dropout.
#pragma once

#include <stdint.h>

#ifndef MSD_HD
#if defined(__HIPCC__)
#define MSD_HD __host__ __device__
#else
#define MSD_HD
#endif
#endif

namespace msd {

struct DropoutArgs {
  uint32_t threshold;  // 0 = dropout off
  float scale;         // 1 / (1 - p)
  uint32_t key0, key1, offset;
};

// First output word of Philox4x32-10 for counter (c0, c1, c2, c3), key (k0, k1).
MSD_HD inline uint32_t philox4x32_10_first(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                           uint32_t k0, uint32_t k1) {
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
    const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
    const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
    const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
  }
  return c0;
}

// Weight factor of tap `tap` of global token row `row`, head `head`: 1 when
// dropout is off, else 0 (dropped) or scale (kept).
MSD_HD inline float dropout_factor(const DropoutArgs& d, int64_t row, int head, int tap) {
  if (d.threshold == 0) return 1.0f;
  const uint64_t r = static_cast<uint64_t>(row);
  const uint32_t u = philox4x32_10_first(static_cast<uint32_t>(tap), static_cast<uint32_t>(r),
                                         static_cast<uint32_t>((r >> 32) << 16) |
                                             static_cast<uint32_t>(head),
                                         d.offset, d.key0, d.key1);
  return u >= d.threshold ? d.scale : 0.0f;
}

}  // namespace msd
