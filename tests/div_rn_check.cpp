// Bit-for-bit check of msd::div_rn against IEEE fp32 division (the host's
// divss), built with g++ -ffp-contract=off by tests/test_coords_cpu.py.
//
//   div_rn_check MANT_DIVS EXTRA_DIVS
// 1. every fp32 mantissa in [1, 2) (which covers every normal numerator up to
//    scaling by a power of two) divided by b = 1 .. MANT_DIVS, and by EXTRA_DIVS
//    divisors spread over (MANT_DIVS, 32766];
// 2. every base-grid numerator 2*pos, pos in [-64, 32831], divided by every
//    b = 1 .. 32766 (the exact set the kernels divide).
// Prints the tested and mismatch counts; exit status 1 on any mismatch.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "div_rn.h"

static bool same(float x, float y) { return std::memcmp(&x, &y, 4) == 0; }

int main(int argc, char** argv) {
  const int mant_divs = argc > 1 ? std::atoi(argv[1]) : 64;
  const int extra_divs = argc > 2 ? std::atoi(argv[2]) : 16;
  long long tested = 0, bad = 0;
  for (int k = 1; k <= mant_divs + extra_divs; ++k) {
    const int b = k <= mant_divs
                      ? k
                      : mant_divs + 1 +
                            static_cast<int>((static_cast<uint64_t>(k - mant_divs) * 2654435761u) %
                                             static_cast<uint64_t>(32766 - mant_divs));
    volatile float bv = static_cast<float>(b);
    const float bf = bv;
    const float rb = 1.0f / bf;
    for (uint32_t m = 0; m < (1u << 23); ++m) {
      const uint32_t bits = 0x3f800000u | m;
      float a;
      std::memcpy(&a, &bits, 4);
      ++tested;
      if (!same(a / bf, msd::div_rn(a, bf, rb))) {
        if (bad < 5) std::printf("mismatch a=%a b=%d\n", a, b);
        ++bad;
      }
    }
  }
  std::printf("mantissa sweep: tested %lld mismatches %lld\n", tested, bad);
  long long tested2 = 0, bad2 = 0;
  for (int b = 1; b <= 32766; ++b) {
    volatile float bv = static_cast<float>(b);
    const float bf = bv;
    const float rb = 1.0f / bf;
    for (int pos = -64; pos <= 32767 + 64; ++pos) {
      const float a = 2.0f * static_cast<float>(pos);
      ++tested2;
      if (!same(a / bf, msd::div_rn(a, bf, rb))) {
        if (bad2 < 5) std::printf("mismatch pos=%d b=%d\n", pos, b);
        ++bad2;
      }
    }
  }
  std::printf("base-grid sweep: tested %lld mismatches %lld\n", tested2, bad2);
  return (bad || bad2) ? 1 : 0;
}
