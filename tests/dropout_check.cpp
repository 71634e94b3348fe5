// Host build of the kernels' dropout header (megaslide_amd/csrc/dropout.h):
// prints Philox4x32-10 first words for counters/keys read from stdin, one
// "c0 c1 c2 c3 k0 k1" line each, and the dropout factor for lines starting with
// "f threshold scale key0 key1 offset row head tap".
#include <cstdio>
#include <cstring>

#include "dropout.h"

int main() {
  char tag[8];
  while (std::scanf("%7s", tag) == 1) {
    if (std::strcmp(tag, "p") == 0) {
      unsigned c0, c1, c2, c3, k0, k1;
      if (std::scanf("%u %u %u %u %u %u", &c0, &c1, &c2, &c3, &k0, &k1) != 6) return 1;
      std::printf("%u\n", msd::philox4x32_10_first(c0, c1, c2, c3, k0, k1));
    } else if (std::strcmp(tag, "f") == 0) {
      msd::DropoutArgs d;
      long long row;
      int head, tap;
      if (std::scanf("%u %f %u %u %u %lld %d %d", &d.threshold, &d.scale, &d.key0, &d.key1,
                     &d.offset, &row, &head, &tap) != 8)
        return 1;
      std::printf("%.9g\n", static_cast<double>(msd::dropout_factor(d, row, head, tap)));
    } else {
      return 1;
    }
  }
  return 0;
}
