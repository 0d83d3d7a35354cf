// Host check of the Q3_K slab regrouping (gmoe_internal.h): reads packed Q3_K blocks
// (110 bytes each) from stdin, builds each block's slab bytes 0..95 with q3s_byte, decodes
// every sub-block's four words back with q3s_word / q3s_pair, and writes the 256 quants
// (v - 4, as int8, in the block's value order 16 s + l) per block to stdout.
#include <cstdio>
#include <cstdint>
#include <vector>

#include "gmoe_internal.h"

int main() {
  std::vector<uint8_t> blk(110);
  while (fread(blk.data(), 1, 110, stdin) == 110) {
    uint32_t w[24];
    for (uint32_t j = 0; j < 24; j++) {
      w[j] = 0;
      for (uint32_t b = 0; b < 4; b++) w[j] |= (uint32_t)gmoe::q3s_byte(blk.data(), 4 * j + b) << (8 * b);
    }
    int8_t q[256];
    for (int s = 0; s < 16; s++) {
      const uint32_t c = s / 8, x0 = 3 * ((s % 8) / 4);
      uint32_t o[4];
      for (uint32_t h = 0; h < 2; h++)
        gmoe::q3s_pair(w[gmoe::q3s_word(c, h, x0)], w[gmoe::q3s_word(c, h, x0 + 1)], w[gmoe::q3s_word(c, h, x0 + 2)],
                       s % 4, o[2 * h], o[2 * h + 1]);
      for (int l = 0; l < 16; l++) q[16 * s + l] = (int8_t)((int)((o[l / 4] >> (8 * (l % 4))) & 0xffu) - 4);
    }
    fwrite(q, 1, 256, stdout);
  }
  return 0;
}
