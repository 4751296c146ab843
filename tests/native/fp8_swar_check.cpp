// Host-side exhaustive check of the FP8 helpers the attention kernels use
// (vllm-lite_amd/csrc/pa_common.hpp): the integer decode fp8x2_ref_bf16x2
// against fp8_decode (the reference's decode, itself checked against the
// oracle), and the fp8_exotic_bits mask against its definition (exponent
// field 0 or 15, byte not 0x00), over every code in every byte position.
// Prints "ok" and exits 0 on success.
#include <cstdio>
#include <cstring>

#include "pa_common.hpp"

static unsigned bf16_of(float f) {
  unsigned u;
  std::memcpy(&u, &f, 4);
  return u >> 16;  // every reference value is exactly a bf16 (NaN: quiet 0x7FC0)
}

int main() {
  int bad = 0;
  for (unsigned a = 0; a < 256; ++a)
    for (unsigned b = 0; b < 256; ++b) {
      const unsigned v = pa::fp8x2_ref_bf16x2(a | (b << 16));
      const float fa = pa::fp8_decode(a), fb = pa::fp8_decode(b);
      const unsigned wa = fa != fa ? 0x7FC0u : bf16_of(fa);
      const unsigned wb = fb != fb ? 0x7FC0u : bf16_of(fb);
      if ((v & 0xFFFFu) != wa || (v >> 16) != wb) {
        if (bad++ < 5) std::printf("decode %02x %02x -> %08x, want %04x %04x\n", a, b, v, wa, wb);
      }
    }
  const unsigned fill[] = {0x00, 0x01, 0x07, 0x08, 0x38, 0x77, 0x78, 0x7B, 0x7C, 0x7F,
                           0x80, 0x87, 0x88, 0xF7, 0xF8, 0xFC, 0xFF};
  for (unsigned a = 0; a < 256; ++a)
    for (int pos = 0; pos < 4; ++pos)
      for (unsigned o : fill) {
        unsigned w = 0;
        for (int i = 0; i < 4; ++i) w |= (i == pos ? a : o) << (8 * i);
        const unsigned m = pa::fp8_exotic_bits(w);
        for (int i = 0; i < 4; ++i) {
          const unsigned x = (w >> (8 * i)) & 0xFF, e = (x >> 3) & 15;
          const bool want = e == 15 || (e == 0 && x != 0);
          if (((m >> (8 * i + 7)) & 1) != (unsigned)want) {
            if (bad++ < 10) std::printf("mask %08x byte %d\n", w, i);
          }
        }
      }
  if (bad) {
    std::printf("%d mismatches\n", bad);
    return 1;
  }
  std::printf("ok\n");
  return 0;
}
