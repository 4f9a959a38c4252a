// Host check of the packed exchange-word helpers of plh_device.h (xw_enc_pair, xw_dec_pair,
// xw_tag, xw_tag_is, xw_tag_bits, xw_step_tag), built and run by tests/test_xw_words.py.  The helpers use
// packed 16-bit arithmetic; here they are compared, exhaustively over one 16-bit half and a stride
// over the other, with their per-half definitions:
//   encode: a half with an all-ones exponent (NaN, infinity) -> sign | 0x3E00, any other -> bit 14 cleared
//   decode: bit 14 cleared, and (sign |) 0x3E00 -> (sign |) 0x7E00 (NaN)
// and the round trip is checked for every half a step can produce (|h| <= 1, NaN, infinity).
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "plh_device.h"

using namespace plh;

static uint32_t enc_half_spec(uint32_t b) { return (b & 0x7C00u) == 0x7C00u ? (b & 0x8000u) | 0x3E00u : b & 0xBFFFu; }
static uint32_t dec_half_spec(uint32_t x) {
  x &= 0xBFFFu;
  return (x & 0x7FFFu) == 0x3E00u ? x | 0x7E00u : x;
}
static bool is_h(uint32_t b) { return (b & 0x7FFFu) <= 0x3C00u; }  // |h| <= 1 (and -0)
static bool is_special(uint32_t b) { return (b & 0x7C00u) == 0x7C00u; }

int main() {
  long bad = 0, n_enc = 0, n_dec = 0, n_rt = 0;
  for (uint32_t lo = 0; lo < 65536; ++lo) {
    for (uint32_t hi = lo % 7; hi < 65536; hi += 7) {
      const uint32_t p = lo | (hi << 16);
      ++n_enc;
      const uint32_t e = xw_enc_pair(p);
      if (e != (enc_half_spec(lo) | (enc_half_spec(hi) << 16))) {
        if (bad++ < 5) std::printf("encode 0x%08x -> 0x%08x\n", p, e);
      }
      if ((e & 0x40004000u) != 0u) {
        if (bad++ < 5) std::printf("encode 0x%08x leaves a tag bit set\n", p);
      }
      // decode of an encoded pair with any tag bits, for halves a word can carry from a live row
      if ((is_h(lo) || is_special(lo)) && (is_h(hi) || is_special(hi))) {
        for (uint32_t tag = 0; tag < 4; ++tag) {
          const uint32_t w = e | ((tag & 1u) << 14) | ((tag >> 1) << 30);
          ++n_dec;
          const uint32_t d = xw_dec_pair(w);
          if (d != (dec_half_spec(w & 0xFFFFu) | (dec_half_spec(w >> 16) << 16))) {
            if (bad++ < 5) std::printf("decode 0x%08x -> 0x%08x\n", w, d);
          }
          // round trip: h back unchanged, NaN and infinity back as NaN of the same sign
          ++n_rt;
          for (int half = 0; half < 2; ++half) {
            const uint32_t b = half ? hi : lo, r = half ? d >> 16 : d & 0xFFFFu;
            const uint32_t want = is_special(b) ? (b & 0x8000u) | 0x7E00u : b;
            if (r != want) {
              if (bad++ < 5) std::printf("round trip 0x%04x -> 0x%04x\n", b, r);
            }
          }
        }
      }
    }
  }
  // tags: the four bits go to bit 14 of each fp16 of a word and come back; step tags are 1..15 and
  // differ between steps t and t + 2 (the two writes to one ring slot)
  for (uint32_t tag = 0; tag < 16; ++tag) {
    const uint64_t bits = xw_tag_bits(tag);
    if ((bits & ~0x4000400040004000ull) != 0u || xw_tag(bits) != tag || xw_tag(bits | 0xBFFFBFFFBFFFBFFFull) != tag) {
      if (bad++ < 5) std::printf("tag %u\n", tag);
    }
  }
  // xw_tag_is: the masked compare agrees with the extracted tag for every tag and word pattern
  for (uint32_t tag = 0; tag < 16; ++tag)
    for (uint32_t k = 0; k < 65536; ++k) {
      const uint64_t w = ((uint64_t)(k * 2654435761u) << 32 | (k * 40503u)) ^ ((uint64_t)k << 14);
      if (xw_tag_is(w, xw_tag_bits(tag)) != (xw_tag(w) == tag)) {
        if (bad++ < 5) std::printf("tag_is %u 0x%016llx\n", tag, (unsigned long long)w);
      }
    }
  for (int t = 0; t < 100000; ++t) {
    const uint32_t a = xw_step_tag(t), b = xw_step_tag(t + 2);
    if (a < 1u || a > 15u || a == b) {
      if (bad++ < 5) std::printf("step tag %d\n", t);
    }
  }
  std::printf("xw helpers: %ld encodes, %ld decodes, %ld round trips, %ld mismatches\n", n_enc, n_dec, n_rt, bad);
  return bad == 0 ? 0 : 1;
}
