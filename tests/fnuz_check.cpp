// CPU check of the FNUZ fp8 conversions (fe2o3_amd/csrc/fp8_fnuz.hpp, the
// functions the gfx950 kernels run) against the oracle (oracle/fp8.c):
// every f32 bit pattern through fnuz_code and every code through fnuz_bits,
// for both formats.  Test infrastructure: built and run by
// tests/test_fnuz_codec.py against oracle/liboracle.so.
#include <stdint.h>
#include <stdio.h>

#include "../fe2o3_amd/csrc/fp8_fnuz.hpp"

extern "C" uint8_t fe2o3o_fnuz_from_f32_bits(uint32_t bits, int32_t format);
extern "C" uint32_t fe2o3o_fnuz_to_f32_bits(uint8_t q, int32_t format);

int main() {
  long long bad = 0;
  for (int f = 0; f < 2; ++f) {
    for (uint32_t c = 0; c < 256; ++c) {
      const uint32_t got = f == 0 ? fe2o3::fnuz_bits<0>(c) : fe2o3::fnuz_bits<1>(c);
      if (got != fe2o3o_fnuz_to_f32_bits((uint8_t)c, f)) {
        if (bad < 10) printf("widen format %d code %02x: %08x\n", f, c, got);
        ++bad;
      }
    }
    long long bad_f = 0;
#pragma omp parallel for reduction(+ : bad_f) schedule(static)
    for (long long hi = 0; hi < 65536; ++hi) {
      for (uint32_t lo = 0; lo < 65536; ++lo) {
        const uint32_t x = ((uint32_t)hi << 16) | lo;
        const uint32_t got = f == 0 ? fe2o3::fnuz_code<0>(x) : fe2o3::fnuz_code<1>(x);
        if (got != fe2o3o_fnuz_from_f32_bits(x, f)) ++bad_f;
      }
    }
    if (bad_f) printf("narrow format %d: %lld mismatches\n", f, bad_f);
    bad += bad_f;
  }
  printf("failures %lld\n", bad);
  return bad == 0 ? 0 : 1;
}
