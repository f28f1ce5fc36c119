// CPU check of the product's fp8 encoder (fe2o3_amd/csrc/fp8_codec.hpp)
// against the oracle's OCP closed form (oracle/fp8.c) over every binary32
// bit pattern.  Test infrastructure: built and run by tests/test_fp8_codec.py.
#include <stdio.h>
#include <string.h>

#include "../fe2o3_amd/csrc/fp8_codec.hpp"

extern "C" unsigned char fe2o3o_fp8e4m3_from_f32(float value);
extern "C" float fe2o3o_fp8e4m3_to_f32(unsigned char bits);

int main() {
  unsigned long long mismatches = 0;
  long long first_bad = -1;
#pragma omp parallel for reduction(+ : mismatches) schedule(static)
  for (long long i = 0; i <= 0xffffffffLL; ++i) {
    const unsigned int bits = (unsigned int)i;
    float f;
    memcpy(&f, &bits, 4);
    const unsigned char want = fe2o3o_fp8e4m3_from_f32(f);
    const unsigned char got = fe2o3::e4m3_from_bits(bits);
    if (got != want) {
      ++mismatches;
#pragma omp critical
      if (first_bad < 0) first_bad = i;
    }
  }
  // the decoder the generic fp8 GEMM stages with: all 256 codes, exact
  unsigned decode_bad = 0;
  for (unsigned q = 0; q < 256; ++q) {
    const unsigned int bits = (unsigned int)fe2o3::bf16_bits_from_e4m3((unsigned char)q) << 16;
    float got;
    memcpy(&got, &bits, 4);
    const float want = fe2o3o_fp8e4m3_to_f32((unsigned char)q);
    unsigned int want_bits;
    memcpy(&want_bits, &want, 4);
    const bool both_nan = got != got && want != want && (bits >> 31) == (want_bits >> 31);
    if (!both_nan && bits != want_bits) ++decode_bad;
  }
  printf("mismatches %llu first %lld decode_mismatches %u\n", mismatches, first_bad, decode_bad);
  return mismatches == 0 && decode_bad == 0 ? 0 : 1;
}
