// u15_refrand.cc -- TEST INFRASTRUCTURE ONLY.
//
// The reference tests draw their inputs from std::mt19937 seeded with a
// small integer and std::normal_distribution<float>(0, stddev)
// (tests/u15-kernels-test.cc:110-118, tests/u15-m5-test.cc:87-94).  The
// distribution's algorithm is the standard library's, so this file calls
// the same library rather than restating it: with this toolchain's
// libstdc++ it reproduces the reference tests' inputs value for value.
#include "u15_oracle.h"

#include <random>

extern "C" void
u15o_randn_mt(uint32_t seed, float stddev, size_t n, float* out)
{
  std::mt19937 g(seed);
  std::normal_distribution<float> d(0.0f, stddev);
  for (size_t i = 0; i < n; ++i) { out[i] = d(g); }
}
