// ref_shim.cc -- TEST INFRASTRUCTURE ONLY.
//
// Exposes the reference's own CPU functions, compiled from
// /root/reference/src/u15-ref.cc where it lies (never copied), under C
// names so the oracle tests can call them through ctypes:
//   u15ref_linear -> u15::ref::linear   (src/u15-ref.h:33-36, u15-ref.cc:33-49)
//   u15ref_silu   -> u15::ref::silu     (src/u15-ref.h:38, u15-ref.cc:51-58)
#include "u15-ref.h"

extern "C" void
u15ref_linear(const float* x, const float* w, const float* b,
              std::size_t rows, std::size_t in_dim, std::size_t out_dim,
              float* out)
{
  u15::ref::linear(x, w, b, rows, in_dim, out_dim, out);
}

extern "C" void
u15ref_silu(float* x, std::size_t n)
{
  u15::ref::silu(x, n);
}
