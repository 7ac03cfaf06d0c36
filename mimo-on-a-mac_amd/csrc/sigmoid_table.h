// The bf16 sigmoid table (entry b = bf16(sigmoid(bf16 value with bits b))) as a compile-time constant.
//
// Reference: sigmoid_table engine/mimo_stream/kernels.py:138-146 (a 65,536-entry bf16 lookup of the sigmoid,
// indexed by the bf16 bits of the gate value).  The sigmoid is the specified one of device.h (sigmoid_spec):
// fp32(1 / (1 + exp(-x))) with x clamped to [-200, 200], exp by Cody-Waite reduction by ln 2 (fdlibm split) and
// a degree-13 Taylor polynomial in Horner form, every step one correctly rounded IEEE double operation; NaN ->
// canonical quiet NaN; then round-to-nearest-even to bf16.
//
// Here every step is a constant expression, so the compiler evaluates the whole table (IEEE double arithmetic,
// round to nearest, no contraction in constant evaluation) and the table is data in the code object: nothing is
// built at run time, so the first prefill of a process may be captured in a HIP graph.  Two spellings differ from
// the run-time sigmoid and give the same doubles: rint(v) for |v| < 2^51 as (v + 1.5 * 2^52) - 1.5 * 2^52 (the
// addition rounds to the nearest even integer), and ldexp(p, n) as p times an exact power of two (no product
// here leaves the normal range).  Host builds of this header (the CPU check of the table) use the same clang
// constant evaluator as the device build.
#pragma once
#include <stdint.h>

namespace mimo {
namespace sigtab_gen {

constexpr double rint_c(double v) { return (v + 0x1.8p52) - 0x1.8p52; }

constexpr double pow2_c(int n) {   // 2^n, exact for |n| <= 1022
  double r = 1.0, b = n < 0 ? 0.5 : 2.0;
  for (int m = n < 0 ? -n : n; m; m >>= 1) {
    if (m & 1) r *= b;
    b *= b;
  }
  return r;
}

constexpr double exp_c(double x) {
  const double LN2_HI = 0x1.62e42feep-1;
  const double LN2_LO = 0x1.a39ef35793c76p-33;
  const double INV_LN2 = 0x1.71547652b82fep+0;
  const double n = rint_c(x * INV_LN2);
  const double r = (x - n * LN2_HI) - n * LN2_LO;
  double p = 1.0 / 6227020800.0;             // 1/13!
  p = p * r + 1.0 / 479001600.0;             // 1/12!
  p = p * r + 1.0 / 39916800.0;
  p = p * r + 1.0 / 3628800.0;
  p = p * r + 1.0 / 362880.0;
  p = p * r + 1.0 / 40320.0;
  p = p * r + 1.0 / 5040.0;
  p = p * r + 1.0 / 720.0;
  p = p * r + 1.0 / 120.0;
  p = p * r + 1.0 / 24.0;
  p = p * r + 1.0 / 6.0;
  p = p * r + 0.5;
  p = p * r + 1.0;
  p = p * r + 1.0;
  return p * pow2_c((int)n);
}

constexpr uint16_t entry(uint32_t bits) {
  const float xf = __builtin_bit_cast(float, bits << 16);
  if (xf != xf) return (uint16_t)0x7FC0;     // NaN -> canonical quiet NaN
  double x = (double)xf;
  x = x < -200.0 ? -200.0 : x;
  x = x > 200.0 ? 200.0 : x;
  const float s = (float)(1.0 / (1.0 + exp_c(-x)));
  const uint32_t v = __builtin_bit_cast(uint32_t, s);   // never NaN here: round to nearest even
  return (uint16_t)((v + 0x7FFFu + ((v >> 16) & 1u)) >> 16);
}

struct Table {
  uint16_t v[65536];
};

constexpr Table make() {
  Table t{};
  for (uint32_t i = 0; i < 65536u; ++i) t.v[i] = entry(i);
  return t;
}

}  // namespace sigtab_gen
}  // namespace mimo
