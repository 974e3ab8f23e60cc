// fp64 exp on a non-positive argument, shared by the device kernels and a
// CPU unit test (it compiles as plain C++ without the HIP headers).
//
// Tang's table-driven method (P. T. P. Tang, "Table-driven implementation of
// the exponential function in IEEE floating-point arithmetic", ACM TOMS
// 15(2), 1989): t = (64 e + j) ln2/64 + r with |r| <= ln2/128, so
// exp(t) = 2^e * 2^(j/64) * exp(r).  The reduction is exact: t - k*L_hi is
// one fused multiply-add whose exact value fits a double (L_hi's last bit is
// 2^-59 and |r| < 2^-7), then the tail k*L_lo is subtracted.  exp(r) - 1 is
// its degree-5 Taylor polynomial (truncation below 3.6e-17 for
// |r| <= ln2/128) and 2^(j/64) the correctly rounded table entry, so the
// result is within a few ulps of exp(t).  k = rint(t * 64/ln2) comes from
// adding 1.5 * 2^52, which leaves k in the low word of the sum.  The
// argument is first clamped to -746 (one max): every t <= -745.14 gives
// exactly 0, -inf included, and NaN also gives 0 (callers see NaN inputs
// through their row sums, which the NaN itself makes NaN).
#pragma once

#if defined(__HIPCC__)
#define NSV_EXP_FN __host__ __device__ __forceinline__
#else
#include <cmath>
#include <cstdint>
#define NSV_EXP_FN inline
#endif

// 2^(j/64), j = 0..63, each the double nearest the exact value
constexpr double kExp2Frac64[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

NSV_EXP_FN double nsv_exp_nonpos(double t, const double* tab) {
  constexpr double kShift = 0x1.8p52;  // adding it rounds to an integer, kept in the low word
  constexpr double kInvL = 0x1.71547652b82fep+6;  // 64 / ln 2 (only picks k)
  constexpr double kLhi = 0x1.62e42fefa39efp-7;   // ln2/64 rounded to a double
  constexpr double kLlo = 0x1.abc9e3b39803fp-62;   // ln2/64 - kLhi
  t = fmax(t, -746.0);
  const double kd = fma(t, kInvL, kShift);
  const int k = (int)(uint32_t)__builtin_bit_cast(unsigned long long, kd);
  const double kf = kd - kShift;
  double r = fma(-kf, kLhi, t);
  r = fma(-kf, kLlo, r);
  double p = fma(fma(fma(1.0 / 120.0, r, 1.0 / 24.0), r, 1.0 / 6.0), r, 0.5);
  p = fma(p, r * r, r);
  const double tj = tab[k & 63];
  return ldexp(fma(tj, p, tj), k >> 6);
}
