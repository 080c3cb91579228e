// gq8_tanh.hpp -- tanh in double from the exponential, for the GeGLU.
//
// tanh|x| = expm1(z) / (expm1(z) + 2), z = 2|x| (the identity tanh y =
// (e^{2y} - 1) / (e^{2y} + 1) with the numerator kept free of cancellation).
// expm1(z) by Cody-Waite range reduction, z = n ln2 + r with |r| <= ln2/2
// (ln2 split into a 32-significant-bit head, so n * head is exact for the
// n this range needs, and a tail), then
//   expm1(z) = 2^n (1 + p(r)) - 1 = 2^n p(r) + (2^n - 1),
// where p(r) = expm1(r) is its Taylor series to r^13 by Horner's rule with
// fused multiply-adds (the truncation is below 2^-56 of p at |r| <= ln2/2).
// About 25 double operations in place of the library's tanh; a few ulps
// from the correctly rounded value over the GeGLU's range |x| < 10
// (tests/test_tanh.py holds it to libm's tanh).
//
// Plain C++ (fma, rint, ldexp, fabs, copysign) so the host tests can build it
// without HIP; GQ8_HD makes it a host and device function under hipcc.
#pragma once

#include <cmath>

#ifndef GQ8_HD
#define GQ8_HD inline
#endif
// GQ8_CONST(c): a constant as its callers want it held (the device build
// keeps it in scalar registers, where a fused multiply-add reads it as an
// operand); the constant itself unchanged
#ifndef GQ8_CONST
#define GQ8_CONST(c) (c)
#endif

namespace gq8 {

GQ8_HD double tanh_from_exp(double x)
{
    const double ln2Head = GQ8_CONST(0x1.62e42feep-1);       // ln2 to 32 significant bits
    const double ln2Tail = GQ8_CONST(0x1.a39ef35793c76p-33); // ln2 - head
    const double invLn2 = GQ8_CONST(1.4426950408889634);
    const double z = 2.0 * fabs(x);
    const double n = rint(z * invLn2);
    const double r = fma(-n, ln2Tail, fma(-n, ln2Head, z));
    double p = GQ8_CONST(1.6059043836821613e-10);     // 1/13!
    p = fma(p, r, GQ8_CONST(2.08767569878681e-09));   // 1/12!
    p = fma(p, r, GQ8_CONST(2.505210838544172e-08));  // 1/11!
    p = fma(p, r, GQ8_CONST(2.755731922398589e-07));  // 1/10!
    p = fma(p, r, GQ8_CONST(2.7557319223985893e-06)); // 1/9!
    p = fma(p, r, GQ8_CONST(2.48015873015873e-05));   // 1/8!
    p = fma(p, r, GQ8_CONST(0.0001984126984126984));  // 1/7!
    p = fma(p, r, GQ8_CONST(0.001388888888888889));   // 1/6!
    p = fma(p, r, GQ8_CONST(0.008333333333333333));   // 1/5!
    p = fma(p, r, GQ8_CONST(0.041666666666666664));   // 1/4!
    p = fma(p, r, GQ8_CONST(0.16666666666666666));    // 1/3!
    p = fma(p, r, 0.5);                               // 1/2!
    p = fma(p, r, 1.0);                               // 1/1!
    p = p * r;                                        // expm1(r)
    const double scale = ldexp(1.0, (int) n);
    const double em1 = fma(scale, p, scale - 1.0);
    return copysign(em1 / (em1 + 2.0), x);
}

} // namespace gq8
