// gq8_numerics.hpp -- the scalar arithmetic every gq8 kernel shares, written
// once for the device and the host (the host side is what the CPU unit tests
// exercise against the oracle without a GPU).
//
// Rule of the path: each operation is evaluated in IEEE double and rounded to
// fp32 at the points where the reference's decoder stores an fp32 buffer;
// int8 dot products are exact.  Floating-point contraction is switched off in
// these helpers so an expression is evaluated exactly as it is written.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#define GQ8_HD __host__ __device__ inline

namespace gq8 {
// A double constant held in a scalar register pair on the device: a VALU
// fused multiply-add then reads it as its addend, where a literal addend is
// rebuilt in the destination register by two v_mov_b32 before each
// v_fmac_f64.  The value is unchanged; the host pass takes it as it is.
__host__ __device__ inline double scalar_constant(double c)
{
#if defined(__HIP_DEVICE_COMPILE__)
    asm("" : "=s"(c) : "0"(c));
#endif
    return c;
}
} // namespace gq8
#define GQ8_CONST(c) ::gq8::scalar_constant(c)

#include "gq8_tanh.hpp"

namespace gq8 {

constexpr int kBlock = 32;          // Int8Blocks.h:56
constexpr float kLargestQuantized = 127.0f;

// IEEE binary16 round-to-nearest-even, via the compiler's _Float16 conversion
// (v_cvt_f16_f32 on gfx950, the libgcc soft conversion on the host).
GQ8_HD uint16_t half_bits(float value)
{
    _Float16 h = (_Float16) value;
    return __builtin_bit_cast(uint16_t, h);
}

GQ8_HD float half_value(uint16_t bits)
{
    return (float) __builtin_bit_cast(_Float16, bits);
}

// blockScaleBits (Lib/HuggingFaceEACP/Kernels/Int8Blocks.cpp:25-36) from a
// block's largest magnitude: amax / 127 as a float division, narrowed to fp16;
// a scale that is zero, infinite or NaN is stored as zero.  The quotient is
// found without a division: the double product amax * (1 / 127) is within
// 2^-52 (relative) of the exact quotient, and the exact quotient lies at least
// 2^-32 (relative) from every fp32 rounding midpoint (its distance from one is
// |t - 127 (2 j + 1)| / (127 2^24) of the fp32 spacing, with t an even
// integer), so both round to the same fp32: the correctly rounded quotient.
GQ8_HD uint16_t scale_bits_from_amax(float amax)
{
#pragma clang fp contract(off)
    const float quotient = (float) ((double) amax * (1.0 / (double) kLargestQuantized));
    const uint16_t bits = half_bits(quotient);
    const float scale = half_value(bits);
    return (scale > 0.f && scale <= 65504.f) ? bits : (uint16_t) 0;
}

// quantizedByte (Int8Blocks.cpp:41-47): nearbyint((double) x / (double) s)
// clamped to [-127, 127], with s the fp16 scale (positive, finite).  The double
// quotient of two such numbers never lands on or across a half-integer the
// exact quotient is not on (the exact distance from a tie is at least 2^-25,
// its rounding error at most 2^-45), so this is round-half-even of the exact
// quotient; it is found here without a division: a candidate from the fp32
// product x * (1 / s) is within one of it, and the exact fp32 products
// (k +- 0.5) * s (at most 10 + 11 significant bits) say which side of each
// boundary x lies on.  A NaN element is stored as zero.  Written without
// branches: the two corrections exclude each other (hi > lo), and a kernel
// quantizing several elements a thread then interleaves them instead of
// running each element's branches in turn.
GQ8_HD int quantize_value(float x, float scale, float inverse)
{
#pragma clang fp contract(off)
    const float k = fminf(fmaxf(rintf(x * inverse), -256.f), 256.f); // NaN x: -256, discarded
    const float hi = (k + 0.5f) * scale;
    const float lo = (k - 0.5f) * scale;
    const bool kOdd = ((int) k & 1) != 0;
    const float up = (x > hi || (x == hi && kOdd)) ? 1.f : 0.f;
    const float down = (x < lo || (x == lo && kOdd)) ? 1.f : 0.f;
    const int q = (int) fminf(fmaxf(k + up - down, -127.f), 127.f);
    return x == x ? q : 0;
}

// quantize_value of an element of a block whose fp16 scale bits are `bits`:
// a block stored with a zero scale holds zero bytes.  The scale's test masks
// the result rather than guarding the arithmetic, so the compiler does not
// turn it into a branch around each element.
GQ8_HD int quantize_in_block(float x, uint16_t bits, float scale, float inverse)
{
    return quantize_value(x, scale, inverse) & (bits ? -1 : 0);
}

// Takes kernel arguments into scalar registers where it stands (kernel entry):
// left to itself the compiler loads an argument just before its first use,
// and a use late in a kernel then waits on a fresh scalar-cache line of the
// argument segment, which a weight stream may have pushed out of the L2.
#define GQ8_ARGS_EARLY(...) asm volatile("" ::__VA_ARGS__)

// The candidate hint of quantize_value on the device: a reciprocal of the
// fp16 scale good to an ulp (v_rcp_f32).  The exact boundary compares above
// make the quantized value independent of the hint as long as the candidate
// lands within one of the exact quotient, which an ulp of error at
// |x / s| <= 256 keeps.
__device__ inline float quantize_hint(float scale)
{
    return __builtin_amdgcn_rcpf(scale);
}

// tanh GELU (Lib/HuggingFaceEACP/Kernels/Gelu.h:27-46, double constants of
// Tests/Kernels/Common.h:170-175), the tanh argument saturating at |z| >= 10;
// tanh from the exponential (gq8_tanh.hpp), within a few ulps of libm's.
GQ8_HD double tanh_gelu(double x)
{
#pragma clang fp contract(off)
    const double rootTwoOverPi = GQ8_CONST(0.7978845608028654);
    const double inner = rootTwoOverPi * (x + GQ8_CONST(0.044715) * x * x * x);
    const double t = inner >= 10.0 ? 1.0 : (inner <= -10.0 ? -1.0 : tanh_from_exp(inner));
    return 0.5 * x * (1.0 + t);
}

GQ8_HD float geglu(float gate, float up)
{
#pragma clang fp contract(off)
    return (float) (tanh_gelu((double) gate) * (double) up);
}

// One rotate-half pair (RoPE.h:7-20, 59-81) in double, rounded once.
GQ8_HD void rotate_pair(float lo, float hi, float c, float s, float *outLo, float *outHi)
{
#pragma clang fp contract(off)
    const double dl = (double) lo, dh = (double) hi, dc = (double) c, ds = (double) s;
    *outLo = (float) (dl * dc - dh * ds);
    *outHi = (float) (dh * dc + dl * ds);
}

// x * scale * (1 + w) of RMSNorm (RMSNorm.h:44-56), scale = 1/sqrt(mean+eps).
GQ8_HD float norm_value(float x, double scale, float weight)
{
#pragma clang fp contract(off)
    return (float) (((double) x * scale) * (1.0 + (double) weight));
}

// A width that is a power of two divides by an exact scaling (the same
// double as the division, without its iteration).
GQ8_HD double norm_scale(double squares, int n, float epsilon)
{
#pragma clang fp contract(off)
    const double mean = (n & (n - 1)) == 0 ? ldexp(squares, -__builtin_ctz((unsigned) n))
                                           : squares / (double) n;
    return 1.0 / sqrt(mean + (double) epsilon);
}

} // namespace gq8
