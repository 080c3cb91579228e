// gq8_lanes.hpp -- cross-lane exchanges of a 64-lane wave without the LDS
// crossbar (gfx950).
//
// __shfl_xor compiles to ds_bpermute, a round trip through the LDS hardware
// of about a hundred clocks; a reduction over 64 lanes takes six of them in
// a row.  The same exchange (lane l receives lane l ^ d) is done here with
// DPP moves inside rows of 16 lanes (distances 1, 2: quad permutes; 8: a
// rotate by 8; 4: rotates by 4 and 12, picked by lane bit 2) and with the
// gfx950 permlane swaps across rows (16, 32).  The pairing is exactly that of
// __shfl_xor, so every reduction keeps its order and its result bit for bit.
// All 64 lanes must be active (every caller is a whole wave).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace gq8 {

template <int D>
__device__ inline uint32_t xor_lane_u32(uint32_t v)
{
    static_assert(D == 1 || D == 2 || D == 4 || D == 8 || D == 16 || D == 32, "a lane distance");
    const int x = (int) v;
    if constexpr (D == 1) {
        return (uint32_t) __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true); // quad_perm [1,0,3,2]
    } else if constexpr (D == 2) {
        return (uint32_t) __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true); // quad_perm [2,3,0,1]
    } else if constexpr (D == 4) {
        const int down = __builtin_amdgcn_mov_dpp(x, 0x124, 0xF, 0xF, true); // row_ror:4
        const int up = __builtin_amdgcn_mov_dpp(x, 0x12C, 0xF, 0xF, true);   // row_ror:12
        return (uint32_t) ((__lane_id() & 4) ? down : up);
    } else if constexpr (D == 8) {
        return (uint32_t) __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true); // row_ror:8
    } else if constexpr (D == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (__lane_id() & 16) ? (uint32_t) r[0] : (uint32_t) r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (__lane_id() & 32) ? (uint32_t) r[0] : (uint32_t) r[1];
    }
}

template <int D>
__device__ inline float xor_lane(float v)
{
    return __uint_as_float(xor_lane_u32<D>(__float_as_uint(v)));
}

template <int D>
__device__ inline int xor_lane(int v)
{
    return (int) xor_lane_u32<D>((uint32_t) v);
}

template <int D>
__device__ inline uint64_t xor_lane(uint64_t v)
{
    const uint32_t lo = xor_lane_u32<D>((uint32_t) v);
    const uint32_t hi = xor_lane_u32<D>((uint32_t) (v >> 32));
    return ((uint64_t) hi << 32) | lo;
}

template <int D>
__device__ inline unsigned long long xor_lane(unsigned long long v)
{
    return (unsigned long long) xor_lane<D>((uint64_t) v);
}

template <int D>
__device__ inline double xor_lane(double v)
{
    return __longlong_as_double((long long) xor_lane<D>((uint64_t) __double_as_longlong(v)));
}

// Butterfly reductions over lane distances D, D / 2, ..., 1 (D = 32: the
// whole wave), in the order of the __shfl_xor loops they replace.
template <int D, typename T>
__device__ inline T sum_lanes(T v)
{
    if constexpr (D >= 1) {
        v += xor_lane<D>(v);
        return sum_lanes<D / 2>(v);
    } else {
        return v;
    }
}

template <int D>
__device__ inline double max_lanes(double v)
{
    if constexpr (D >= 1)
        return max_lanes<D / 2>(fmax(v, xor_lane<D>(v)));
    else
        return v;
}

template <int D>
__device__ inline float max_lanes(float v)
{
    if constexpr (D >= 1)
        return max_lanes<D / 2>(fmaxf(v, xor_lane<D>(v)));
    else
        return v;
}

// max_lanes<D> of K values at once, one exchange distance at a time across
// all K (the same pairing and order for each value), so the K chains
// interleave instead of running one after another.
template <int D, int K>
__device__ inline void max_lanes_each(float (&v)[K])
{
    if constexpr (D >= 1) {
        float other[K];
#pragma unroll
        for (int k = 0; k < K; ++k)
            other[k] = xor_lane<D>(v[k]);
#pragma unroll
        for (int k = 0; k < K; ++k)
            v[k] = fmaxf(v[k], other[k]);
        max_lanes_each<D / 2, K>(v);
    }
}

template <int D>
__device__ inline unsigned long long max_lanes(unsigned long long v)
{
    if constexpr (D >= 1) {
        const unsigned long long other = xor_lane<D>(v);
        return max_lanes<D / 2>(other > v ? other : v);
    } else {
        return v;
    }
}

// The value of a lane known at compile time (a scalar read, no exchange).
__device__ inline double lane_value(double v, int lane)
{
    const uint64_t bits = (uint64_t) __double_as_longlong(v);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) bits, lane);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) (bits >> 32), lane);
    return __longlong_as_double((long long) (((uint64_t) hi << 32) | lo));
}

// acc[r] += s' x part[r], r = 0..3, where s' is the s held by lane N_r of this
// lane's row of 16: v_fmac_f64 with a DPP row_newbcast source operand, so the
// value crosses lanes inside the multiply-add itself (no LDS read, no extra
// instruction).  One rounding, as fma(s', part[r], acc[r]).  The leading
// s_nop 1 gives the two wait states a DPP source needs after a VALU write of
// its register.
template <int N0, int N1, int N2, int N3>
__device__ inline void fmac_row_bcast4(double (&acc)[4], double s, const double (&part)[4])
{
    static_assert(N0 >= 0 && N0 < 16 && N1 >= 0 && N1 < 16 && N2 >= 0 && N2 < 16 && N3 >= 0
                      && N3 < 16,
                  "a lane of the row");
    asm volatile("s_nop 1\n\t"
                 "v_fmac_f64_dpp %0, %4, %5 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f64_dpp %1, %4, %6 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f64_dpp %2, %4, %7 row_newbcast:%11 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f64_dpp %3, %4, %8 row_newbcast:%12 row_mask:0xf bank_mask:0xf"
                 : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
                 : "v"(s), "v"(part[0]), "v"(part[1]), "v"(part[2]), "v"(part[3]),
                   "n"(N0), "n"(N1), "n"(N2), "n"(N3));
}

// acc += s' x part, s' the s held by lane N of this lane's row of 16 (the
// one-accumulator form of fmac_row_bcast4)
template <int N>
__device__ inline void fmac_row_bcast1(double &acc, double s, double part)
{
    static_assert(N >= 0 && N < 16, "a lane of the row");
    asm volatile("s_nop 1\n\t"
                 "v_fmac_f64_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                 : "+v"(acc)
                 : "v"(s), "v"(part), "n"(N));
}

// f(std::integral_constant<int, i>) for i = 0 .. N - 1, in order: a loop body
// with compile-time indices (DPP lane numbers, register arrays)
template <int N, typename F>
__device__ inline void unrolled(F &&f)
{
    if constexpr (N > 0) {
        unrolled<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

} // namespace gq8
