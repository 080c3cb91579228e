// gq8_device.hpp -- device helpers shared by the decode kernels: wave
// reductions that keep a fixed summation tree, Int8Blocks weight-block loads,
// agent-scope (cross-XCD coherent) loads and stores, and the tagged words in
// which one workgroup hands a row on to others.
//
// A tagged word is one 64-bit store of a 32-bit value and a 32-bit tag
// (word_tag: the launch's epoch and the row's version), single-copy atomic;
// a reader polls until the word carries the tag it expects, so a hand-over is
// one trip through the memory system.  Every wait is a bounded spin: past
// kWaitSpinLimit polls, or once another wave has set the error word, it gives
// up and sets the error word itself, so a failure ends a launch instead of
// hanging it.
#pragma once

#include "gq8_lanes.hpp"
#include "gq8_numerics.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gq8 {

constexpr int kWaitSpinLimit = 1 << 20;

__device__ inline double wave_sum_d(double v)
{
    return sum_lanes<32>(v);
}

__device__ inline double wave_max_d(double v)
{
    return max_lanes<32>(v);
}

// The merge weights of one head's key splits (MultiQueryAttention.h:43-49),
// one split a lane: lane sp < splits holds split sp's (max, sum).  Returns
// the split's factor exp(max - row max) and leaves the row's total, the sum
// of sum x factor, in `total` (every lane).  Every merge of split partials
// uses this, so they all agree bit for bit.
__device__ inline double merge_factor(double m, double s, bool live, double &total)
{
    const double rowMax = wave_max_d(live ? m : -INFINITY);
    const double f = live ? exp(m - rowMax) : 0.0;
    total = wave_sum_d(live ? s * f : 0.0);
    return f;
}

__device__ inline int dot32(const int4 &w0, const int4 &w1, const int4 &a0, const int4 &a1)
{
    int d = 0;
    d = __builtin_amdgcn_sdot4(w0.x, a0.x, d, false);
    d = __builtin_amdgcn_sdot4(w0.y, a0.y, d, false);
    d = __builtin_amdgcn_sdot4(w0.z, a0.z, d, false);
    d = __builtin_amdgcn_sdot4(w0.w, a0.w, d, false);
    d = __builtin_amdgcn_sdot4(w1.x, a1.x, d, false);
    d = __builtin_amdgcn_sdot4(w1.y, a1.y, d, false);
    d = __builtin_amdgcn_sdot4(w1.z, a1.z, d, false);
    d = __builtin_amdgcn_sdot4(w1.w, a1.w, d, false);
    return d;
}

// Sums U per-lane values (one per row) across the 64 lanes with U - 1 + 6 -
// log2(U) shuffles instead of 6 U: each halving step keeps half of the rows
// and adds the partner lane's share of them.  Returns the total of row
// row_of_lane(lane) (every lane holds one; lanes whose low bits are zero are
// the ones that store).
// One halving step a lane bit, every index fixed at compile time (a runtime
// row count turns v[i] into select chains over the whole array).
template <int N, int Mask, int U>
__device__ inline void reduce_halving(double (&v)[U], int lane)
{
    if constexpr (N > 1) {
        const bool upper = (lane & Mask) != 0;
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            const double keep = upper ? v[i + N / 2] : v[i];
            const double send = upper ? v[i] : v[i + N / 2];
            v[i] = keep + xor_lane<Mask>(send);
        }
        reduce_halving<N / 2, Mask / 2, U>(v, lane);
    } else if constexpr (Mask >= 1) {
        v[0] += xor_lane<Mask>(v[0]);
        reduce_halving<1, Mask / 2, U>(v, lane);
    }
}

template <int U>
__device__ inline double reduce_rows(double (&v)[U], int lane)
{
    static_assert(U >= 1 && U <= 64 && (U & (U - 1)) == 0, "a power of two rows");
    reduce_halving<U, 32, U>(v, lane);
    return v[0];
}

// The row whose total reduce_rows<U> leaves in `lane`: the halving steps
// consume lane bits 5, 4, ... in turn, the upper half of the rows going to
// the lanes with the bit set.
template <int U>
__device__ inline int row_of_lane(int lane)
{
    int row = 0, n = U, bit = 32;
    while (n > 1) {
        n /= 2;
        if (lane & bit)
            row += n;
        bit >>= 1;
    }
    return row;
}

// Whether `lane` is the one that stores its row's total (the lowest lane
// holding it).
template <int U>
__device__ inline bool stores_row(int lane)
{
    int bits = 0, n = U, bit = 32;
    while (n > 1) {
        n /= 2;
        bits |= bit;
        bit >>= 1;
    }
    return (lane & ~bits) == 0;
}

// The lowest lane holding row r's total after reduce_rows<U>.
template <int U>
__device__ inline int lane_of_row(int r)
{
    int lane = 0, n = U, bit = 32;
    while (n > 1) {
        n /= 2;
        if (r >= n) {
            lane |= bit;
            r -= n;
        }
        bit >>= 1;
    }
    return lane;
}

// The 32-byte weight block and fp16 scale of (row, block) in an Int8Blocks
// tensor of `rows` x `inner`.  The loads are unconditional (an invalid pair
// reads block 0 of row 0 with its scale masked to zero) and the scale comes in the
// aligned 32-bit word holding it, so the compiler neither branches around the
// loads nor packs 16-bit results: every load of a wave is in flight before
// the first wait.
struct WeightBlock {
    int4 w0, w1;
    uint32_t scalePair; // the fp16 scale is the high half when `high`
    bool high;
};

__device__ inline WeightBlock load_block(const uint8_t *w8, int64_t rows, int inner, int64_t row,
                                         int block, bool valid)
{
    WeightBlock b;
    const int64_t r = valid ? row : 0;
    const int c = valid ? block : 0;
    const int4 *p = reinterpret_cast<const int4 *>(w8 + r * inner + (int64_t) c * kBlock);
    b.w0 = p[0];
    b.w1 = p[1];
    const int64_t index = r * (inner / kBlock) + c;
    // masking (not selecting) the word keeps the load unconditional; a zero
    // scale zeroes the term
    b.scalePair = reinterpret_cast<const uint32_t *>(w8 + rows * inner)[index >> 1]
                  & (valid ? 0xFFFFFFFFu : 0u);
    b.high = (index & 1) != 0;
    return b;
}

__device__ inline double block_term(const WeightBlock &b, const int4 &a0, const int4 &a1, double sa)
{
    const uint16_t bits = (uint16_t) (b.high ? b.scalePair >> 16 : b.scalePair & 0xFFFFu);
    return (double) dot32(b.w0, b.w1, a0, a1) * ((double) half_value(bits) * sa);
}

// Larger floats give larger keys; NaN gives 0, below every ordered value, so
// it is never chosen (a NaN logit never compares greater in the scan either).
// -0 is folded into +0 first: the two compare equal, so the lower index must
// win between them as between any equal values (Sampler.cpp:60-76).
__device__ inline unsigned long long candidate_key(float value, uint32_t index)
{
    const uint32_t bits = value == 0.f ? 0u : __float_as_uint(value);
    uint32_t key = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    if (value != value)
        key = 0;
    return ((unsigned long long) key << 32) | (unsigned long long) (0xFFFFFFFFu - index);
}

__device__ inline unsigned long long fold_wave_max(unsigned long long c)
{
    return max_lanes<32>(c);
}

__device__ inline uint32_t ld_agent_u(const uint32_t *p)
{
    return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t ld_agent_u64(const uint64_t *p)
{
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int ld_agent_i(const int *p)
{
    return __hip_atomic_load(const_cast<int *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent_i(int *p, int v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes at byte `offset` of a `bytes`-long buffer, with an agent-coherent
// (sc1) buffer load; bytes past the end read as zero.
constexpr int kCoherentLoad = 16; // the sc1 cache-policy bit of a buffer load
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
__device__ inline v4u ld_agent_16(const void *base, uint32_t offset, uint32_t bytes)
{
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int) bytes, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int) offset, 0, kCoherentLoad);
}

// 16 bytes to byte `offset` of a `bytes`-long buffer with an agent-coherent
// (sc1) buffer store; a store past the end is dropped.
__device__ inline void st_agent_16(void *base, uint32_t offset, uint32_t bytes, v4u value)
{
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, (int) bytes, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b128(value, r, (int) offset, 0, kCoherentLoad);
}

// A double and the tag as two tagged words in one 16-byte store: (low half,
// tag, high half, tag).  A reader checks both tags, so a store seen half
// done is read again.
__device__ inline v4u tagged_double(double d, uint32_t tag)
{
    const uint64_t bits = (uint64_t) __double_as_longlong(d);
    v4u v;
    v.x = (uint32_t) bits;
    v.y = tag;
    v.z = (uint32_t) (bits >> 32);
    v.w = tag;
    return v;
}

// ---- tagged words -----------------------------------------------------------
// tag = epoch << 8 | version.  Versions of the residual row: 0 the embedding
// row, 2 l + 1 after layer l's o projection, 2 l + 2 after its down
// projection; every other row has the layer as its version.
__device__ inline uint32_t word_tag(uint32_t epoch, int version)
{
    return (epoch << 8) | (uint32_t) version;
}

__device__ inline void ll_put(uint64_t *p, uint32_t value, uint32_t tag)
{
    __hip_atomic_store(p, ((uint64_t) tag << 32) | value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline bool wait_give_up(const int *error, int &spins)
{
    if ((++spins & 63) == 0 && (ld_agent_i(error) != 0 || spins > kWaitSpinLimit)) {
        __hip_atomic_fetch_or(const_cast<int *>(error), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
    __builtin_amdgcn_s_sleep(1);
    return false;
}

// The value of word `p` once it carries `tag`; false after giving up.
__device__ inline bool ll_get(const uint64_t *p, uint32_t tag, const int *error, uint32_t &value)
{
    int spins = 0;
    for (;;) {
        const uint64_t w = ld_agent_u64(p);
        if ((uint32_t) (w >> 32) == tag) {
            value = (uint32_t) w;
            return true;
        }
        if (wait_give_up(error, spins))
            return false;
    }
}

// Words `word` and `word + 1` (word even) of a `words`-long row; a second word
// past the end is not waited for.
__device__ inline bool ll_get2(const uint64_t *row, int word, int words, uint32_t tag, const int *error,
                               uint32_t &v0, uint32_t &v1)
{
    int spins = 0;
    for (;;) {
        const v4u w = ld_agent_16(row, (uint32_t) word * 8, (uint32_t) words * 8);
        if (w.y == tag && (word + 1 >= words || w.w == tag)) {
            v0 = w.x;
            v1 = w.z;
            return true;
        }
        if (wait_give_up(error, spins))
            return false;
    }
}

} // namespace gq8
