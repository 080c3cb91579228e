// gq8_decode.hip -- the fused kernels of a one-token decode step.
//
// A decode step is a chain of global dependencies (every product needs the
// whole of its input row), so its cost on MI355X is the weight bytes plus a
// fixed cost per kernel boundary.  These kernels cut the chain to five
// kernels a layer and three for the head:
//
//   qkv_rope_kernel      norm + Q8 of the hidden row (per workgroup, in LDS),
//                        the fused q|k|v product, RoPE on q and k, k and v
//                        stored fp16 at the step's cache row (layer 0 also
//                        gathers the embedding row);
//   attention_kernel     split-key attention over the fp16 cache with an
//                        online softmax; the last workgroup of a row merges
//                        the splits and writes the Q8 row for o_proj;
//   (o_proj, down)       q8_matvec_kernel with the residual add;
//   gateup_geglu_kernel  norm + Q8 prologue, the gate|up product, GeGLU and
//                        the Q8 row for down_proj;
//   (final norm)         rmsnorm_kernel: the final norm and its Q8 row;
//   lmhead_argmax_kernel the tied lm_head over the whole vocabulary, each
//                        workgroup's first maximum merged into one packed
//                        64-bit word by atomicMax;
//   head_finalize_kernel the id into the next sequence slot and the position
//                        advance.
//
// Reference counterparts: Decoder.cpp:579-706 (the layer), Embed.h, RMSNorm.h,
// RoPE.h, Linear.h, MultiQueryAttention.h, GeGLU.h, Argmax.h.  The arithmetic
// is gq8_numerics.hpp's, identical to the unfused kernels'.
#include "gq8_decode.hpp"
#include "gq8_device.hpp"
#include "gq8_numerics.hpp"

#include <algorithm>
#include <cfloat>

#include "gq8_lanes.hpp"

namespace gq8 {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// The Q8 form of one normalised row, shared by a workgroup.
struct RowQ8 {
    int8_t q[kFusedMaxWidth];
    double scale[kFusedMaxWidth / kBlock];
};

// RMSNorm (RMSNorm.h:44-56) of one row and its Int8Blocks quantization into
// LDS, in two parts so that a kernel can issue the row's loads before its
// weight loads (the loads of one wave complete in order, so the norm then
// runs while the weights stream in).  Thread t owns elements [E t, E t + E)
// (E = 8 for 256-thread workgroups, 4 for 512), so 32 / E consecutive lanes
// hold one 32-element block.  The row is either x or, with `table`, the
// embedding row of `*token` (Embed.h:45-82), which workgroup 0 also stores to
// hidden_out for the residual stream.
template <int E>
struct RowSlice {
    float v[E];
    float w[E];
    bool active;
};

template <int E>
__device__ inline void load4(const float *p, float *out)
{
#pragma unroll
    for (int k = 0; k < E; k += 4) {
        const float4 f = reinterpret_cast<const float4 *>(p)[k / 4];
        out[k] = f.x;
        out[k + 1] = f.y;
        out[k + 2] = f.z;
        out[k + 3] = f.w;
    }
}

template <int E>
__device__ inline RowSlice<E> load_row_slice(const float *x, const uint32_t *token,
                                             const uint8_t *table, int64_t vocab,
                                             float embed_scale, float *hidden_out,
                                             const float *weight, int width)
{
    static_assert(E == 4 || E == 8, "four or eight elements a thread");
    // branch-free: an inactive thread reads elements [0, E) and is zeroed at use
    RowSlice<E> r;
    const int t = threadIdx.x;
    r.active = t * E < width;
    const int i0 = r.active ? t * E : 0;
    load4<E>(weight + i0, r.w);
    if (table) {
        uint32_t id = *token; // the sequence slot at the position
        if (id >= (uint32_t) vocab) // ids are validated on the host; a guard, not a rule
            id = 0;
        const int64_t e0 = (int64_t) id * width + i0;
        const uint16_t bits = reinterpret_cast<const uint16_t *>(table + vocab * width)[e0 / kBlock];
        const float s = half_value(bits);
        int8_t b[E];
        if (E == 8) {
            const int2 packed = *reinterpret_cast<const int2 *>(table + e0);
            __builtin_memcpy(b, &packed, E);
        } else {
            const int packed = *reinterpret_cast<const int *>(table + e0);
            __builtin_memcpy(b, &packed, E);
        }
#pragma unroll
        for (int k = 0; k < E; ++k)
            r.v[k] = (float) ((double) embed_scale * (double) (s * (float) b[k]));
        if (hidden_out && blockIdx.x == 0 && r.active)
#pragma unroll
            for (int k = 0; k < E; k += 4)
                reinterpret_cast<float4 *>(hidden_out + i0)[k / 4] =
                    make_float4(r.v[k], r.v[k + 1], r.v[k + 2], r.v[k + 3]);
    } else {
        load4<E>(x + i0, r.v);
    }
    return r;
}

// The norm of the loaded slices and the Q8 row in LDS.  Workgroup 0
// optionally writes the normalised row (fp32) and its Q8 bytes (the debug
// view and the final-norm outputs).
template <int E>
__device__ void norm_q8_finish(const RowSlice<E> &r, int width, float epsilon, RowQ8 &row,
                               double *sPartial, float *normalised_out, uint8_t *q8_out)
{
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // a workgroup covers the widest row with E elements a thread; a compile-
    // time count (reading blockDim would be a scalar load from the kernel's
    // implicit arguments, waited for at the first barrier)
    constexpr int waves = kFusedMaxWidth / E / 64;
    const int i0 = t * E;
    float v[E];
#pragma unroll
    for (int k = 0; k < E; ++k)
        v[k] = r.active ? r.v[k] : 0.f;
    double squares = 0.0;
#pragma unroll
    for (int k = 0; k < E; ++k)
        squares += (double) v[k] * (double) v[k];
    squares = wave_sum_d(squares);
    if (lane == 0)
        sPartial[wave] = squares;
    __syncthreads();
    double total = 0.0;
    for (int w = 0; w < waves; ++w)
        total += sPartial[w];
    const double scale = norm_scale(total, width, epsilon);

    float n[E];
    float amax = 0.f;
#pragma unroll
    for (int k = 0; k < E; ++k) {
        n[k] = r.active ? norm_value(v[k], scale, r.w[k]) : 0.f;
        amax = fmaxf(amax, fabsf(n[k]));
    }
    amax = max_lanes<kBlock / E / 2>(amax);
    const uint16_t bits = scale_bits_from_amax(amax);
    const float s = half_value(bits);
    const float inverse = bits ? quantize_hint(s) : 0.f;
    int packed[E / 4] = {};
#pragma unroll
    for (int k = 0; k < E; ++k) {
        const int q = quantize_in_block(n[k], bits, s, inverse);
        packed[k / 4] |= (q & 0xFF) << (8 * (k % 4));
    }
    const bool first = (t % (kBlock / E)) == 0; // the block's first thread
    if (r.active) {
        __builtin_memcpy(row.q + i0, packed, E);
        if (first)
            row.scale[i0 / kBlock] = (double) s;
        if (blockIdx.x == 0) {
            if (normalised_out)
#pragma unroll
                for (int k = 0; k < E; ++k)
                    normalised_out[i0 + k] = n[k];
            if (q8_out) {
                __builtin_memcpy(q8_out + i0, packed, E);
                if (first)
                    reinterpret_cast<uint16_t *>(q8_out + width)[i0 / kBlock] = bits;
            }
        }
    }
    __syncthreads();
}

// ---- q|k|v + RoPE + fp16 KV ---------------------------------------------------
// A pair task is the two rows (i, i + half) of one head of q, k or v; a wave
// owns kPairsPerWave of them.  Lane l owns block l of every row (width <= 2048).
constexpr int kPairsPerWave = 1;

// Embed: the first layer, which gathers its row from the embedding table at
// the id in the position's sequence slot (the position is then needed before
// the row loads); the other layers load the residual row.
template <bool Embed>
__global__ __launch_bounds__(kThreads) void qkv_rope_kernel(QkvArgs a)
{
    __shared__ RowQ8 row;
    __shared__ double sPartial[kWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int half = a.head_dim / 2;
    const int qWidth = a.heads * a.head_dim, kvWidth = a.kv_heads * a.head_dim;
    const int outputs = qWidth + 2 * kvWidth;
    const int pairs = (a.heads + 2 * a.kv_heads) * half;
    const int nb = a.width / kBlock;
    const int firstPair = (blockIdx.x * kWaves + wave) * kPairsPerWave;

    // The position is requested first, with a vector load: the rotation's
    // table rows depend on it, and a scalar load still in flight would hold
    // up the norm's LDS waits (LDS and scalar memory share one wait counter).
    // Past the first layer it is not waited for until the row and weight
    // loads are issued.
    const int positionLoaded = ld_agent_i(a.position);
    int position = 0;
    RowSlice<8> slice;
    if constexpr (Embed) {
        position = __builtin_amdgcn_readfirstlane(positionLoaded);
        slice = load_row_slice<8>(nullptr, a.sequence + position, a.embedding, a.vocab,
                                  a.embed_scale, a.hidden_out, a.norm_weight, a.width);
    } else {
        slice = load_row_slice<8>(a.hidden, nullptr, nullptr, 0, 0.f, nullptr, a.norm_weight,
                                  a.width);
    }
    WeightBlock lo[kPairsPerWave], hi[kPairsPerWave];
    int rowLo[kPairsPerWave];
#pragma unroll
    for (int p = 0; p < kPairsPerWave; ++p) {
        const int pair = firstPair + p;
        const int head = pair / half, i = pair % half;
        rowLo[p] = head * a.head_dim + i; // q heads, then k heads, then v heads
        const bool valid = pair < pairs && lane < nb;
        lo[p] = load_block(a.weights, outputs, a.width, rowLo[p], lane, valid);
        hi[p] = load_block(a.weights, outputs, a.width, rowLo[p] + half, lane, valid);
    }
    __builtin_amdgcn_sched_barrier(0); // every load issued before the norm's first wait
    if constexpr (!Embed)
        position = __builtin_amdgcn_readfirstlane(positionLoaded);

    // the rotation of this wave's pairs, fetched while the weights stream in,
    // with vector loads (every lane the same address), so that the norm's
    // LDS waits below do not wait for them
    float cosine[kPairsPerWave], sine[kPairsPerWave];
#pragma unroll
    for (int p = 0; p < kPairsPerWave; ++p) {
        const int pair = firstPair + p;
        const int64_t angle = (int64_t) position * half + (pair < pairs ? pair % half : 0);
        cosine[p] = __builtin_nontemporal_load(a.cosines + angle);
        sine[p] = __builtin_nontemporal_load(a.sines + angle);
    }

    norm_q8_finish(slice, a.width, a.epsilon, row, sPartial, a.debug_normalised, a.debug_q8);

    int4 a0 = make_int4(0, 0, 0, 0), a1 = a0;
    double sa = 0.0;
    if (lane < nb) {
        a0 = reinterpret_cast<const int4 *>(row.q + lane * kBlock)[0];
        a1 = reinterpret_cast<const int4 *>(row.q + lane * kBlock)[1];
        sa = row.scale[lane];
    }
    constexpr int kRows = 2 * kPairsPerWave;
    double y[kRows];
#pragma unroll
    for (int p = 0; p < kPairsPerWave; ++p) {
        y[2 * p] = block_term(lo[p], a0, a1, sa);
        y[2 * p + 1] = block_term(hi[p], a0, a1, sa);
    }
    const double total = reduce_rows<kRows>(y, lane);
    double rowTotal[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
        rowTotal[r] = lane_value(total, lane_of_row<kRows>(r));
#pragma unroll
    for (int p = 0; p < kPairsPerWave; ++p) {
        const double yLo = rowTotal[2 * p], yHi = rowTotal[2 * p + 1];
        const int pair = firstPair + p;
        if (lane != 0 || pair >= pairs)
            continue;
        const int r = rowLo[p];
        const float fLo = (float) yLo, fHi = (float) yHi; // the product's fp32 outputs
        if (r < qWidth) {
            float outLo, outHi;
            rotate_pair(fLo, fHi, cosine[p], sine[p], &outLo, &outHi);
            a.query[r] = outLo;
            a.query[r + half] = outHi;
        } else if (r < qWidth + kvWidth) {
            float outLo, outHi;
            rotate_pair(fLo, fHi, cosine[p], sine[p], &outLo, &outHi);
            uint16_t *keys = a.key_cache + (int64_t) position * kvWidth + (r - qWidth);
            keys[0] = half_bits(outLo);
            keys[half] = half_bits(outHi);
        } else {
            uint16_t *values = a.value_cache + (int64_t) position * kvWidth + (r - qWidth - kvWidth);
            values[0] = half_bits(fLo);
            values[half] = half_bits(fHi);
        }
    }
    // the tag of the attention launch after this one
    if (blockIdx.x == 0 && threadIdx.x == 0 && a.tag_epoch)
        a.tag_epoch[0] += 1;
}

// ---- split-key attention, merged per head group by its live splits -------------
// The grid is (key split, head group).  A workgroup of eight waves owns the
// keys [k0, k0 + n) of one split and the G heads of one group (G = 1 when a
// head is at least a 32-element block wide, else the heads of one block).
// Lane l owns channels [C l, C l + C) of a head, so the query lives in
// registers and no LDS staging is needed.  Keys go in rounds of 8 B (B = 4
// or 8 keys a wave, by the launch's key-count range), wave w taking keys w,
// w + 8, ..., w + 8 (B - 1) of a round:
//   scores   the round's keys and values are loaded at once; the B keys'
//            per-lane partial dots (C channels, every head of the group) are
//            summed across the wave together (reduce_rows);
//   softmax  wave g takes head g: the split's maximum, exp(s - max) and sum;
//   values   the same keys (the first round's values still in registers);
//            the eight waves' sums are added in LDS, in wave order.
// The split's partial (double) and its (max, sum) are stored as tagged words
// (a 32-bit half and the launch's tag in one single-copy-atomic agent-scope
// store, coherent across the chip's L2s); the tag is an epoch the q|k|v
// launch before advances, so no word is ever cleared.  The group's live
// splits then merge its 32-channel blocks among themselves (split s takes
// blocks s, s + splits, ...; a wave a block, a lane a channel): each polls
// the words it needs until they carry the tag, with a bounded wait that sets
// the error word when it gives up.  No workgroup takes a ticket or reads the
// whole group's partials.  The merge (MultiQueryAttention.h:43-49: every
// split rescaled to the row maximum in split order, the sums divided by the
// total) rounds to fp32 and quantizes the block.  The splits of a launch
// wait on each other, so its workgroups must be resident together: the
// kernel is held to four waves a SIMD (at most 128 VGPRs), two 512-thread
// workgroups a compute unit, and the largest launch is 64 splits x 8 heads =
// 512 workgroups.  Scores, weights and sums are double throughout.
constexpr int kAttnThreads = 512;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kScoreBatch = 8;                          // keys a wave takes a round
constexpr int kRoundKeys = kAttnWaves * kScoreBatch;    // 64
constexpr int kMaxSplitKeys = 256;                      // so the window is at most 16384
constexpr int kMaxGroupWidth = 256;                     // G * head_dim
constexpr int kPollSplits = 8; // split partials a merging lane polls at once (a run of at most 64 / 8)

struct SplitPlan {
    int splits, perSplit;
};

// Whole rounds a split, as few as the launch's gridSplits splits allow.
__device__ inline SplitPlan plan_splits(int keyCount, int gridSplits, int roundKeys)
{
    const int roundsPerSplit =
        (keyCount + roundKeys * gridSplits - 1) / (roundKeys * gridSplits);
    const int perSplit = roundsPerSplit * roundKeys;
    return {(keyCount + perSplit - 1) / perSplit, perSplit};
}

// C consecutive halves of an fp16 row.
template <int C>
__device__ inline void load_halves(const uint16_t *p, uint16_t (&h)[C])
{
    if constexpr (C == 4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        h[0] = (uint16_t) (v.x & 0xFFFFu); h[1] = (uint16_t) (v.x >> 16);
        h[2] = (uint16_t) (v.y & 0xFFFFu); h[3] = (uint16_t) (v.y >> 16);
    } else if constexpr (C == 2) {
        const uint32_t v = *reinterpret_cast<const uint32_t *>(p);
        h[0] = (uint16_t) (v & 0xFFFFu); h[1] = (uint16_t) (v >> 16);
    } else {
        h[0] = *p;
    }
}

// The same C halves kept as loaded, (C + 1) / 2 words (half the registers of
// one a half), and half i of them.
template <int C>
__device__ inline void load_words(const uint16_t *p, uint32_t (&w)[(C + 1) / 2])
{
    if constexpr (C == 4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        w[0] = v.x;
        w[1] = v.y;
    } else if constexpr (C == 2) {
        w[0] = *reinterpret_cast<const uint32_t *>(p);
    } else {
        w[0] = *p;
    }
}

template <int C>
__device__ inline double word_half(const uint32_t (&w)[(C + 1) / 2], int i)
{
    return (double) half_value((uint16_t) (w[i >> 1] >> (16 * (i & 1))));
}

template <int C, int G, int B>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(4)))
void attention_kernel(AttentionArgs a)
{
    GQ8_ARGS_EARLY("s"(a.grid_splits), "s"(a.scale), "s"(a.part_ll), "s"(a.ml_ll), "s"(a.tag_epoch),
                   "s"(a.error), "s"(a.out), "s"(a.q8));
    constexpr int kRound = kAttnWaves * B; // keys a round: B a wave
    constexpr int kRows = B * G; // reduce_rows width: (key, head) pairs
    __shared__ double sScore[G][kMaxSplitKeys];
    __shared__ double sAcc[kAttnWaves][kMaxGroupWidth];
    __shared__ double sMax[G], sSum[G];
    __shared__ double sSplitMax[G][kDecodeSplits];

    // a 1-D grid: the head groups' splits, a group's splits consecutive
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hd = a.head_dim, kvWidth = a.kv_heads * hd;
    const int heads = a.heads, qWidth = heads * hd;
    const int perKv = heads / a.kv_heads;
    const int group = (int) blockIdx.x / a.grid_splits, h0 = group * G;
    const int groupWidth = G * hd;
    const int split = (int) blockIdx.x % a.grid_splits;

    // the query channels of this lane, before the position is known
    // (unconditional loads, masked: a selected load would be sunk into a
    // branch and waited for on its own)
    const bool active = lane * C < hd;
    const int c0 = active ? lane * C : 0;
    const uint32_t keep = active ? 0xFFFFFFFFu : 0u;
    double q[G][C];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < C; ++i)
            q[g][i] = (double) __uint_as_float(__float_as_uint(a.query[(h0 + g) * hd + c0 + i]) & keep);

    int kvOffset[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
        kvOffset[g] = ((h0 + g) / perKv) * hd + c0;

    // Split s is expected to be the keys [s S, s S + S) (S = spec_keys: one
    // round of 64 while at most grid_splits rounds are attended, two while at
    // most 2 grid_splits are): its rows are loaded before the position arrives
    // (rows past the position are read, inside the cache, and never used), so
    // the two loads do not wait on each other.
    constexpr int CW = (C + 1) / 2; // words of a lane's channels of one row
    uint32_t kh[B][G][CW], vh[B][G][CW];
    uint32_t kh2[B][G][CW], vh2[B][G][CW];
    const bool specTwo = a.spec_keys == 2 * kRound;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const int j = min(split * a.spec_keys + wave + b * kAttnWaves, a.max_positions - 1);
        const int j2 = min(j + kRound, a.max_positions - 1);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            load_words<C>(a.key_cache + (int64_t) j * kvWidth + kvOffset[g], kh[b][g]);
            load_words<C>(a.value_cache + (int64_t) j * kvWidth + kvOffset[g], vh[b][g]);
            if (specTwo) { // uniform: the launch's
                load_words<C>(a.key_cache + (int64_t) j2 * kvWidth + kvOffset[g], kh2[b][g]);
                load_words<C>(a.value_cache + (int64_t) j2 * kvWidth + kvOffset[g], vh2[b][g]);
            }
        }
    }
    // keeps the loads above the position-dependent exit: the compiler would
    // otherwise sink them below it, after the position's own round trip
    asm volatile("" ::: "memory");

    const int keyCount = *a.position + 1;
    const SplitPlan plan = plan_splits(keyCount, a.grid_splits, kRound);
    // a launch too small for its step's keys (the host sizes it to the range:
    // attention_grid_splits) would overrun sScore; it does nothing instead
    if (split >= plan.splits || plan.perSplit > kMaxSplitKeys)
        return;
    const int k0 = split * plan.perSplit;
    const int n = min(plan.perSplit, keyCount - k0);
    const uint16_t *keys = a.key_cache + (int64_t) k0 * kvWidth;
    const uint16_t *values = a.value_cache + (int64_t) k0 * kvWidth;

    // a round's rows for this wave: keys r0 + wave + 8 b, clamped into range
    // (the clamped duplicates are masked where they are used)
    auto load_round = [&](const uint16_t *base, int r0, uint32_t (&dst)[B][G][CW]) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int j = min(r0 + wave + b * kAttnWaves, n - 1);
#pragma unroll
            for (int g = 0; g < G; ++g)
                load_words<C>(base + (int64_t) j * kvWidth + kvOffset[g], dst[b][g]);
        }
    };
    // a two-round split (a window of 4097 .. 8192 keys) has its second round's
    // rows in flight with the first's
    const bool twoRounds = plan.perSplit == 2 * kRound;
    if (plan.perSplit != a.spec_keys) { // not the split expected: its rows again, from k0
        load_round(keys, 0, kh);
        load_round(values, 0, vh);
        if (twoRounds) {
            load_round(keys, kRound, kh2);
            load_round(values, kRound, vh2);
        }
    }

    auto score_round = [&](const uint32_t (&k)[B][G][CW], int r0) {
        double y[kRows];
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                double p = 0.0;
#pragma unroll
                for (int i = 0; i < C; ++i)
                    p += q[g][i] * word_half<C>(k[b][g], i);
                y[b * G + g] = p;
            }
        const double total = reduce_rows<kRows>(y, lane);
        if (stores_row<kRows>(lane)) {
            const int r = row_of_lane<kRows>(lane);
            const int j = r0 + wave + (r / G) * kAttnWaves;
            if (j < n)
                sScore[r % G][j] = (double) a.scale * total;
        }
    };
    score_round(kh, 0);
    if (twoRounds) {
        score_round(kh2, kRound);
    } else {
        for (int r0 = kRound; r0 < n; r0 += kRound) {
            load_round(keys, r0, kh);
            score_round(kh, r0);
        }
    }
    __syncthreads();

    // softmax of the split, one wave a head; the weights replace the scores
    if (wave < G) {
        double largest = -INFINITY;
        for (int j = lane; j < n; j += 64)
            largest = fmax(largest, sScore[wave][j]);
        largest = wave_max_d(largest);
        double sum = 0.0;
        for (int j = lane; j < n; j += 64) {
            const double w = exp(sScore[wave][j] - largest);
            sScore[wave][j] = w;
            sum += w;
        }
        sum = wave_sum_d(sum);
        if (lane == 0) {
            sMax[wave] = largest;
            sSum[wave] = sum;
        }
    }
    __syncthreads();

    double acc[G][C];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < C; ++i)
            acc[g][i] = 0.0;
    auto value_round = [&](const uint32_t (&v)[B][G][CW], int r0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int j = r0 + wave + b * kAttnWaves;
            if (j >= n)
                break;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const double w = sScore[g][j];
#pragma unroll
                for (int i = 0; i < C; ++i)
                    acc[g][i] += w * word_half<C>(v[b][g], i);
            }
        }
    };
    value_round(vh, 0);
    if (twoRounds) {
        value_round(vh2, kRound);
    } else {
        for (int r0 = kRound; r0 < n; r0 += kRound) {
            load_round(values, r0, vh);
            value_round(vh, r0);
        }
    }
    if (active)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < C; ++i)
                sAcc[wave][g * hd + c0 + i] = acc[g][i];
    __syncthreads();

    // the split's partial: the waves' sums in wave order, then (max, sum), as
    // tagged words (two a double) that the merging workgroups poll
    const uint32_t tag = a.tag_epoch[0];
    if (t < groupWidth) {
        double o = 0.0;
        for (int w = 0; w < kAttnWaves; ++w)
            o += sAcc[w][t];
        uint64_t *dst = a.part_ll + ((int64_t) split * qWidth + h0 * hd + t) * 2;
        const uint64_t bits = (uint64_t) __double_as_longlong(o);
        ll_put(dst, (uint32_t) bits, tag);
        ll_put(dst + 1, (uint32_t) (bits >> 32), tag);
    }
    if (t < G) {
        uint64_t *dst = a.ml_ll + ((int64_t) split * heads + h0 + t) * 4;
        const uint64_t m = (uint64_t) __double_as_longlong(sMax[t]);
        const uint64_t sum = (uint64_t) __double_as_longlong(sSum[t]);
        ll_put(dst, (uint32_t) m, tag);
        ll_put(dst + 1, (uint32_t) (m >> 32), tag);
        ll_put(dst + 2, (uint32_t) sum, tag);
        ll_put(dst + 3, (uint32_t) (sum >> 32), tag);
    }

    // The merge (MultiQueryAttention.h:43-49: every split rescaled to the row
    // maximum, in split order, the sums divided by the total): the group's
    // live splits share its 32-channel blocks (split s takes blocks s,
    // s + splits, ...), each polling the words it needs, so no workgroup
    // waits on a ticket or reads the whole group's partials.  A merging
    // workgroup's waves share its blocks: wpb waves a block, each taking a
    // run of consecutive splits in one round of polls; the runs' sums are
    // added in LDS in split order.
    const int splits = plan.splits;
    const int blocks = groupWidth / kBlock;
    const int mine = split < blocks ? (blocks - split + splits - 1) / splits : 0;
    if (mine == 0)
        return;
    const uint32_t mlBytes = (uint32_t) (kDecodeSplits * heads * 4 * 8);
    const uint32_t partBytes = (uint32_t) ((int64_t) kDecodeSplits * qWidth * 16);
    // lanes 32..63 of a merging wave repeat lanes 0..31 (the cross-lane sums
    // below take whole waves); lanes 0..31 store
    const int wpb = kAttnWaves / mine;                // waves a block (mine <= 8 blocks)
    const int bi = wave / wpb, ci = wave % wpb;       // this wave's block and run
    const bool merging = bi < mine;
    const int b = split + bi * splits;                // the block of the group
    const int c = b * kBlock + (lane & (kBlock - 1)); // this lane's channel in the group
    const int run = (splits + wpb - 1) / wpb;
    const int sBegin = min(ci * run, splits), sEnd = min(sBegin + run, splits);
    // waves g < G: the split factors of head h0 + g, lane s taking split s
    if (wave < G) {
        const bool liveSplit = lane < splits;
        const int sp = liveSplit ? lane : 0;
        const uint32_t off = (uint32_t) ((sp * heads + h0 + wave) * 4 * 8);
        double m = -INFINITY, sum = 0.0;
        int spins = 0;
        for (;;) {
            const v4u w0 = ld_agent_16(a.ml_ll, off, mlBytes);
            const v4u w1 = ld_agent_16(a.ml_ll, off + 16, mlBytes);
            if (w0.y == tag && w0.w == tag && w1.y == tag && w1.w == tag) {
                m = __longlong_as_double((long long) (((uint64_t) w0.z << 32) | w0.x));
                sum = __longlong_as_double((long long) (((uint64_t) w1.z << 32) | w1.x));
                break;
            }
            if (wait_give_up(a.error, spins))
                break;
        }
        double total;
        const double f = merge_factor(m, sum, liveSplit, total);
        if (liveSplit)
            sSplitMax[wave][sp] = f; // now the split's factor
        if (lane == 0)
            sSum[wave] = total;
    }
    // the partial sums above have been read out of sAcc: it takes the runs'
    __syncthreads();
    const int g = c / hd;
    double weighted = 0.0;
    if (merging) {
        for (int s0 = sBegin; s0 < sEnd; s0 += kPollSplits) {
            double part[kPollSplits];
            int spins = 0;
            for (;;) {
                v4u w[kPollSplits];
#pragma unroll
                for (int u = 0; u < kPollSplits; ++u) {
                    const int sp = min(s0 + u, sEnd - 1);
                    w[u] = ld_agent_16(a.part_ll, (uint32_t) ((sp * qWidth + h0 * hd + c) * 16), partBytes);
                }
                bool all = true;
#pragma unroll
                for (int u = 0; u < kPollSplits; ++u)
                    all = all && w[u].y == tag && w[u].w == tag;
                if (all) {
#pragma unroll
                    for (int u = 0; u < kPollSplits; ++u)
                        part[u] = __longlong_as_double((long long) (((uint64_t) w[u].z << 32) | w[u].x));
                    break;
                }
                if (wait_give_up(a.error, spins)) {
#pragma unroll
                    for (int u = 0; u < kPollSplits; ++u)
                        part[u] = 0.0;
                    break;
                }
            }
#pragma unroll
            for (int u = 0; u < kPollSplits; ++u)
                if (s0 + u < sEnd)
                    weighted += part[u] * sSplitMax[g][s0 + u];
        }
    }
    double *sRun = &sAcc[0][0]; // [kAttnWaves][kBlock]: each wave's run sums
    if (merging && lane < kBlock)
        sRun[wave * kBlock + lane] = weighted;
    __syncthreads();
    if (!merging || ci != 0)
        return;
    double total = sRun[wave * kBlock + (lane & (kBlock - 1))];
    for (int k = 1; k < wpb; ++k)
        total += sRun[(wave + k) * kBlock + (lane & (kBlock - 1))];
    const int idx = h0 * hd + c;
    const float v = (float) (total / sSum[g]);
    float amax = fabsf(v);
    amax = max_lanes<16>(amax); // lanes 0..31: the block
    const uint16_t bits = scale_bits_from_amax(amax);
    const float sc = half_value(bits);
    const int byte = quantize_in_block(v, bits, sc, quantize_hint(sc));
    if (lane >= kBlock)
        return;
    if (a.out)
        a.out[idx] = v;
    a.q8[idx] = (uint8_t) (int8_t) byte;
    if (lane == 0)
        reinterpret_cast<uint16_t *>(a.q8 + qWidth)[idx / kBlock] = bits;
}

// ---- gate|up + GeGLU + Q8 -----------------------------------------------------------
// A workgroup of eight waves owns one 32-element block of the GeGLU output:
// gate rows [32 b, 32 b + 32) and the matching up rows; a wave owns four of
// them (eight rows, reduced together).
constexpr int kGluThreads = 512;
constexpr int kGluWaves = kGluThreads / 64;
constexpr int kGluPerWave = kBlock / kGluWaves; // 4

// Element t of one activation block (thread t < 32): the GeGLU value and its
// Int8Blocks byte and block scale.
struct ActElement {
    float v;
    int q;
    uint16_t bits;
};

// The body both gate|up launches share: the post-attention norm of the
// residual row and its Q8 in LDS (issued before the weight loads), the gate
// rows [32 b, 32 b + 32) and the matching up rows of block b = blockIdx.x,
// GeGLU and the block's Q8.  Thread t < 32 gets element t.
__device__ __attribute__((always_inline)) inline ActElement
gateup_geglu_block(const float *hidden, const float *normWeight, int width, float epsilon,
                   const uint8_t *weights, int F, RowQ8 &row, double *sPartial, float *sGate,
                   float *sUp)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = width / kBlock;
    const int o0 = blockIdx.x * kBlock + wave * kGluPerWave;
    const bool valid = lane < nb;

    const RowSlice<4> slice = load_row_slice<4>(hidden, nullptr, nullptr, 0, 0.f, nullptr,
                                                normWeight, width);
    // rows 0..3 gate, 4..7 up
    WeightBlock w[2 * kGluPerWave];
#pragma unroll
    for (int k = 0; k < kGluPerWave; ++k) {
        w[k] = load_block(weights, 2 * (int64_t) F, width, o0 + k, lane, valid);
        w[kGluPerWave + k] = load_block(weights, 2 * (int64_t) F, width, (int64_t) F + o0 + k, lane, valid);
    }
    __builtin_amdgcn_sched_barrier(0); // every load issued before the norm's first wait
    norm_q8_finish(slice, width, epsilon, row, sPartial, nullptr, nullptr);
    int4 a0 = make_int4(0, 0, 0, 0), a1 = a0;
    double sa = 0.0;
    if (valid) {
        a0 = reinterpret_cast<const int4 *>(row.q + lane * kBlock)[0];
        a1 = reinterpret_cast<const int4 *>(row.q + lane * kBlock)[1];
        sa = row.scale[lane];
    }
    double y[2 * kGluPerWave];
#pragma unroll
    for (int k = 0; k < 2 * kGluPerWave; ++k)
        y[k] = block_term(w[k], a0, a1, sa);
    const double total = reduce_rows<2 * kGluPerWave>(y, lane);
    if (stores_row<2 * kGluPerWave>(lane)) {
        const int r = row_of_lane<2 * kGluPerWave>(lane);
        const int o = wave * kGluPerWave + (r % kGluPerWave);
        if (r < kGluPerWave)
            sGate[o] = (float) total;
        else
            sUp[o] = (float) total;
    }
    __syncthreads();
    ActElement e{0.f, 0, 0};
    if (threadIdx.x < kBlock) {
        e.v = geglu(sGate[threadIdx.x], sUp[threadIdx.x]);
        float amax = fabsf(e.v);
        amax = max_lanes<16>(amax);
        e.bits = scale_bits_from_amax(amax);
        const float sc = half_value(e.bits);
        e.q = quantize_in_block(e.v, e.bits, sc, quantize_hint(sc));
    }
    return e;
}

__global__ __launch_bounds__(kGluThreads) __attribute__((amdgpu_waves_per_eu(4)))
void gateup_geglu_kernel(GateUpArgs a)
{
    GQ8_ARGS_EARLY("s"(a.q8), "s"(a.debug_activated));
    __shared__ RowQ8 row;
    __shared__ double sPartial[kGluWaves];
    __shared__ float sGate[kBlock], sUp[kBlock];
    const ActElement e = gateup_geglu_block(a.hidden, a.norm_weight, a.width, a.epsilon, a.weights,
                                            a.intermediate, row, sPartial, sGate, sUp);
    if (threadIdx.x < kBlock) {
        const int o = blockIdx.x * kBlock + threadIdx.x;
        if (a.debug_activated)
            a.debug_activated[o] = e.v;
        a.q8[o] = (uint8_t) (int8_t) e.q;
        if (threadIdx.x == 0)
            reinterpret_cast<uint16_t *>(a.q8 + a.intermediate)[blockIdx.x] = e.bits;
    }
}

// ---- final norm + tied lm_head + argmax ----------------------------------------------
// The final norm and its Q8 row come from a one-workgroup kernel; the lm_head
// is then a one-shot product (every wave loads its eight rows' blocks once,
// the activation block of its lane straight from the Q8 row) whose rows are
// reduced together.  Each workgroup folds its rows into one 64-bit candidate
// (an order-preserving key of the logit above the complemented row index) and
// merges it into one of kHeadSlots device words (spread over cache lines, so
// that the atomics do not queue on one address) with one atomicMax, so the
// largest logit wins and, among equal logits, the lowest index -- the first
// maximum.  No workgroup waits for another; a one-wave kernel then folds the
// slots, turns the winner into the token id, stores it in the sequence slot
// after the position, advances the position and clears the slots.
constexpr int kHeadRows = 8;
// eight waves a workgroup (4 000 workgroups over the 256 000 rows): a plain
// read of the tied embedding in this pattern streams at 6.3-6.4 TB/s, against
// 6.0-6.1 TB/s for 8 000 four-wave workgroups
constexpr int kHeadThreads = 512;
constexpr int kHeadWaves = kHeadThreads / 64;


__global__ __launch_bounds__(kHeadThreads) void lmhead_argmax_kernel(HeadArgs a)
{
    GQ8_ARGS_EARLY("s"(a.best), "s"(a.logits));
    __shared__ unsigned long long sBest[kHeadWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = a.width / kBlock;
    const bool valid = lane < nb;
    const int64_t V = a.vocab;
    const int64_t r0 = ((int64_t) blockIdx.x * kHeadWaves + wave) * kHeadRows;

    WeightBlock w[kHeadRows];
#pragma unroll
    for (int k = 0; k < kHeadRows; ++k)
        w[k] = load_block(a.weights, V, a.width, r0 + k, lane, valid && r0 + k < V);
    const int ab = valid ? lane : 0; // an invalid lane's terms are zeroed by block_term
    const int4 a0 = reinterpret_cast<const int4 *>(a.q8 + ab * kBlock)[0];
    const int4 a1 = reinterpret_cast<const int4 *>(a.q8 + ab * kBlock)[1];
    const double sa = (double) half_value(reinterpret_cast<const uint16_t *>(a.q8 + a.width)[ab]);
    __builtin_amdgcn_sched_barrier(0); // every load issued before the first wait
    double y[kHeadRows];
#pragma unroll
    for (int k = 0; k < kHeadRows; ++k)
        y[k] = block_term(w[k], a0, a1, sa);
    const double total = reduce_rows<kHeadRows>(y, lane);
    const int64_t row = r0 + row_of_lane<kHeadRows>(lane);
    unsigned long long best = 0;
    if (stores_row<kHeadRows>(lane) && row < V) {
        const float logit = (float) total;
        a.logits[row] = logit;
        best = candidate_key(logit, (uint32_t) row);
    }
    best = fold_wave_max(best);
    if (lane == 0)
        sBest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long c = sBest[0];
        for (int k = 1; k < kHeadWaves; ++k)
            c = sBest[k] > c ? sBest[k] : c;
        if (c != 0)
            atomicMax(a.best + (blockIdx.x % kHeadSlots) * kHeadSlotStride, c);
    }
}

// One wave folds the slots, stores the id and clears the slots.
__global__ __launch_bounds__(64) void head_finalize_kernel(HeadArgs a)
{
    const int lane = threadIdx.x;
    unsigned long long *slot = a.best + lane * kHeadSlotStride;
    const unsigned long long c = fold_wave_max(lane < kHeadSlots ? *slot : 0ull);
    if (lane < kHeadSlots)
        *slot = 0;
    if (lane == 0) {
        const uint32_t token = c == 0 ? 0u : 0xFFFFFFFFu - (uint32_t) (c & 0xFFFFFFFFull);
        const int position = *a.position;
        if (a.sequence)
            a.sequence[position + 1] = token;
        if (a.advance)
            *a.position = position + 1;
    }
}

// ============================================================================
// The dataflow decode step (one launch a token)
// ============================================================================
// Item order = dependency order: per layer the q|k|v items, the attention
// (split, head group) items, the o, gate|up and down items; then the final
// norm, the lm_head items and the finalize item.  Workgroups start in id order
// on each XCD, so an item only ever waits on items that started before it:
// the earliest unfinished item has nothing left to wait for, and every wait
// ends.  A wait is a bounded spin; giving up sets the error word, which every
// other wait checks, so a failure ends the launch instead of hanging it.
//
// Items hand rows on in tagged words: one 64-bit store of a 32-bit value and
// a 32-bit tag (the launch's epoch and the row's version), single-copy atomic.
// A reader polls the words it needs until each carries the tag it expects, so
// a hand-over is one trip through the memory system; a counter and a flag
// would take four (the data, the count, the flag, the data again).  Readers
// of a whole row first poll the word its last producer writes, then read the
// row once.  Every version of a row is read only by items that the writer of
// its next version depends on, so no version is overwritten while it is read.
// Tagged words are written and read with agent-scope (sc1) accesses, which
// the eight XCD L2s keep coherent.
//
// Weights and the K/V rows of earlier steps were written before the launch:
// plain cached loads, issued before the wait.  The lm_head items and the idle
// attention splits count themselves on trees of counters (sub-counters of 16
// arrivals, then a top count, then 16 flags that waiters spread their polls
// over), which the finalize item waits on.
constexpr int kFlowWaves = kFlowThreads / 64;
constexpr int kFlowPairsPerWave = 2;
constexpr int kFlowQkvPairs = kFlowWaves * kFlowPairsPerWave;   // 16 pairs (32 rows) an item
constexpr int kFlowORows = kFlowWaves * 2;                  // 16 rows an item
constexpr int kFlowDownRows = kFlowWaves;                   // 8 rows an item
constexpr int kFlowDownBlocks = 8;                          // blocks a lane (inner <= 16384)
constexpr int kFlowHeadRows = kFlowWaves * kHeadRows;       // 64 rows an item
constexpr int kFlowMaxInner = 64 * kBlock * kFlowDownBlocks;  // 16384
constexpr int kFlowActWords = kFlowMaxInner / 4 + kFlowMaxInner / kBlock + 4; // a staged Q8 row
constexpr int kFlowMergePieces = 8;    // partials a merging lane loads at once
constexpr int kFlowStagePieces = (kFlowActWords / 2 + kFlowThreads - 1) / kFlowThreads; // 5
constexpr int kFlowRowPieces = ((kFusedMaxWidth / 4 + kFusedMaxWidth / kBlock) / 2 + kFlowThreads - 1)
                               / kFlowThreads; // a Q8 row of at most the fused width: 1

enum { kCounterHead = 0, kCounterIdle = 1 };

// N consecutive pieces (2 N words) from even word `word` of a `words`-long
// row: every load issued first, then the words not yet tagged polled again.
template <int N>
__device__ inline bool ll_get_pieces(const uint64_t *row, int word, int words, uint32_t tag, const int *error,
                                     uint32_t (&v)[2 * N])
{
    v4u w[N];
#pragma unroll
    for (int k = 0; k < N; ++k)
        w[k] = ld_agent_16(row, (uint32_t) (word + 2 * k) * 8, (uint32_t) words * 8);
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        v[2 * k] = w[k].x;
        v[2 * k + 1] = w[k].z;
        if (w[k].y != tag || (word + 2 * k + 1 < words && w[k].w != tag))
            ok = ll_get2(row, word + 2 * k, words, tag, error, v[2 * k], v[2 * k + 1]) && ok;
    }
    return ok;
}

// The values of a `words`-long tagged row (at most 2 P words a thread) into
// LDS; thread 0 first waits for word `sentinel` (the one its last producer
// writes).  False for every thread after a wait gave up.
template <int P>
__device__ inline bool flow_stage_ll(const FlowArgs &a, const uint64_t *row, int words, int sentinel,
                                     uint32_t tag, uint32_t *sDst)
{
    bool ok = true;
    if (threadIdx.x == 0) {
        uint32_t v;
        ok = ll_get(row + sentinel, tag, a.error, v);
    }
    if (__syncthreads_or(!ok))
        return false;
    const int pieces = (words + 1) / 2;
    v4u w[P];
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const int p = threadIdx.x + k * kFlowThreads;
        if (p < pieces)
            w[k] = ld_agent_16(row, (uint32_t) p * 16, (uint32_t) words * 8);
    }
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const int p = threadIdx.x + k * kFlowThreads;
        if (p < pieces) {
            uint32_t v0 = w[k].x, v1 = w[k].z;
            if (w[k].y != tag || (2 * p + 1 < words && w[k].w != tag))
                ok = ll_get2(row, 2 * p, words, tag, a.error, v0, v1) && ok;
            sDst[2 * p] = v0;
            sDst[2 * p + 1] = v1;
        }
    }
    return !__syncthreads_or(!ok);
}

// The Q8 byte of each of four consecutive lanes packed into the first lane's
// word; lanes 32 k also put the block's scale word (the row's word layout:
// inner / 4 words of bytes, then one scale word a block).
__device__ inline void flow_put_q8(uint64_t *row, int inner, int idx, uint8_t byte, uint16_t bits, bool live,
                                   uint32_t tag)
{
    const uint32_t b = byte;
    const uint32_t w = b | ((uint32_t) __shfl_down((int) b, 1) << 8)
                       | ((uint32_t) __shfl_down((int) b, 2) << 16)
                       | ((uint32_t) __shfl_down((int) b, 3) << 24);
    if (live && (idx & 3) == 0)
        ll_put(row + idx / 4, w, tag);
    if (live && (idx & 31) == 0)
        ll_put(row + inner / 4 + idx / kBlock, bits, tag);
}

// The activation block `block` of a Q8 row staged in LDS.
__device__ inline void lds_act_block(const uint32_t *sAct, int inner, int block, int4 &a0, int4 &a1,
                                     double &sa)
{
    const int4 *w = reinterpret_cast<const int4 *>(sAct + block * (kBlock / 4));
    a0 = w[0];
    a1 = w[1];
    sa = (double) half_value((uint16_t) sAct[inner / 4 + block]);
}

// ---- counter trees (lm_head items, idle attention splits) --------------------
__device__ inline int *flow_line(const FlowArgs &a, int counter, int line)
{
    return a.counters + ((int64_t) counter * kFlowCounterLines + line) * kFlowLineInts;
}

// Waits until counter `counter` has completed; false after giving up.
__device__ __forceinline__ bool flow_wait(const FlowArgs &a, int counter)
{
    bool ok = true;
    if (threadIdx.x == 0) {
        int spins = 0;
        const int *flag = flow_line(a, counter, 1 + (int) (blockIdx.x % kFlowFlagLines));
        while (ld_agent_i(flag) == 0)
            if (wait_give_up(a.error, spins)) {
                ok = false;
                break;
            }
    }
    return !__syncthreads_or(!ok);
}

// One arrival on sub-counter `sub` (complete at `inSub` arrivals) of a counter
// complete when `subs` sub-counters are; the arrival that completes it raises
// the flags.  Completed lines go back to zero for the next launch.
__device__ inline void flow_arrive(const FlowArgs &a, int counter, int sub, int inSub, int subs)
{
    int *subLine = flow_line(a, counter, 1 + kFlowFlagLines + sub);
    if (__hip_atomic_fetch_add(subLine, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != inSub - 1)
        return;
    st_agent_i(subLine, 0);
    int *top = flow_line(a, counter, 0);
    if (__hip_atomic_fetch_add(top, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != subs - 1)
        return;
    st_agent_i(top, 0);
    for (int k = 0; k < kFlowFlagLines; ++k)
        st_agent_i(flow_line(a, counter, 1 + k), 1);
}

// Every thread's stores have completed; then item `index` of `count` arrives.
__device__ __forceinline__ void flow_signal(const FlowArgs &a, int counter, int index, int count)
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const int sub = index / kFlowFanIn;
        flow_arrive(a, counter, sub, min(kFlowFanIn, count - sub * kFlowFanIn),
                    (count + kFlowFanIn - 1) / kFlowFanIn);
    }
}

// ---- rows into the norms -------------------------------------------------------
// Thread t's four elements of the residual row at version `tag`, with their
// norm weights; thread 0 first waits for the last element (its last writer).
__device__ __forceinline__ bool flow_hidden_slice(const FlowArgs &a, const float *weight, uint32_t tag,
                                                  RowSlice<4> &r)
{
    const int t = threadIdx.x;
    r.active = t * 4 < a.width;
    const int i0 = r.active ? t * 4 : 0;
    load4<4>(weight + i0, r.w);
    bool ok = true;
    if (t == 0) {
        uint32_t v;
        ok = ll_get(a.hidden_ll + a.width - 1, tag, a.error, v);
    }
    if (__syncthreads_or(!ok))
        return false;
    uint32_t v[4];
    ok = ll_get_pieces<2>(a.hidden_ll, i0, a.width, tag, a.error, v);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        r.v[k] = __uint_as_float(v[k]);
    return !__syncthreads_or(!ok);
}

// Thread t's four elements of the embedding row of sequence[position] (scaled)
// with their norm weights; with `publish`, also put as the residual row's
// version 0.
__device__ __forceinline__ RowSlice<4> flow_embed_slice(const FlowArgs &a, const float *weight, int position,
                                                        bool publish, uint32_t tag)
{
    RowSlice<4> r;
    const int t = threadIdx.x;
    r.active = t * 4 < a.width;
    const int i0 = r.active ? t * 4 : 0;
    load4<4>(weight + i0, r.w);
    uint32_t id = a.sequence[position];
    if (id >= (uint32_t) a.vocab) // ids are validated on the host; a guard, not a rule
        id = 0;
    const int64_t e0 = (int64_t) id * a.width + i0;
    const int64_t V = a.vocab;
    const uint16_t bits = reinterpret_cast<const uint16_t *>(a.embedding + V * a.width)[e0 / kBlock];
    const float sc = half_value(bits);
    const int packed = *reinterpret_cast<const int *>(a.embedding + e0);
    int8_t b[4];
    __builtin_memcpy(b, &packed, 4);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        r.v[k] = (float) ((double) a.embed_scale * (double) (sc * (float) b[k]));
    if (publish && r.active)
#pragma unroll
        for (int k = 0; k < 4; ++k)
            ll_put(a.hidden_ll + i0 + k, __float_as_uint(r.v[k]), tag);
    return r;
}

// ---- items ----------------------------------------------------------------------
__device__ __forceinline__ void flow_qkv(const FlowArgs &a, int l, int item, uint32_t epoch)
{
    __shared__ RowQ8 row;
    __shared__ double sPartial[kFlowWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hd = a.head_dim, half = hd / 2;
    const int qWidth = a.heads * hd, kvWidth = a.kv_heads * hd;
    const int outputs = qWidth + 2 * kvWidth;
    const int pairs = (a.heads + 2 * a.kv_heads) * half;
    const int nb = a.width / kBlock;
    const int firstPair = (item * kFlowWaves + wave) * kFlowPairsPerWave;
    const uint8_t *weights = a.qkv + a.qkv_stride * l;

    WeightBlock lo[kFlowPairsPerWave], hi[kFlowPairsPerWave];
#pragma unroll
    for (int p = 0; p < kFlowPairsPerWave; ++p) {
        const int pair = firstPair + p;
        const int rowLo = (pair / half) * hd + pair % half;
        const bool valid = pair < pairs && lane < nb;
        lo[p] = load_block(weights, outputs, a.width, rowLo, lane, valid);
        hi[p] = load_block(weights, outputs, a.width, rowLo + half, lane, valid);
    }
    const int position = *a.position;
    __builtin_amdgcn_sched_barrier(0);
    RowSlice<4> slice;
    if (l == 0)
        slice = flow_embed_slice(a, a.input_norm, position, item == 0, word_tag(epoch, 0));
    else if (!flow_hidden_slice(a, a.input_norm + a.norm_stride * l, word_tag(epoch, 2 * l), slice))
        return;
    norm_q8_finish<4>(slice, a.width, a.epsilon, row, sPartial, nullptr, nullptr);

    int4 a0 = make_int4(0, 0, 0, 0), a1 = a0;
    double sa = 0.0;
    if (lane < nb) {
        a0 = reinterpret_cast<const int4 *>(row.q + lane * kBlock)[0];
        a1 = reinterpret_cast<const int4 *>(row.q + lane * kBlock)[1];
        sa = row.scale[lane];
    }
    constexpr int kRows = 2 * kFlowPairsPerWave;
    double y[kRows];
#pragma unroll
    for (int p = 0; p < kFlowPairsPerWave; ++p) {
        y[2 * p] = block_term(lo[p], a0, a1, sa);
        y[2 * p + 1] = block_term(hi[p], a0, a1, sa);
    }
    const double total = reduce_rows<kRows>(y, lane);
    double rowTotal[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
        rowTotal[r] = lane_value(total, lane_of_row<kRows>(r));
    // lane 0: the wave's two pairs are the consecutive elements (i, i + 1) and
    // (i + half, i + half + 1) of one head
    if (lane == 0 && firstPair < pairs) {
        const uint32_t tag = word_tag(epoch, l);
        const int head = firstPair / half, i = firstPair % half;
        const int rLo = head * hd + i;
        const bool second = firstPair + 1 < pairs;
        float fLo[2] = {(float) rowTotal[0], (float) rowTotal[2]};
        float fHi[2] = {(float) rowTotal[1], (float) rowTotal[3]};
        if (rLo < qWidth + kvWidth) { // q and k heads rotate
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int64_t angle = (int64_t) position * half + i + p;
                float outLo, outHi;
                rotate_pair(fLo[p], fHi[p], a.cosines[angle], a.sines[angle], &outLo, &outHi);
                fLo[p] = outLo;
                fHi[p] = outHi;
            }
        }
        if (rLo < qWidth) {
            ll_put(a.q_ll + rLo, __float_as_uint(fLo[0]), tag);
            ll_put(a.q_ll + rLo + half, __float_as_uint(fHi[0]), tag);
            if (second) {
                ll_put(a.q_ll + rLo + 1, __float_as_uint(fLo[1]), tag);
                ll_put(a.q_ll + rLo + half + 1, __float_as_uint(fHi[1]), tag);
            }
        } else {
            // the fp16 row into the cache (for later steps) and, tagged, for
            // this step's attention: one word a pair of halves
            const bool isKey = rLo < qWidth + kvWidth;
            uint16_t *cache = (isKey ? a.key_cache : a.value_cache)
                              + ((int64_t) l * a.max_positions + position) * kvWidth;
            uint64_t *fresh = isKey ? a.k_ll : a.v_ll;
            const int c = rLo - qWidth - (isKey ? 0 : kvWidth);
            const uint32_t wordLo = (uint32_t) half_bits(fLo[0]) | ((uint32_t) half_bits(fLo[1]) << 16);
            const uint32_t wordHi = (uint32_t) half_bits(fHi[0]) | ((uint32_t) half_bits(fHi[1]) << 16);
            *reinterpret_cast<uint32_t *>(cache + c) = wordLo;
            *reinterpret_cast<uint32_t *>(cache + c + half) = wordHi;
            ll_put(fresh + c / 2, wordLo, tag);
            ll_put(fresh + (c + half) / 2, wordHi, tag);
        }
    }
}

// Attention plan of the flow kernel: whole 64-key rounds a split, at most
// `maxSplits` splits.
__device__ inline SplitPlan flow_plan(int keyCount, int maxSplits)
{
    const int roundsPerSplit = (keyCount + kRoundKeys * maxSplits - 1) / (kRoundKeys * maxSplits);
    const int perSplit = roundsPerSplit * kRoundKeys;
    return {(keyCount + perSplit - 1) / perSplit, perSplit};
}

// Halves c .. c + C of this step's K or V row (tagged words of two halves).
template <int C>
__device__ inline bool ll_halves(const FlowArgs &a, const uint64_t *fresh, int c, uint32_t tag, uint16_t (&h)[C])
{
    if constexpr (C == 4) { // c is a multiple of 4: one piece
        uint32_t w[2];
        const bool ok = ll_get_pieces<1>(fresh, c / 2, a.kv_heads * a.head_dim / 2, tag, a.error, w);
        h[0] = (uint16_t) (w[0] & 0xFFFFu); h[1] = (uint16_t) (w[0] >> 16);
        h[2] = (uint16_t) (w[1] & 0xFFFFu); h[3] = (uint16_t) (w[1] >> 16);
        return ok;
    } else if constexpr (C == 2) {
        uint32_t w0 = 0;
        const bool ok = ll_get(fresh + c / 2, tag, a.error, w0);
        h[0] = (uint16_t) (w0 & 0xFFFFu); h[1] = (uint16_t) (w0 >> 16);
        return ok;
    } else {
        uint32_t w0 = 0;
        const bool ok = ll_get(fresh + c / 2, tag, a.error, w0);
        h[0] = (uint16_t) ((c & 1) ? w0 >> 16 : w0 & 0xFFFFu);
        return ok;
    }
}

// A double as two tagged words (low word first).
__device__ inline void ll_put_double(uint64_t *p, double v, uint32_t tag)
{
    const uint64_t bits = (uint64_t) __double_as_longlong(v);
    ll_put(p, (uint32_t) bits, tag);
    ll_put(p + 1, (uint32_t) (bits >> 32), tag);
}

template <int C, int G>
__device__ __forceinline__ void flow_attention(const FlowArgs &a, int l, int item, uint32_t epoch)
{
    constexpr int kRows = kScoreBatch * G;
    __shared__ double sScore[G][kMaxSplitKeys];
    __shared__ double sAcc[kAttnWaves][kMaxGroupWidth];
    __shared__ double sMax[G], sSum[G];
    __shared__ double sSplitMax[G][kDecodeSplits];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hd = a.head_dim, kvWidth = a.kv_heads * hd;
    const int heads = a.heads, qWidth = heads * hd;
    const int perKv = heads / a.kv_heads;
    const int group = item / a.attn_splits, split = item % a.attn_splits;
    const int h0 = group * G;
    const int groupWidth = G * hd;

    const int keyCount = *a.position + 1;
    const SplitPlan plan = flow_plan(keyCount, a.attn_splits);
    const int groups = a.attn_items / a.attn_splits;
    if (split >= plan.splits) {
        // no work at this length; counted so that the finalize item (which
        // advances the position) knows every item has read the position
        if (t == 0)
            flow_arrive(a, kCounterIdle, l * groups + group, a.attn_splits - plan.splits, a.layers * groups);
        return;
    }
    const uint32_t tag = word_tag(epoch, l);

    const bool active = lane * C < hd;
    const int c0 = active ? lane * C : 0;
    const uint32_t keep = active ? 0xFFFFFFFFu : 0u;
    const int k0 = split * plan.perSplit;
    const int n = min(plan.perSplit, keyCount - k0);
    const int newest = keyCount - 1 - k0; // this step's own row (not in this split when >= n)
    const int64_t layerBase = (int64_t) l * a.max_positions * kvWidth;
    const uint16_t *keys = a.key_cache + layerBase + (int64_t) k0 * kvWidth;
    const uint16_t *values = a.value_cache + layerBase + (int64_t) k0 * kvWidth;
    int kvOffset[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
        kvOffset[g] = ((h0 + g) / perKv) * hd + c0;

    // rows of earlier steps: plain loads, before the wait; this step's row (a
    // wave-uniform case): its tagged words once the q|k|v items have put them
    bool ok = true;
    uint16_t kh[kScoreBatch][G][C], vh[kScoreBatch][G][C];
    auto load_round = [&](bool isKeys, int r0, uint16_t (&dst)[kScoreBatch][G][C], bool waited) {
        const uint16_t *base = isKeys ? keys : values;
#pragma unroll
        for (int b = 0; b < kScoreBatch; ++b) {
            const int j = min(r0 + wave + b * kAttnWaves, n - 1);
            if (j != newest) {
#pragma unroll
                for (int g = 0; g < G; ++g)
                    load_halves<C>(base + (int64_t) j * kvWidth + kvOffset[g], dst[b][g]);
            } else if (waited) {
#pragma unroll
                for (int g = 0; g < G; ++g)
                    ok = ll_halves<C>(a, isKeys ? a.k_ll : a.v_ll, kvOffset[g], tag, dst[b][g]) && ok;
            }
        }
    };
    load_round(true, 0, kh, false);
    load_round(false, 0, vh, false);
    __builtin_amdgcn_sched_barrier(0);
    double q[G][C];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        uint32_t bits[C > 1 ? C : 2] = {};
        if constexpr (C > 1) // c0 even: C / 2 pieces
            ok = ll_get_pieces<C / 2>(a.q_ll, (h0 + g) * hd + c0, qWidth, tag, a.error, bits) && ok;
        else
            ok = ll_get(a.q_ll + (h0 + g) * hd + c0, tag, a.error, bits[0]) && ok;
#pragma unroll
        for (int i = 0; i < C; ++i)
            q[g][i] = (double) __uint_as_float(bits[i] & keep);
    }
#pragma unroll
    for (int b = 0; b < kScoreBatch; ++b) {
        const int j = min(wave + b * kAttnWaves, n - 1);
        if (j == newest) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                ok = ll_halves<C>(a, a.k_ll, kvOffset[g], tag, kh[b][g]) && ok;
                ok = ll_halves<C>(a, a.v_ll, kvOffset[g], tag, vh[b][g]) && ok;
            }
        }
    }

    for (int r0 = 0; r0 < n; r0 += kRoundKeys) {
        if (r0 > 0)
            load_round(true, r0, kh, true);
        double y[kRows];
#pragma unroll
        for (int b = 0; b < kScoreBatch; ++b)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                double p = 0.0;
#pragma unroll
                for (int i = 0; i < C; ++i)
                    p += q[g][i] * (double) half_value(kh[b][g][i]);
                y[b * G + g] = p;
            }
        const double total = reduce_rows<kRows>(y, lane);
        if (stores_row<kRows>(lane)) {
            const int r = row_of_lane<kRows>(lane);
            const int j = r0 + wave + (r / G) * kAttnWaves;
            if (j < n)
                sScore[r % G][j] = (double) a.attn_scale * total;
        }
    }
    __syncthreads();
    if (wave < G) {
        double largest = -INFINITY;
        for (int j = lane; j < n; j += 64)
            largest = fmax(largest, sScore[wave][j]);
        largest = wave_max_d(largest);
        double sum = 0.0;
        for (int j = lane; j < n; j += 64) {
            const double w = exp(sScore[wave][j] - largest);
            sScore[wave][j] = w;
            sum += w;
        }
        sum = wave_sum_d(sum);
        if (lane == 0) {
            sMax[wave] = largest;
            sSum[wave] = sum;
        }
    }
    __syncthreads();
    double acc[G][C];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < C; ++i)
            acc[g][i] = 0.0;
    for (int r0 = 0; r0 < n; r0 += kRoundKeys) {
        if (r0 > 0)
            load_round(false, r0, vh, true);
#pragma unroll
        for (int b = 0; b < kScoreBatch; ++b) {
            const int j = r0 + wave + b * kAttnWaves;
            if (j >= n)
                break;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const double w = sScore[g][j];
#pragma unroll
                for (int i = 0; i < C; ++i)
                    acc[g][i] += w * (double) half_value(vh[b][g][i]);
            }
        }
    }
    if (active)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < C; ++i)
                sAcc[wave][g * hd + c0 + i] = acc[g][i];
    if (__syncthreads_or(!ok))
        return;
    double own = 0.0;
    if (t < groupWidth)
        for (int w = 0; w < kAttnWaves; ++w)
            own += sAcc[w][t];

    // every split but the last puts its partial (unnormalised output, max,
    // sum); the last split, which holds this step's row, merges them
    uint64_t *partO = a.part_ll + (int64_t) split * qWidth * 2;
    uint64_t *partMl = a.part_ml_ll + (int64_t) split * heads * 4;
    const int splits = plan.splits;
    if (split != splits - 1) {
        if (t < groupWidth)
            ll_put_double(partO + (h0 * hd + t) * 2, own, tag);
        if (t < G) {
            ll_put_double(partMl + (h0 + t) * 4, sMax[t], tag);
            ll_put_double(partMl + (h0 + t) * 4 + 2, sSum[t], tag);
        }
        return;
    }

    if (wave < G) { // wave g takes head h0 + g, one split a lane
        const bool liveSplit = lane < splits;
        double m = sMax[wave], sum = sSum[wave];
        if (liveSplit && lane != split) {
            const int ml = (lane * heads + h0 + wave) * 4, mlWords = kDecodeSplits * heads * 4;
            uint32_t w[4];
            ok = ll_get_pieces<2>(a.part_ml_ll, ml, mlWords, tag, a.error, w);
            m = __longlong_as_double((long long) (((uint64_t) w[1] << 32) | w[0]));
            sum = __longlong_as_double((long long) (((uint64_t) w[3] << 32) | w[2]));
        }
        double total;
        const double f = merge_factor(m, sum, liveSplit, total);
        if (liveSplit)
            sSplitMax[wave][lane] = f;
        if (lane == 0)
            sSum[wave] = total;
    }
    if (__syncthreads_or(!ok))
        return;
    const bool live = t < groupWidth;
    const int g = min(t / hd, G - 1);
    double weighted = 0.0;
    const int tt = live ? t : 0;
    const uint32_t partBytes = (uint32_t) kDecodeSplits * qWidth * 16;
    for (int s0 = 0; s0 < splits; s0 += kFlowMergePieces) {
        v4u part[kFlowMergePieces]; // every lane loads (clamped), so the loads issue together
#pragma unroll
        for (int u = 0; u < kFlowMergePieces; ++u) {
            const int sp = min(s0 + u, splits - 1);
            part[u] = ld_agent_16(a.part_ll, (uint32_t) (sp * qWidth + h0 * hd + tt) * 16, partBytes);
        }
#pragma unroll
        for (int u = 0; u < kFlowMergePieces; ++u)
            if (s0 + u < splits) {
                double v = own;
                if (s0 + u != split) {
                    uint32_t lo = part[u].x, hi = part[u].z;
                    if (part[u].y != tag || part[u].w != tag)
                        ok = ll_get2(a.part_ll, ((s0 + u) * qWidth + h0 * hd + tt) * 2, kDecodeSplits * qWidth * 2,
                                     tag, a.error, lo, hi) && ok;
                    v = __longlong_as_double((long long) (((uint64_t) hi << 32) | lo));
                }
                weighted += (live ? v : 0.0) * sSplitMax[g][s0 + u];
            }
    }
    if (__syncthreads_or(!ok))
        return;
    const int idx = h0 * hd + t;
    const float v = live ? (float) (weighted / sSum[g]) : 0.f;
    float amax = fabsf(v);
    amax = max_lanes<16>(amax);
    const uint16_t bits = scale_bits_from_amax(amax);
    const float sc = half_value(bits);
    const uint8_t byte = (uint8_t) (int8_t) quantize_in_block(v, bits, sc, quantize_hint(sc));
    flow_put_q8(a.attn_ll, qWidth, idx, byte, bits, live, tag);
}

__device__ __forceinline__ void flow_o(const FlowArgs &a, int l, int item, uint32_t epoch, uint32_t *sAct)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int W = a.width, qWidth = a.heads * a.head_dim, nb = qWidth / kBlock;
    const int r0 = item * kFlowORows + wave * 2;
    const bool valid = lane < nb;
    WeightBlock w[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
        w[k] = load_block(a.out + a.out_stride * l, W, qWidth, r0 + k, lane, valid && r0 + k < W);
    __builtin_amdgcn_sched_barrier(0);
    const int words = qWidth / 4 + qWidth / kBlock;
    if (!flow_stage_ll<kFlowRowPieces>(a, a.attn_ll, words, words - 1, word_tag(epoch, l), sAct))
        return;
    int4 a0, a1;
    double sa;
    lds_act_block(sAct, qWidth, valid ? lane : 0, a0, a1, sa);
    double y[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
        y[k] = block_term(w[k], a0, a1, sa);
    const double total = reduce_rows<2>(y, lane);
    const int row = r0 + row_of_lane<2>(lane);
    if (stores_row<2>(lane) && row < W) {
        uint32_t old;
        if (ll_get(a.hidden_ll + row, word_tag(epoch, 2 * l), a.error, old))
            ll_put(a.hidden_ll + row, __float_as_uint((float) (total + (double) __uint_as_float(old))),
                   word_tag(epoch, 2 * l + 1));
    }
}

__device__ __forceinline__ void flow_gateup(const FlowArgs &a, int l, int item, uint32_t epoch)
{
    __shared__ RowQ8 row;
    __shared__ double sPartial[kFlowWaves];
    __shared__ float sGate[kBlock], sUp[kBlock];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = a.width / kBlock;
    const int F = a.intermediate;
    const int o0 = item * kBlock + wave * kGluPerWave;
    const bool valid = lane < nb;
    const uint8_t *weights = a.gate_up + a.gate_up_stride * l;
    WeightBlock w[2 * kGluPerWave];
#pragma unroll
    for (int k = 0; k < kGluPerWave; ++k) {
        w[k] = load_block(weights, 2 * (int64_t) F, a.width, o0 + k, lane, valid);
        w[kGluPerWave + k] = load_block(weights, 2 * (int64_t) F, a.width, (int64_t) F + o0 + k,
                                        lane, valid);
    }
    __builtin_amdgcn_sched_barrier(0);
    RowSlice<4> slice;
    if (!flow_hidden_slice(a, a.post_norm + a.norm_stride * l, word_tag(epoch, 2 * l + 1), slice))
        return;
    norm_q8_finish<4>(slice, a.width, a.epsilon, row, sPartial, nullptr, nullptr);
    int4 a0 = make_int4(0, 0, 0, 0), a1 = a0;
    double sa = 0.0;
    if (valid) {
        a0 = reinterpret_cast<const int4 *>(row.q + lane * kBlock)[0];
        a1 = reinterpret_cast<const int4 *>(row.q + lane * kBlock)[1];
        sa = row.scale[lane];
    }
    double y[2 * kGluPerWave];
#pragma unroll
    for (int k = 0; k < 2 * kGluPerWave; ++k)
        y[k] = block_term(w[k], a0, a1, sa);
    const double total = reduce_rows<2 * kGluPerWave>(y, lane);
    if (stores_row<2 * kGluPerWave>(lane)) {
        const int r = row_of_lane<2 * kGluPerWave>(lane);
        const int o = wave * kGluPerWave + (r % kGluPerWave);
        if (r < kGluPerWave)
            sGate[o] = (float) total;
        else
            sUp[o] = (float) total;
    }
    __syncthreads();
    if (threadIdx.x < 64) { // the first wave: lanes 0..31 hold the block's 32 outputs
        const bool live = threadIdx.x < kBlock;
        const int o = item * kBlock + (live ? threadIdx.x : 0);
        const float v = live ? geglu(sGate[threadIdx.x & 31], sUp[threadIdx.x & 31]) : 0.f;
        float amax = fabsf(v);
        amax = max_lanes<16>(amax);
        const uint16_t bits = scale_bits_from_amax(amax);
        const float sc = half_value(bits);
        const uint8_t byte = (uint8_t) (int8_t) quantize_in_block(v, bits, sc, quantize_hint(sc));
        flow_put_q8(a.act_ll, F, o, byte, bits, live, word_tag(epoch, l));
    }
}

__device__ __forceinline__ void flow_down(const FlowArgs &a, int l, int item, uint32_t epoch, uint32_t *sAct)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int W = a.width, F = a.intermediate, nb = F / kBlock;
    const int row = item * kFlowDownRows + wave;
    WeightBlock w[kFlowDownBlocks];
#pragma unroll
    for (int j = 0; j < kFlowDownBlocks; ++j) {
        const int b = lane + 64 * j;
        w[j] = load_block(a.down + a.down_stride * l, W, F, row, b, row < W && b < nb);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int words = F / 4 + F / kBlock;
    if (!flow_stage_ll<kFlowStagePieces>(a, a.act_ll, words, words - 1, word_tag(epoch, l), sAct))
        return;
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < kFlowDownBlocks; ++j) {
        const int b = lane + 64 * j;
        int4 a0, a1;
        double sa;
        lds_act_block(sAct, F, b < nb ? b : 0, a0, a1, sa);
        acc += block_term(w[j], a0, a1, sa);
    }
    const double total = wave_sum_d(acc);
    if (lane == 0 && row < W) {
        uint32_t old;
        if (ll_get(a.hidden_ll + row, word_tag(epoch, 2 * l + 1), a.error, old))
            ll_put(a.hidden_ll + row, __float_as_uint((float) (total + (double) __uint_as_float(old))),
                   word_tag(epoch, 2 * l + 2));
    }
}

__device__ __forceinline__ void flow_final_norm(const FlowArgs &a, uint32_t epoch)
{
    __shared__ RowQ8 row;
    __shared__ double sPartial[kFlowWaves];
    RowSlice<4> slice;
    if (!flow_hidden_slice(a, a.final_norm, word_tag(epoch, 2 * a.layers), slice))
        return;
    norm_q8_finish<4>(slice, a.width, a.epsilon, row, sPartial, nullptr, nullptr);
    const int t = threadIdx.x;
    const uint32_t tag = word_tag(epoch, 0);
    if (t * 4 < a.width) {
        uint32_t word;
        __builtin_memcpy(&word, row.q + t * 4, 4);
        ll_put(a.head_ll + t, word, tag);
    }
    if (t < a.width / kBlock)
        ll_put(a.head_ll + a.width / 4 + t, half_bits((float) row.scale[t]), tag);
}

__device__ __forceinline__ void flow_lmhead(const FlowArgs &a, int item, uint32_t epoch, uint32_t *sAct)
{
    __shared__ unsigned long long sBest[kFlowWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = a.width / kBlock;
    const bool valid = lane < nb;
    const int64_t V = a.vocab;
    const int64_t r0 = ((int64_t) item * kFlowWaves + wave) * kHeadRows;
    WeightBlock w[kHeadRows];
#pragma unroll
    for (int k = 0; k < kHeadRows; ++k)
        w[k] = load_block(a.embedding, V, a.width, r0 + k, lane, valid && r0 + k < V);
    __builtin_amdgcn_sched_barrier(0);
    const int words = a.width / 4 + a.width / kBlock;
    if (!flow_stage_ll<kFlowRowPieces>(a, a.head_ll, words, words - 1, word_tag(epoch, 0), sAct))
        return;
    int4 a0, a1;
    double sa;
    lds_act_block(sAct, a.width, valid ? lane : 0, a0, a1, sa);
    double y[kHeadRows];
#pragma unroll
    for (int k = 0; k < kHeadRows; ++k)
        y[k] = block_term(w[k], a0, a1, sa);
    const double total = reduce_rows<kHeadRows>(y, lane);
    const int64_t rowIndex = r0 + row_of_lane<kHeadRows>(lane);
    unsigned long long best = 0;
    if (stores_row<kHeadRows>(lane) && rowIndex < V) {
        const float logit = (float) total;
        a.logits[rowIndex] = logit;
        best = candidate_key(logit, (uint32_t) rowIndex);
    }
    best = fold_wave_max(best);
    if (lane == 0)
        sBest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long c = sBest[0];
        for (int k = 1; k < kFlowWaves; ++k)
            c = sBest[k] > c ? sBest[k] : c;
        if (c != 0)
            atomicMax(a.best + (item % kHeadSlots) * kHeadSlotStride, c);
    }
    flow_signal(a, kCounterHead, item, a.head_items);
}

__device__ __forceinline__ void flow_finalize(const FlowArgs &a, uint32_t epoch)
{
    // every other item has read the position and the epoch: the lm_head items
    // (whose inputs chain back through every working item) and the idle
    // attention splits
    const int position = *a.position;
    const int idle = a.attn_splits - flow_plan(position + 1, a.attn_splits).splits;
    if (!flow_wait(a, kCounterHead) || (idle > 0 && !flow_wait(a, kCounterIdle)))
        return;
    const int t = threadIdx.x;
    if (t < 64) {
        unsigned long long *slot = a.best + t * kHeadSlotStride;
        const unsigned long long c =
            fold_wave_max(t < kHeadSlots ? (unsigned long long) ld_agent_u64(reinterpret_cast<uint64_t *>(slot)) : 0ull);
        if (t < kHeadSlots)
            __hip_atomic_store(reinterpret_cast<uint64_t *>(slot), (uint64_t) 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (t == 0) {
            const uint32_t token = c == 0 ? 0u : 0xFFFFFFFFu - (uint32_t) (c & 0xFFFFFFFFull);
            if (a.sample)
                a.sequence[position + 1] = token;
            *a.position = position + 1;
            // the next launch's tags (24 bits of epoch; zero is never used, so
            // words cleared to zero never match)
            const uint32_t next = (epoch + 1) & 0xFFFFFFu;
            *a.epoch = next == 0 ? 1u : next;
        }
    }
    // every waiter has passed its wait: the flags start the next step lowered
    // (completed sub-counters and tops went back to zero as they completed)
    if (t < kFlowCounters * kFlowFlagLines)
        st_agent_i(flow_line(a, t / kFlowFlagLines, 1 + t % kFlowFlagLines), 0);
}

template <int C, int G>
__global__ __launch_bounds__(kFlowThreads) __attribute__((amdgpu_waves_per_eu(4)))
void flow_step_kernel(FlowArgs a)
{
    __shared__ __attribute__((aligned(16))) uint32_t sAct[kFlowActWords];
    const uint32_t epoch = *a.epoch;
    const int perLayer = a.qkv_items + a.attn_items + a.o_items + a.gate_up_items + a.down_items;
    int item = blockIdx.x;
    if (item < a.layers * perLayer) {
        const int l = item / perLayer;
        item -= l * perLayer;
        if (item < a.qkv_items)
            return flow_qkv(a, l, item, epoch);
        item -= a.qkv_items;
        if (item < a.attn_items)
            return flow_attention<C, G>(a, l, item, epoch);
        item -= a.attn_items;
        if (item < a.o_items)
            return flow_o(a, l, item, epoch, sAct);
        item -= a.o_items;
        if (item < a.gate_up_items)
            return flow_gateup(a, l, item, epoch);
        item -= a.gate_up_items;
        return flow_down(a, l, item, epoch, sAct);
    }
    item -= a.layers * perLayer;
    if (item == 0)
        return flow_final_norm(a, epoch);
    if (item <= a.head_items)
        return flow_lmhead(a, item - 1, epoch, sAct);
    flow_finalize(a, epoch);
}

} // namespace

// ============================================================================
// Launchers
// ============================================================================
// Channels a lane owns and heads a workgroup merges, by head width.
static bool attention_layout(int head_dim, int *channels, int *group)
{
    if (head_dim == 256 || head_dim == 128 || head_dim == 64) {
        *channels = head_dim / 64;
        *group = 1;
        return true;
    }
    if (head_dim == 32 || head_dim == 16) {
        *channels = 1;
        *group = 32 / head_dim;
        return true;
    }
    return false;
}

bool flow_decode_supported(int layers, int width, int heads, int kv_heads, int head_dim, int intermediate,
                           int vocab, int max_positions)
{
    const int qWidth = heads * head_dim;
    int channels = 0, group = 0;
    return fused_decode_supported(width, heads, kv_heads, head_dim, intermediate, max_positions)
           && attention_layout(head_dim, &channels, &group)
           && layers <= kFlowMaxLayers
           && (int64_t) layers * (heads / group) <= kFlowSubLines            // idle-split sub-counters
           && (vocab + kFlowHeadRows - 1) / kFlowHeadRows <= kFlowSubLines * kFlowFanIn
           && intermediate / kBlock <= kFlowSubLines * kFlowFanIn && width % 4 == 0
           && width <= kFlowThreads * 4 && qWidth <= 64 * kBlock && width <= 64 * kBlock
           && intermediate <= kFlowMaxInner && intermediate % kBlock == 0
           && (head_dim / 2) % 2 == 0
           && flow_attention_splits(max_positions) * kMaxSplitKeys >= max_positions;
}

int flow_attention_splits(int max_positions)
{
    // enough splits that a split never takes more than kMaxSplitKeys keys
    const int needed = (max_positions + kMaxSplitKeys - 1) / kMaxSplitKeys;
    return needed < 16 ? 16 : (needed > kDecodeSplits ? kDecodeSplits : needed);
}

int flow_items(FlowArgs &a)
{
    int channels = 0, group = 1;
    attention_layout(a.head_dim, &channels, &group);
    const int pairs = (a.heads + 2 * a.kv_heads) * (a.head_dim / 2);
    a.qkv_items = (pairs + kFlowQkvPairs - 1) / kFlowQkvPairs;
    a.attn_items = a.attn_splits * (a.heads / group);
    a.o_items = (a.width + kFlowORows - 1) / kFlowORows;
    a.gate_up_items = a.intermediate / kBlock;
    a.down_items = (a.width + kFlowDownRows - 1) / kFlowDownRows;
    a.head_items = (int) ((a.vocab + kFlowHeadRows - 1) / kFlowHeadRows);
    const int perLayer = a.qkv_items + a.attn_items + a.o_items + a.gate_up_items + a.down_items;
    return a.layers * perLayer + 1 + a.head_items + 1;
}

hipError_t launch_flow_step(const FlowArgs &a, hipStream_t stream)
{
    int channels = 0, group = 0;
    if (!attention_layout(a.head_dim, &channels, &group))
        return hipErrorInvalidValue;
    FlowArgs b = a;
    const int grid = flow_items(b);
    if (channels == 4)
        hipLaunchKernelGGL((flow_step_kernel<4, 1>), dim3(grid), dim3(kFlowThreads), 0, stream, b);
    else if (channels == 2)
        hipLaunchKernelGGL((flow_step_kernel<2, 1>), dim3(grid), dim3(kFlowThreads), 0, stream, b);
    else if (group == 1)
        hipLaunchKernelGGL((flow_step_kernel<1, 1>), dim3(grid), dim3(kFlowThreads), 0, stream, b);
    else
        hipLaunchKernelGGL((flow_step_kernel<1, 2>), dim3(grid), dim3(kFlowThreads), 0, stream, b);
    return hipGetLastError();
}

bool fused_decode_supported(int width, int heads, int kv_heads, int head_dim, int intermediate,
                            int max_positions)
{
    const int qWidth = heads * head_dim, kvWidth = kv_heads * head_dim;
    int channels = 0, group = 0;
    return attention_layout(head_dim, &channels, &group) && heads % group == 0
           && group <= kAttnWaves && group * head_dim <= kMaxGroupWidth
           && width % kBlock == 0 && width <= kFusedMaxWidth && qWidth % kBlock == 0
           && heads % kv_heads == 0 && kvWidth % 8 == 0
           && max_positions <= kDecodeSplits * kMaxSplitKeys && intermediate % kBlock == 0
           && intermediate <= 16384;
}


static int head_groups(int vocab)
{
    return (vocab + kHeadWaves * kHeadRows - 1) / (kHeadWaves * kHeadRows);
}

hipError_t launch_qkv_rope(const QkvArgs &a, hipStream_t stream)
{
    const int pairs = (a.heads + 2 * a.kv_heads) * (a.head_dim / 2);
    const int perGroup = kWaves * kPairsPerWave;
    const dim3 grid((pairs + perGroup - 1) / perGroup);
    if (a.embedding)
        hipLaunchKernelGGL(qkv_rope_kernel<true>, grid, dim3(kThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(qkv_rope_kernel<false>, grid, dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

// The one-token attention launch for each key-count range: its splits, the
// keys of a round (4 or 8 a wave), and the keys a split is expected to cover
// (its rows loaded before the position).  Short contexts take half rounds,
// so twice the workgroups share the keys; past 4096 keys a split takes two
// rounds at once.
struct AttentionRange {
    int lastKeys, splits, roundKeys, specKeys;
};
constexpr AttentionRange kAttentionTable[kAttentionRanges] = {
    {512, 16, 32, 32}, {1024, 32, 32, 32}, {2048, 64, 32, 32}, {4096, 64, 64, 64},
    {INT32_MAX, 64, 64, 128}};

int attention_graph_range(int keyCount)
{
    int r = 0;
    while (r + 1 < kAttentionRanges && keyCount > kAttentionTable[r].lastKeys)
        ++r;
    return r;
}

int attention_grid_splits(int keyCount)
{
    return kAttentionTable[attention_graph_range(keyCount)].splits;
}

int attention_round_keys(int keyCount)
{
    return kAttentionTable[attention_graph_range(keyCount)].roundKeys;
}

int attention_spec_keys(int keyCount)
{
    return kAttentionTable[attention_graph_range(keyCount)].specKeys;
}

int attention_key_range(int keyCount, int maxPositions)
{
    return std::min(kAttentionTable[attention_graph_range(keyCount)].lastKeys, maxPositions);
}

hipError_t launch_attention(const AttentionArgs &a, hipStream_t stream)
{
    int channels = 0, group = 0;
    if (!attention_layout(a.head_dim, &channels, &group) || a.heads % group != 0 || !a.q8
        || !a.part_ll || !a.ml_ll || !a.tag_epoch || !a.error)
        return hipErrorInvalidValue;
    if (a.grid_splits < 1 || a.grid_splits > kDecodeSplits
        || (a.round_keys != 32 && a.round_keys != 64)
        || (a.spec_keys != a.round_keys && a.spec_keys != 2 * a.round_keys))
        return hipErrorInvalidValue;
    const dim3 grid(a.grid_splits * (a.heads / group));
#define GQ8_ATTENTION(CC, GG)                                                                  \
    do {                                                                                       \
        if (a.round_keys == 32)                                                                \
            hipLaunchKernelGGL((attention_kernel<CC, GG, 4>), grid, dim3(kAttnThreads), 0, stream, a); \
        else                                                                                   \
            hipLaunchKernelGGL((attention_kernel<CC, GG, 8>), grid, dim3(kAttnThreads), 0, stream, a); \
    } while (0)
    if (channels == 4)
        GQ8_ATTENTION(4, 1);
    else if (channels == 2)
        GQ8_ATTENTION(2, 1);
    else if (group == 1)
        GQ8_ATTENTION(1, 1);
    else
        GQ8_ATTENTION(1, 2);
#undef GQ8_ATTENTION
    return hipGetLastError();
}

hipError_t launch_gateup_geglu(const GateUpArgs &a, hipStream_t stream)
{
    hipLaunchKernelGGL(gateup_geglu_kernel, dim3(a.intermediate / kBlock), dim3(kGluThreads), 0,
                       stream, a);
    return hipGetLastError();
}

// The final norm of the step's row: the row-norm kernel, whose one row takes
// a workgroup for each element a thread holds (each sums the whole row's
// squares and normalizes its share), so the chain after the row arrives is
// one element long.
hipError_t launch_final_norm(const HeadArgs &a, hipStream_t stream)
{
    return launch_rmsnorm(a.hidden, a.norm_weight, 1, a.width, a.epsilon, a.normalised_out, a.q8,
                          stream);
}

hipError_t launch_lmhead_argmax(const HeadArgs &a, hipStream_t stream)
{
    hipLaunchKernelGGL(lmhead_argmax_kernel, dim3(head_groups(a.vocab)), dim3(kHeadThreads), 0, stream,
                       a);
    return hipGetLastError();
}

hipError_t launch_head_finalize(const HeadArgs &a, hipStream_t stream)
{
    hipLaunchKernelGGL(head_finalize_kernel, dim3(1), dim3(64), 0, stream, a);
    return hipGetLastError();
}

} // namespace gq8
