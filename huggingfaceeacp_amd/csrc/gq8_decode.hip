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
//   attention_kernel     split-key attention over the fp16 cache, a
//                        workgroup per (KV head, key split, query-head
//                        group) reading its split's rows once for the group;
//                        every live split merges a share of the channel
//                        blocks from the others' tagged partials and writes
//                        them as the Q8 row for o_proj;
//   (o_proj, down)       q8_matvec_kernel with the residual add;
//   gateup_geglu_kernel  norm + Q8 prologue, the gate|up product, GeGLU and
//                        the Q8 row for down_proj;
//   lmhead_argmax_kernel the final norm and its Q8 row (per workgroup, in
//                        LDS), the tied lm_head over the whole vocabulary,
//                        each workgroup's first maximum merged into one
//                        packed 64-bit word by atomicMax;
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

// ---- KV-stationary split-key attention ---------------------------------------
// Every query head of a KV head reads the same key and value rows
// (MultiQueryAttention.h:138-260: all eight heads read KV head 0), so a
// workgroup takes one key split of one KV head and G of its query heads, and
// loads the split's rows once for all G.  The grid is (KV head, key split,
// head group); the head groups of one (KV head, split) get workgroup ids of
// one residue mod 8, so they run on one XCD and the split's rows come from
// HBM once into that XCD's L2.  Keys go in rounds of 32 (wave w takes keys
// w, w + 8, w + 16, w + 24 of a round; lane l the channels [C l, C l + C)):
//   scores   the round's key rows and the G queries (registers) give G x 4
//            dots a lane, summed across the wave together (reduce_rows); the
//            round's value rows go to LDS;
//   softmax  wave g takes head g: the split's maximum, exp(s - max) and sum;
//   values   wave w owns a channel slice of every head (lane l: head
//            l / (64 / G), VT channels of the slice), reading weights and
//            value rows from LDS, so no cross-wave sum is needed.
// The split's partial (double) and its (max, sum) go out as tagged words (a
// 32-bit half and the launch's tag in one single-copy-atomic agent-scope
// store, coherent across the chip's L2s); the tag is an epoch the q|k|v
// launch before advances, so no word is ever cleared.  Every workgroup of
// the launch, live or not, then merges a share of its head group's 32-channel
// blocks (split s takes blocks s, s + splits, ...): it polls the words it
// needs until they carry the tag, with a bounded wait that sets the error
// word when it gives up.  The merge (MultiQueryAttention.h:43-49: every split
// rescaled to the row maximum in split order, the sums divided by the total)
// rounds to fp32 and quantizes the block.  The workgroups of a launch wait on
// each other, so they must be resident together: the host checks the largest
// grid against the occupancy of the kernel before it takes this path.
// Scores, weights and sums are double throughout.
constexpr int kAttnThreads = 512;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kRoundKeys = 32;                           // keys a round: four a wave
constexpr int kMaxRounds = 4;
constexpr int kMaxSplitKeys = kRoundKeys * kMaxRounds;   // 128: a window of 64 x 128 = 8192
constexpr int kPollSplits = 8; // split partials a merging lane polls (a run of at most 16)

struct SplitPlan {
    int splits, perSplit;
};

// Whole rounds a split, as few as the launch's gridSplits splits allow.
__device__ inline SplitPlan plan_splits(int keyCount, int gridSplits)
{
    const int rounds = (keyCount + kRoundKeys * gridSplits - 1) / (kRoundKeys * gridSplits);
    const int perSplit = rounds * kRoundKeys;
    return {(keyCount + perSplit - 1) / perSplit, perSplit};
}

// The channels of a head row that lane l of a key's 16 lanes holds: SC of
// them, in pieces of at most eight halves (16 bytes) with the 16 lanes'
// pieces side by side, so that each load instruction reads whole lines of
// the row (a lane's 32 contiguous bytes would use half of every line an
// instruction touches).  Half i of the lane's slice is channel
// row_channel<SC>(l, i).
template <int SC>
__device__ inline int row_channel(int l, int i)
{
    static_assert(SC == 4 || SC == 8 || SC == 16, "4, 8 or 16 halves");
    if constexpr (SC == 4)
        return 4 * l + i;
    else
        return (i / 8) * 128 + 8 * l + i % 8;
}

// The lane's SC halves of the fp16 row at p as SC / 2 words (half i in word
// i / 2), and the same words stored to a row in LDS.
template <int SC>
__device__ inline void load_row(const uint16_t *p, int l, uint32_t (&w)[SC / 2])
{
    if constexpr (SC == 4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p + row_channel<SC>(l, 0));
        w[0] = v.x;
        w[1] = v.y;
    } else {
#pragma unroll
        for (int k = 0; k < SC / 8; ++k) {
            const uint4 v = *reinterpret_cast<const uint4 *>(p + row_channel<SC>(l, 8 * k));
            w[4 * k] = v.x;
            w[4 * k + 1] = v.y;
            w[4 * k + 2] = v.z;
            w[4 * k + 3] = v.w;
        }
    }
}

template <int SC>
__device__ inline void store_row(uint16_t *p, int l, const uint32_t (&w)[SC / 2])
{
    if constexpr (SC == 4) {
        *reinterpret_cast<uint2 *>(p + row_channel<SC>(l, 0)) = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
        for (int k = 0; k < SC / 8; ++k)
            *reinterpret_cast<uint4 *>(p + row_channel<SC>(l, 8 * k))
                = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
    }
}

__device__ inline double half_word(uint32_t w, int i)
{
    return (double) half_value((uint16_t) (w >> (16 * i)));
}

// The sum over a value-layout channel's key partitions (lane bits from
// log2(CPW) up), every lane ending with the same total.
template <int CPW>
__device__ inline double sum_partitions(double v)
{
    if constexpr (CPW < 64) {
        v += xor_lane<CPW>(v);
        return sum_partitions<CPW * 2>(v);
    } else {
        return v;
    }
}

// The (key, head) row a lane holds after reduce_halving<G, 8, G> over a
// key's 16 lanes (lane bits 3, 2, ... give the upper half of the rows), and
// whether it is the lowest lane holding it.
template <int U>
__device__ inline int row_of_lane16(int lane)
{
    int row = 0, n = U, bit = 8;
    while (n > 1) {
        n /= 2;
        if (lane & bit)
            row += n;
        bit >>= 1;
    }
    return row;
}

template <int U>
__device__ inline bool stores_row16(int lane)
{
    int bits = 0, n = U, bit = 8;
    while (n > 1) {
        n /= 2;
        bits |= bit;
        bit >>= 1;
    }
    return (lane & 15 & ~bits) == 0;
}

// C: the head width is 64 C; G: query heads a workgroup; R: 32-key rounds a
// split at most (the launch's key-count range).  Score layout: 16 lanes a
// key, lane l the channels [SC (l % 16), SC (l % 16) + SC) of every head of
// the group, wave w the keys 4 w .. 4 w + 3 of a round.  Value layout: lane
// l of wave w the channel w CPW + l % CPW of every head of the group and the
// keys of partition l / CPW (keys j = partition + KP t).
template <int C, int G, int R>
__global__ __launch_bounds__(kAttnThreads)
void attention_kernel(AttentionArgs a)
{
    GQ8_ARGS_EARLY("s"(a.grid_splits), "s"(a.scale), "s"(a.part_ll), "s"(a.ml_ll), "s"(a.tag_epoch),
                   "s"(a.error), "s"(a.out), "s"(a.q8));
    constexpr int kHd = 64 * C;
    constexpr int SC = kHd / 16;                 // score layout: channels a lane
    constexpr int SW = SC / 2;                   // their words
    constexpr int VC = 2;                        // value layout: channels a lane
    constexpr int KP = 512 * VC / kHd;           // value layout: key partitions
    constexpr int CPW = 64 / KP;                 // value layout: lanes of a partition in a wave
    constexpr int kBlocks = G * kHd / kBlock;    // the group's 32-channel blocks
    static_assert(kAttnWaves * 4 == kRoundKeys, "a round is one key a 16-lane group");
    static_assert(CPW * VC * kAttnWaves == kHd, "the value layout covers the head width");
    __shared__ __attribute__((aligned(16))) double sScore[kMaxSplitKeys][G];
    __shared__ __attribute__((aligned(16))) uint16_t sV[kMaxSplitKeys * kHd];
    __shared__ double sMax[G], sSum[G];
    constexpr int kTasks = kBlocks > kAttnWaves ? kBlocks : kAttnWaves;
    __shared__ double sRun[kTasks][kBlock]; // the merge's run sums
    __shared__ double sTotal[kTasks];       // and each run's head total

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int heads = a.heads, kvHeads = a.kv_heads;
    const int perKv = heads / kvHeads, groups = perKv / G;
    const int gridSplits = a.grid_splits, units = kvHeads * gridSplits;
    const int b = (int) blockIdx.x;
    int unit, grp;
    if (units % 8 == 0) { // a unit's head groups on one XCD (ids of one residue mod 8)
        unit = 8 * ((b / 8) / groups) + b % 8;
        grp = (b / 8) % groups;
    } else {
        unit = b / groups;
        grp = b % groups;
    }
    const int kvh = unit / gridSplits, split = unit % gridSplits;
    const int h0 = kvh * perKv + grp * G; // the group's first query head
    const int kvWidth = kvHeads * kHd, qWidth = heads * kHd;
    const int sub = lane >> 4;            // score layout: the wave's key of four
    const int l16 = lane & 15;            // and the lane's slice of a row
    const int kvOffset = kvh * kHd;

    // the position first: its round trip runs beside the rows' loads, which
    // would otherwise all have to return before it
    const int positionLoaded = ld_agent_i(a.position);
    double q[G][SC];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < SC; i += 4) {
            const float4 f = *reinterpret_cast<const float4 *>(a.query + (h0 + g) * kHd
                                                               + row_channel<SC>(l16, i));
            q[g][i] = f.x;
            q[g][i + 1] = f.y;
            q[g][i + 2] = f.z;
            q[g][i + 3] = f.w;
        }

    // The split expected for the launch's range (spec_keys keys from
    // split * spec_keys) has its rows loaded before the position arrives (rows
    // past the position are read, inside the cache, and never used).
    uint32_t kh[R][SW], vh[R][SW];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int j = min(split * a.spec_keys + r * kRoundKeys + 4 * wave + sub, a.max_positions - 1);
        load_row<SC>(a.key_cache + (int64_t) j * kvWidth + kvOffset, l16, kh[r]);
        load_row<SC>(a.value_cache + (int64_t) j * kvWidth + kvOffset, l16, vh[r]);
    }
    // keeps the loads above the position-dependent code
    asm volatile("" ::: "memory");

    const int keyCount = __builtin_amdgcn_readfirstlane(positionLoaded) + 1;
    const SplitPlan plan = plan_splits(keyCount, gridSplits);
    if (plan.perSplit > R * kRoundKeys) {
        // a launch too small for its step's keys (the host sizes it to the
        // range): nothing is computed and the step is reported invalid
        if (t == 0)
            __hip_atomic_fetch_or(a.error, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const bool live = split < plan.splits;
    const uint32_t tag = a.tag_epoch[0];
    if (live) {
        const int k0 = split * plan.perSplit;
        const int n = min(plan.perSplit, keyCount - k0);
        const int rounds = (n + kRoundKeys - 1) / kRoundKeys;
        if (plan.perSplit != a.spec_keys) { // not the split expected: its rows again, from k0
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int j = k0 + min(r * kRoundKeys + 4 * wave + sub, n - 1);
                load_row<SC>(a.key_cache + (int64_t) j * kvWidth + kvOffset, l16, kh[r]);
                load_row<SC>(a.value_cache + (int64_t) j * kvWidth + kvOffset, l16, vh[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r >= rounds) // uniform
                break;
            // the lane's share of each head's dot, in two sums (even and odd
            // channels), then the key's 16 lanes summed together
            double y[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                double p0 = 0.0, p1 = 0.0;
#pragma unroll
                for (int i = 0; i < SC; i += 2) {
                    p0 += q[g][i] * half_word(kh[r][i / 2], 0);
                    p1 += q[g][i + 1] * half_word(kh[r][i / 2], 1);
                }
                y[g] = p0 + p1;
            }
            reduce_halving<G, 8, G>(y, lane);
            const int j = r * kRoundKeys + 4 * wave + sub;
            if (j < n) {
                if (stores_row16<G>(lane))
                    sScore[j][row_of_lane16<G>(lane)] = (double) a.scale * y[0];
                store_row<SC>(sV + j * kHd, l16, vh[r]);
            }
        }
        __syncthreads();

        // softmax of the split, one wave a head; the weights replace the scores
        if (wave < G) {
            double largest = -INFINITY;
            for (int j = lane; j < n; j += 64)
                largest = fmax(largest, sScore[j][wave]);
            largest = wave_max_d(largest);
            double sum = 0.0;
            for (int j = lane; j < n; j += 64) {
                const double w = exp(sScore[j][wave] - largest);
                sScore[j][wave] = w;
                sum += w;
            }
            sum = wave_sum_d(sum);
            if (lane == 0) {
                sMax[wave] = largest;
                sSum[wave] = sum;
            }
        }
        __syncthreads();
        // the split's (max, sum) go out before its values are weighted, so
        // the merging splits have them (and their factors) early
        // (the stored words stay in their registers until the partials are
        // stored: reusing them would wait for these stores to complete)
        const v4u mlMax = tagged_double(sMax[t < G ? t : 0], tag);
        const v4u mlSum = tagged_double(sSum[t < G ? t : 0], tag);
        if (t < G) {
            const uint32_t mlBytes = (uint32_t) (kDecodeSplits * heads * 4 * 8);
            const uint32_t off = (uint32_t) ((split * heads + h0 + t) * 4 * 8);
            st_agent_16(a.ml_ll, off, mlBytes, mlMax);
            st_agent_16(a.ml_ll, off + 16, mlBytes, mlSum);
        }

        // the weighted values: each lane two channels of every head over its
        // partition's keys, four keys a batch in two sums a head; the
        // partitions' sums are then added across lanes in a fixed order
        {
            const int part = lane / CPW;
            const int c = (wave * CPW + lane % CPW) * VC;
            double acc[2][G][VC];
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int i = 0; i < VC; ++i)
                        acc[k][g][i] = 0.0;
            for (int t0 = 0; t0 < n; t0 += 4 * KP) { // the same trip count in every lane
                double w[4][G];
                uint32_t v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int j = t0 + u * KP + part;
                    const int jj = min(j, n - 1); // past n: zero values (reads unconditional)
#pragma unroll
                    for (int g = 0; g < G; ++g)
                        w[u][g] = sScore[jj][g];
                    const uint32_t h = *reinterpret_cast<const uint32_t *>(sV + jj * kHd + c);
                    v[u] = j < n ? h : 0u;
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int i = 0; i < VC; ++i) {
                        const double x = half_word(v[u], i);
#pragma unroll
                        for (int g = 0; g < G; ++g)
                            acc[u & 1][g][i] += w[u][g] * x;
                    }
            }
            asm volatile("" ::"v"(mlMax), "v"(mlSum));
            const uint32_t partBytes = (uint32_t) ((int64_t) kDecodeSplits * qWidth * 16);
            static_assert(VC * CPW <= 64, "a head's channels of the wave in one store");
            const int i = lane / CPW; // lanes i CPW .. i CPW + CPW - 1 store channel c + i
#pragma unroll
            for (int g = 0; g < G; ++g) {
                double total[VC];
#pragma unroll
                for (int k = 0; k < VC; ++k)
                    total[k] = sum_partitions<CPW>(acc[0][g][k] + acc[1][g][k]);
                double mine = total[0];
#pragma unroll
                for (int k = 1; k < VC; ++k)
                    mine = i == k ? total[k] : mine;
                // the split's partials as tagged words (two a double): the
                // wave's VC CPW channels of the head, contiguous, in one store
                if (lane < VC * CPW)
                    st_agent_16(a.part_ll,
                                (uint32_t) (((int64_t) split * qWidth + (h0 + g) * kHd + c + i) * 16),
                                partBytes, tagged_double(mine, tag));
            }
        }
    }

    // The merge (MultiQueryAttention.h:43-49: every split rescaled to the row
    // maximum, in split order, the sums divided by the total): every
    // live split of the group takes blocks split, split + splits, ...; a
    // block's waves each take a run of consecutive splits (lanes 32..63 the
    // second half of the run) and poll every split's (max, sum) of the
    // block's head (stored before the split weighs its values) and their run's
    // partial words, a lane loading again only the words it lacks.  The runs'
    // sums are added in LDS in split order.
    const int splits = plan.splits;
    if (!live)
        return;
    const int mine = split < kBlocks ? (kBlocks - split + splits - 1) / splits : 0;
    if (mine == 0)
        return;
    const int wpb = mine >= kAttnWaves ? 1 : kAttnWaves / mine; // tasks a block
    const int run = (splits + wpb - 1) / wpb;        // splits a task
    const int halfRun = (run + 1) / 2;               // splits a lane
    if (halfRun > kPollSplits) {
        // a lane polls at most kPollSplits splits: with at most 64 splits a
        // block has at least 4 tasks whenever a workgroup has at most two
        // blocks, and a workgroup with more blocks has fewer splits
        if (t == 0)
            __hip_atomic_fetch_or(a.error, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const uint32_t mlBytes = (uint32_t) (kDecodeSplits * heads * 4 * 8);
    const uint32_t partBytes = (uint32_t) ((int64_t) kDecodeSplits * qWidth * 16);
    for (int task = wave; task < mine * wpb; task += kAttnWaves) {
        const int bi = task / wpb, ci = task % wpb;
        const int cg = (split + bi * splits) * kBlock + (lane & (kBlock - 1)); // channel of the group
        const int g = cg / kHd;
        const int sBegin = min(ci * run, splits), sEnd = min(sBegin + run, splits);
        const int lo0 = sBegin, lo1 = min(sBegin + halfRun, sEnd); // the two halves' first splits
        const int lo = lane < 32 ? lo0 : lo1, hi = lane < 32 ? lo1 : sEnd;
        const bool liveSplit = lane < splits;
        const uint32_t mlOff = (uint32_t) (((liveSplit ? lane : 0) * heads + h0 + g) * 4 * 8);
        // every split's (max, sum) and the run's partial words, each lane
        // loading again only the words it still lacks, so that after the last
        // split stores, one trip through the memory system is left
        v4u m0 = v4u{0u, 0u, 0u, 0u}, m1 = m0;
        v4u w[kPollSplits];
#pragma unroll
        for (int u = 0; u < kPollSplits; ++u)
            w[u] = v4u{0u, 0u, 0u, 0u};
        bool mlReady = !liveSplit;
        uint32_t pending = 0; // the run's words not yet seen with the tag
#pragma unroll
        for (int u = 0; u < kPollSplits; ++u)
            pending |= (lo + u < hi ? 1u : 0u) << u;
        int spins = 0;
        for (;;) {
            if (!mlReady) {
                m0 = ld_agent_16(a.ml_ll, mlOff, mlBytes);
                m1 = ld_agent_16(a.ml_ll, mlOff + 16, mlBytes);
            }
#pragma unroll
            for (int u = 0; u < kPollSplits; ++u)
                if (pending & (1u << u))
                    w[u] = ld_agent_16(a.part_ll, (uint32_t) (((lo + u) * qWidth + h0 * kHd + cg) * 16), partBytes);
            mlReady = mlReady || (m0.y == tag && m0.w == tag && m1.y == tag && m1.w == tag);
#pragma unroll
            for (int u = 0; u < kPollSplits; ++u)
                if (w[u].y == tag && w[u].w == tag)
                    pending &= ~(1u << u);
            if (__all(mlReady && pending == 0))
                break;
            if (wait_give_up(a.error, spins)) {
#pragma unroll
                for (int u = 0; u < kPollSplits; ++u)
                    w[u] = v4u{0u, tag, 0u, tag};
                break;
            }
        }
        const double m = __longlong_as_double((long long) (((uint64_t) m0.z << 32) | m0.x));
        const double sum = __longlong_as_double((long long) (((uint64_t) m1.z << 32) | m1.x));
        double total;
        const double f = merge_factor(m, sum, liveSplit, total);
        // this lane's splits' factors, read from the lanes holding them (the
        // two halves' split indices are uniform across their lanes)
        double fu[kPollSplits];
#pragma unroll
        for (int u = 0; u < kPollSplits; ++u) {
            const double f0 = lane_value(f, min(lo0 + u, 63));
            const double f1 = lane_value(f, min(lo1 + u, 63));
            fu[u] = lane < 32 ? f0 : f1;
        }
        double weighted = 0.0;
#pragma unroll
        for (int u = 0; u < kPollSplits; ++u)
            if (lo + u < hi)
                weighted += __longlong_as_double((long long) (((uint64_t) w[u].z << 32) | w[u].x)) * fu[u];
        weighted += xor_lane<32>(weighted); // lanes 0..31: the first half's sum, then the second's
        if (lane < kBlock)
            sRun[task][lane] = weighted;
        if (lane == 0)
            sTotal[task] = total;
    }
    __syncthreads();
    for (int bi = wave; bi < mine; bi += kAttnWaves) {
        const int cg = (split + bi * splits) * kBlock + (lane & (kBlock - 1));
        double total = sRun[bi * wpb][lane & (kBlock - 1)];
        for (int k = 1; k < wpb; ++k)
            total += sRun[bi * wpb + k][lane & (kBlock - 1)];
        const int idx = h0 * kHd + cg;
        const float v = (float) (total / sTotal[bi * wpb]);
        float amax = fabsf(v);
        amax = max_lanes<16>(amax); // lanes 0..31: the block (32..63 repeat it)
        const uint16_t bits = scale_bits_from_amax(amax);
        const float sc = half_value(bits);
        const int byte = quantize_in_block(v, bits, sc, quantize_hint(sc));
        if (lane < kBlock) {
            if (a.out)
                a.out[idx] = v;
            a.q8[idx] = (uint8_t) (int8_t) byte;
            if (lane == 0)
                reinterpret_cast<uint16_t *>(a.q8 + qWidth)[idx / kBlock] = bits;
        }
    }
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
// Every workgroup of the lm_head takes the final norm of the residual row and
// its Q8 into LDS itself (the row's loads issued before its weight loads, the
// norm's chain run while the weights stream in, as gate|up does; workgroup 0
// also writes the normalised row and the Q8 row, the hiddenStates and debug
// views); the lm_head is a one-shot product (every wave loads its eight rows'
// blocks once, the activation block of its lane from the LDS row) whose rows
// are reduced together.  Each workgroup folds its rows into one 64-bit candidate
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
    GQ8_ARGS_EARLY("s"(a.best), "s"(a.logits), "s"(a.q8), "s"(a.normalised_out));
    static_assert(kFusedMaxWidth / 4 / 64 == kHeadWaves, "four row elements a thread");
    __shared__ RowQ8 normRow;
    __shared__ double sPartial[kHeadWaves];
    __shared__ unsigned long long sBest[kHeadWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = a.width / kBlock;
    const bool valid = lane < nb;
    const int64_t V = a.vocab;
    const int64_t r0 = ((int64_t) blockIdx.x * kHeadWaves + wave) * kHeadRows;

    const RowSlice<4> slice = load_row_slice<4>(a.hidden, nullptr, nullptr, 0, 0.f, nullptr,
                                                a.norm_weight, a.width);
    WeightBlock w[kHeadRows];
#pragma unroll
    for (int k = 0; k < kHeadRows; ++k)
        w[k] = load_block(a.weights, V, a.width, r0 + k, lane, valid && r0 + k < V);
    __builtin_amdgcn_sched_barrier(0); // every load issued before the norm's first wait
    norm_q8_finish(slice, a.width, a.epsilon, normRow, sPartial, a.normalised_out, a.q8);
    int4 a0 = make_int4(0, 0, 0, 0), a1 = a0; // an invalid lane's terms are zeroed by block_term
    double sa = 0.0;
    if (valid) {
        a0 = reinterpret_cast<const int4 *>(normRow.q + lane * kBlock)[0];
        a1 = reinterpret_cast<const int4 *>(normRow.q + lane * kBlock)[1];
        sa = normRow.scale[lane];
    }
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

} // namespace

// ============================================================================
// Launchers
// ============================================================================
// Channels a lane owns and heads a workgroup merges, by head width.
bool fused_decode_supported(int width, int heads, int kv_heads, int head_dim, int intermediate)
{
    const int qWidth = heads * head_dim, kvWidth = kv_heads * head_dim;
    return width % kBlock == 0 && width <= kFusedMaxWidth && qWidth % kBlock == 0
           && heads % kv_heads == 0 && kvWidth % 8 == 0 && head_dim % 4 == 0
           && intermediate % kBlock == 0 && intermediate <= 16384;
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

// The one-token attention launch for each key-count range: its splits and
// the 32-key rounds a split takes at most (the rows of that many rounds are
// loaded before the position arrives).  Splits past the step's keys merge
// without attending, so a launch sized to the range keeps its idle splits'
// loads few.
struct AttentionRange {
    int lastKeys, splits, rounds;
};
constexpr AttentionRange kAttentionTable[kAttentionRanges] = {
    {512, 16, 1}, {1024, 32, 1}, {2048, 64, 1}, {4096, 64, 2}, {INT32_MAX, 64, 4}};

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

int attention_rounds(int keyCount)
{
    return kAttentionTable[attention_graph_range(keyCount)].rounds;
}

int attention_key_range(int keyCount, int maxPositions)
{
    return std::min(kAttentionTable[attention_graph_range(keyCount)].lastKeys, maxPositions);
}

int attention_group_heads(int heads, int kv_heads)
{
    const int perKv = kv_heads > 0 ? heads / kv_heads : 0;
    return perKv % 2 == 0 ? 2 : 1;
}

bool split_attention_supported(int heads, int kv_heads, int head_dim, int max_positions)
{
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && kv_heads > 0 && heads > 0
           && heads % kv_heads == 0 && (heads * head_dim) % kBlock == 0
           && max_positions <= kDecodeSplits * kMaxSplitKeys;
}

int attention_grid(int heads, int kv_heads, int keyCount)
{
    const int perKv = heads / kv_heads;
    return kv_heads * attention_grid_splits(keyCount) * (perKv / attention_group_heads(heads, kv_heads));
}

// The kernel instance of a launch: head width, heads a workgroup and rounds.
template <typename F>
static bool with_attention_kernel(int head_dim, int group, int rounds, F &&f)
{
#define GQ8_ATTN_R(CC, GG)                                          \
    do {                                                            \
        if (rounds == 1)                                            \
            f(reinterpret_cast<const void *>(attention_kernel<CC, GG, 1>)); \
        else if (rounds == 2)                                       \
            f(reinterpret_cast<const void *>(attention_kernel<CC, GG, 2>)); \
        else if (rounds == 4)                                       \
            f(reinterpret_cast<const void *>(attention_kernel<CC, GG, 4>)); \
        else                                                        \
            return false;                                           \
    } while (0)
#define GQ8_ATTN_G(CC)                  \
    do {                                \
        if (group == 4)                 \
            GQ8_ATTN_R(CC, 4);          \
        else if (group == 2)            \
            GQ8_ATTN_R(CC, 2);          \
        else if (group == 1)            \
            GQ8_ATTN_R(CC, 1);          \
        else                            \
            return false;               \
    } while (0)
    if (head_dim == 256)
        GQ8_ATTN_G(4);
    else if (head_dim == 128)
        GQ8_ATTN_G(2);
    else if (head_dim == 64)
        GQ8_ATTN_G(1);
    else
        return false;
#undef GQ8_ATTN_G
#undef GQ8_ATTN_R
    return true;
}

bool split_attention_fits(int heads, int kv_heads, int head_dim, int max_positions,
                          const int (&resident)[kAttentionRanges])
{
    if (!split_attention_supported(heads, kv_heads, head_dim, max_positions))
        return false;
    for (int r = 0; r < kAttentionRanges; ++r) {
        const int firstKeys = r == 0 ? 1 : kAttentionTable[r - 1].lastKeys + 1;
        if (firstKeys > max_positions)
            break;
        if (attention_grid(heads, kv_heads, firstKeys) > resident[r])
            return false;
    }
    return true;
}

bool split_attention_resident(int device, int heads, int kv_heads, int head_dim, int max_positions,
                              int (&resident)[kAttentionRanges])
{
    int units = 0;
    if (hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return false;
    const int group = attention_group_heads(heads, kv_heads);
    for (int r = 0; r < kAttentionRanges; ++r) {
        int perUnit = 0;
        hipError_t status = hipSuccess;
        const bool known = with_attention_kernel(head_dim, group, kAttentionTable[r].rounds,
                                                 [&](const void *kernel) {
            status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&perUnit, kernel, kAttnThreads, 0);
        });
        if (!known || status != hipSuccess)
            return false;
        resident[r] = perUnit * units;
    }
    return true;
}

hipError_t launch_attention(const AttentionArgs &a, hipStream_t stream)
{
    if (!split_attention_supported(a.heads, a.kv_heads, a.head_dim, a.max_positions) || !a.q8
        || !a.part_ll || !a.ml_ll || !a.tag_epoch || !a.error)
        return hipErrorInvalidValue;
    if (a.grid_splits < 1 || a.grid_splits > kDecodeSplits || a.rounds < 1 || a.rounds > kMaxRounds
        || a.spec_keys != a.rounds * kRoundKeys)
        return hipErrorInvalidValue;
    const int group = attention_group_heads(a.heads, a.kv_heads);
    const dim3 grid(a.kv_heads * a.grid_splits * (a.heads / a.kv_heads / group));
    const bool known = with_attention_kernel(a.head_dim, group, a.rounds, [&](const void *kernel) {
        hipLaunchKernelGGL(reinterpret_cast<void (*)(AttentionArgs)>(const_cast<void *>(kernel)), grid,
                           dim3(kAttnThreads), 0, stream, a);
    });
    if (!known)
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_gateup_geglu(const GateUpArgs &a, hipStream_t stream)
{
    hipLaunchKernelGGL(gateup_geglu_kernel, dim3(a.intermediate / kBlock), dim3(kGluThreads), 0,
                       stream, a);
    return hipGetLastError();
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
