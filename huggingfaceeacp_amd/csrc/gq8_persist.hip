// gq8_persist.hip -- the one-token decode step as one persistent launch.
//
// A batch-1 decode step is a chain of global dependencies (every product needs
// the whole of its input row) over 2.7 GB of weights.  As separate kernels,
// each link costs a launch, a ramp and a tail, during which the HBM idles.
// Here one launch runs the whole step: one workgroup a compute unit, all
// resident at once, each with a fixed program over every phase of the step
// and a fixed share of every phase's work.  Its eight waves have two roles:
//
//   prefetch waves (4-7)  stream the workgroup's share of every gate|up, down
//                         and lm_head weight row into a ring of four LDS slots
//                         of 34 KB, each wave holding its slot's next stage in
//                         registers, in the order the compute waves consume
//                         them.  They wait only for a slot to be consumed,
//                         never on another workgroup, so these weights stream
//                         while the step's latency-bound links run;
//   compute waves (0-3)   run the chain: q|k|v + RoPE (weights loaded into
//                         registers before the input row arrives), attention
//                         over key splits, the split merge, o (+ residual),
//                         gate|up + GeGLU, down (+ residual), the final norm,
//                         the lm_head and the argmax.
//
// Stage s of the ring (a slot's worth of rows) goes to slot s mod 4, loaded by
// prefetch wave 4 + s mod 4 and consumed by compute wave s mod 4.  Two LDS
// counters a slot say how many stages it has received and given back.
//
// Rows pass between workgroups in tagged words (gq8_device.hpp): the residual
// row, q, this step's k and v, the attention partials, the attention and
// GeGLU Q8 rows and the argmax candidates.  Version of the residual row: 2 l + 1
// after layer l's o, 2 l + 2 after its down; every other row's version is its
// layer.  Every version of a row is read only by waves whose own outputs the
// writer of its next version depends on, so no version is overwritten while
// it is read.  The same argument orders the LDS row buffer's uses inside a
// workgroup: a wave's LDS writes complete before its next global store.
//
// Arithmetic (gq8_numerics.hpp): the same expressions, and for the products the
// same summation trees, as the fused kernels of gq8_decode.hip: the norm of a
// row in the thread layout of norm_q8_finish, a row's blocks reduced across
// the wave by reduce_rows, down's four 128-block parts added in part order.
// Attention takes its own split plan (16 keys a split up to 1024 keys, with
// an online softmax inside longer splits): double throughout, so its results
// differ from the fused kernels' only in the rounding of double sums.
//
// Reference counterparts: Decoder.cpp:579-706 (the layer), Embed.h, RMSNorm.h,
// RoPE.h, Linear.h, MultiQueryAttention.h, GeGLU.h, Argmax.h; the greedy
// loop's on-device token feedback, Gemma.cpp:459-543.
#include "gq8_decode.hpp"
#include "gq8_device.hpp"
#include "gq8_lanes.hpp"
#include "gq8_numerics.hpp"

namespace gq8 {
namespace {

constexpr int kComputeWaves = 4;
constexpr int kSlots = 4;
constexpr int kSlotBytes = 34 * 1024;
constexpr int kSlotScales = 32 * 1024;       // byte offset of a slot's fp16 scales
constexpr int kGateActs = 8;                  // a gate|up stage: 8 gate rows + the 8 up rows
constexpr int kDownStageRows = 2;
constexpr int kHeadStageRows = 16;
constexpr int kMaxWgRows = 8;                 // o / down rows a workgroup
constexpr int kMaxWgBlocks = 8;               // GeGLU output blocks a workgroup
constexpr int kMaxPairsPerWave = 2;           // q|k|v rotate pairs a compute wave
constexpr int kMaxWidth = 2048;
constexpr int kMaxInner = 16384;
constexpr int kRowBufBytes = kMaxInner + kMaxInner / kBlock * 4; // a staged Q8 row (scales as words)
constexpr int kChunkKeys = 16;                // attention keys scored together
constexpr int kMaxSplitKeys = 256;

static_assert(kRowBufBytes >= kMaxWidth * 4, "the row buffer holds an fp32 residual row");

struct Shared {
    uint8_t ring[kSlots][kSlotBytes];
    uint8_t row[kRowBufBytes];                // fp32 residual row, or a Q8 row with scale words
    float act[kMaxWgBlocks][kBlock];          // GeGLU outputs of a block before their Q8
    float resid[kMaxWgRows];                  // the workgroup's rows of the residual stream
    unsigned long long best[kComputeWaves];
    int ready[kSlots], consumed[kSlots];      // stages a slot has received / given back
    int bar;                                  // compute-wave barrier arrivals
    int blockArrivals[kMaxWgBlocks];
    int bestArrivals;
};

// The workgroup's LDS, at file scope so that the out-of-line helpers (shared
// by several phases, to keep the step's code within the instruction cache)
// address it directly.
__shared__ __attribute__((aligned(16))) Shared g_sh;

// ---- the workgroup's share of each phase ----------------------------------------
struct Plan {
    int P, g;
    int nb, nbF, nbQ;           // blocks of width, intermediate, q width
    int pairs, pairsPerWave;    // q|k|v rotate pairs
    int r0, r1;                 // o and down rows
    int gb0, gb1;               // GeGLU output blocks
    int nG, nD, perLayer;       // ring stages a layer
    int hr0, hr1, nH;           // lm_head rows and stages
};

__device__ __forceinline__ int ceil_div(int a, int b)
{
    return (a + b - 1) / b;
}

__device__ __forceinline__ Plan make_plan(const PersistArgs &a, int g)
{
    Plan p;
    p.P = a.grid;
    p.g = g;
    const int W = a.width, F = a.intermediate, hd = a.head_dim;
    p.nb = W / kBlock;
    p.nbF = F / kBlock;
    p.nbQ = a.heads * hd / kBlock;
    p.pairs = (a.heads + 2 * a.kv_heads) * (hd / 2);
    p.pairsPerWave = ceil_div(p.pairs, kComputeWaves * p.P);
    const int rows = ceil_div(W, p.P);
    p.r0 = min(W, g * rows);
    p.r1 = min(W, p.r0 + rows);
    const int blocks = ceil_div(p.nbF, p.P);
    p.gb0 = min(p.nbF, g * blocks);
    p.gb1 = min(p.nbF, p.gb0 + blocks);
    p.nG = (p.gb1 - p.gb0) * (kBlock / kGateActs);
    p.nD = ceil_div(p.r1 - p.r0, kDownStageRows);
    p.perLayer = p.nG + p.nD;
    const int headRows = ceil_div(a.vocab, p.P);
    p.hr0 = min(a.vocab, g * headRows);
    p.hr1 = min(a.vocab, p.hr0 + headRows);
    p.nH = ceil_div(p.hr1 - p.hr0, kHeadStageRows);
    return p;
}

// The lane index, opaque to the optimizer: the phases run inside the layer
// loop, and lane-derived addresses hoisted out of it would stay live across
// the whole step (and spill); recomputing them in each phase costs a few
// integer operations.
__device__ __forceinline__ int opaque_lane()
{
    int lane = __lane_id();
    asm volatile("" : "+v"(lane));
    return lane;
}

// ---- waits inside the workgroup (LDS counters) ---------------------------------
// A wait on an LDS counter polls the LDS only; the error word (a device-scope
// load that costs microseconds while the HBM streams) is read once every
// kLdsErrorCheck polls, so a wave does not sit in that load when the counter
// moves.  A wait gives up after kWaitSpinLimit error checks.
constexpr int kLdsErrorCheck = 1 << 14;

__device__ __forceinline__ bool lds_wait(int *counter, int target, const int *error)
{
    int spins = 0, checks = 0;
    while (__hip_atomic_load(counter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        if ((++spins & (kLdsErrorCheck - 1)) == 0) {
            if (ld_agent_i(error) != 0 || ++checks > kWaitSpinLimit / kLdsErrorCheck) {
                __hip_atomic_fetch_or(const_cast<int *>(error), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return false;
            }
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

__device__ __forceinline__ void lds_release(int *counter, int value)
{
    __hip_atomic_store(counter, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// A barrier of the four compute waves (the prefetch waves keep streaming).
__device__ __forceinline__ bool compute_sync(Shared &sh, int &target, const int *error)
{
    target += kComputeWaves;
    if (__lane_id() == 0)
        __hip_atomic_fetch_add(&sh.bar, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    return lds_wait(&sh.bar, target, error);
}

// LDS writes of this wave complete before its next global store.
__device__ __forceinline__ void lds_writes_done()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
}

// ---- tagged rows ---------------------------------------------------------------
// Words [w0, w1) (w0 even) of a `words`-long tagged row into the row buffer as 32-bit
// values, once each carries `tag`: a lane's batch of 16-byte loads is issued
// at once and re-issued whole until every piece is tagged (one copy of the
// code; re-reading a piece that was already there costs nothing).
__device__ __attribute__((noinline)) bool stage_words(const uint64_t *row, int words, int w0, int w1, uint32_t tag,
                                                      const int *error)
{
    uint32_t *dst = reinterpret_cast<uint32_t *>(g_sh.row);
    constexpr int kBatch = 10; // a quarter of a 16384-wide Q8 row (1152 words) in one batch
    const int lane = opaque_lane();
    for (int base = w0; base < w1; base += 2 * 64 * kBatch) {
        int spins = 0;
        for (;;) {
            v4u v[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int w = base + 2 * (lane + 64 * k);
                v[k] = ld_agent_16(row, (uint32_t) min(w, words - 1) * 8, (uint32_t) words * 8);
            }
            bool ok = true;
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int w = base + 2 * (lane + 64 * k);
                ok = ok && (w >= w1 || (v[k].y == tag && (w + 1 >= words || v[k].w == tag)));
            }
            if (ok) {
#pragma unroll
                for (int k = 0; k < kBatch; ++k) {
                    const int w = base + 2 * (lane + 64 * k);
                    if (w < w1) {
                        dst[w] = v[k].x;
                        if (w + 1 < w1)
                            dst[w + 1] = v[k].z;
                    }
                }
                break;
            }
            if (wait_give_up(error, spins))
                return false;
        }
    }
    return true;
}

// This compute wave's quarter of a tagged row (boundaries even).
__device__ __forceinline__ void quarter(int words, int cw, int &w0, int &w1)
{
    w0 = ((int64_t) words * cw / kComputeWaves) & ~1;
    w1 = cw + 1 == kComputeWaves ? words : (((int64_t) words * (cw + 1) / kComputeWaves) & ~1);
}

// The Q8 byte of each of four consecutive lanes packed into the first lane's
// word; lane 0 of a block also puts the block's scale word (a Q8 row's word
// layout: inner / 4 words of bytes, then one scale word a block).
__device__ __forceinline__ void put_q8(uint64_t *row, int inner, int idx, int byte, uint16_t bits, bool live,
                              uint32_t tag)
{
    const uint32_t b = (uint32_t) byte & 0xFFu;
    const uint32_t w = b | ((uint32_t) __shfl_down((int) b, 1) << 8)
                       | ((uint32_t) __shfl_down((int) b, 2) << 16)
                       | ((uint32_t) __shfl_down((int) b, 3) << 24);
    if (live && (idx & 3) == 0)
        ll_put(row + idx / 4, w, tag);
    if (live && (idx & 31) == 0)
        ll_put(row + inner / 4 + idx / kBlock, bits, tag);
}

__device__ __forceinline__ void put_double(uint64_t *p, double v, uint32_t tag)
{
    const uint64_t bits = (uint64_t) __double_as_longlong(v);
    ll_put(p, (uint32_t) bits, tag);
    ll_put(p + 1, (uint32_t) (bits >> 32), tag);
}

__device__ __forceinline__ double join_double(uint32_t lo, uint32_t hi)
{
    return __longlong_as_double((long long) (((uint64_t) hi << 32) | lo));
}

// A 16-byte piece (two words) of a tagged row, polled until both carry `tag`.
__device__ __forceinline__ bool get_pair(const uint64_t *row, int word, int words, uint32_t tag, const int *error,
                                uint32_t &v0, uint32_t &v1)
{
    const v4u v = ld_agent_16(row, (uint32_t) word * 8, (uint32_t) words * 8);
    v0 = v.x;
    v1 = v.z;
    if (v.y == tag && (word + 1 >= words || v.w == tag))
        return true;
    return ll_get2(row, word, words, tag, error, v0, v1);
}

// N 16-byte pieces (word pairs from even indices) of a tagged row: every load
// issued before the first wait, then each piece not yet tagged polled again,
// so N pieces that are already there cost one round trip, not N.
// Piece k comes from word word[k] of row rows[k] (words[k] words long); the
// batch is re-issued whole until every piece is tagged.
template <int N>
__device__ __forceinline__ bool get_pieces(const uint64_t *const (&rows)[N], const int (&word)[N],
                                           const int (&words)[N], uint32_t tag, const int *error,
                                           uint32_t (&lo)[N], uint32_t (&hi)[N])
{
    int spins = 0;
    for (;;) {
        v4u v[N];
#pragma unroll
        for (int k = 0; k < N; ++k)
            v[k] = ld_agent_16(rows[k], (uint32_t) word[k] * 8, (uint32_t) words[k] * 8);
        bool ok = true;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            lo[k] = v[k].x;
            hi[k] = v[k].z;
            ok = ok && v[k].y == tag && (word[k] + 1 >= words[k] || v[k].w == tag);
        }
        if (ok)
            return true;
        if (wait_give_up(error, spins))
            return false;
    }
}

// N pieces of one row.
template <int N>
__device__ __forceinline__ bool get_pairs(const uint64_t *row, const int (&word)[N], int words, uint32_t tag,
                                          const int *error, uint32_t (&lo)[N], uint32_t (&hi)[N])
{
    const uint64_t *rows[N];
    int sizes[N];
#pragma unroll
    for (int k = 0; k < N; ++k) {
        rows[k] = row;
        sizes[k] = words;
    }
    return get_pieces<N>(rows, word, sizes, tag, error, lo, hi);
}

// C consecutive words from word w (w even unless C == 1) of a tagged row,
// with M more pieces of another row in the same batch.
template <int C>
struct Words {
    static constexpr int kPieces = C == 1 ? 1 : C / 2;
    int piece[kPieces];
    __device__ __forceinline__ void at(int w)
    {
#pragma unroll
        for (int k = 0; k < kPieces; ++k)
            piece[k] = C == 1 ? (w & ~1) : w + 2 * k;
    }
    __device__ __forceinline__ uint32_t value(int w, int i, const uint32_t (&lo)[kPieces],
                                              const uint32_t (&hi)[kPieces]) const
    {
        if (C == 1)
            return (w & 1) ? hi[0] : lo[0];
        return (i & 1) ? hi[i / 2] : lo[i / 2];
    }
};

// ---- norm of a staged fp32 row ---------------------------------------------------
// The Q8 row of a normalised row, a quarter of its 32-blocks a compute wave:
// lane l of wave cw takes elements [32 b + 8 (l % 4), + 8) of block
// b = cw * ceil(nb / 4) + l / 4 (norm_q8_finish's thread layout), so the bytes
// and scales equal the fused kernels'.  Their norm weights are loaded early.
struct NormQuarter {
    float4 w[2];
    int block, part;
    bool live;
};

__device__ __forceinline__ NormQuarter load_norm_quarter(const float *weight, int nb, int cw)
{
    const int lane = opaque_lane();
    NormQuarter q;
    const int per = (nb + kComputeWaves - 1) / kComputeWaves;
    q.block = cw * per + lane / 4;
    q.part = lane % 4;
    q.live = lane / 4 < per && q.block < nb;
    const int e0 = q.live ? q.block * kBlock + q.part * 8 : 0;
    q.w[0] = reinterpret_cast<const float4 *>(weight + e0)[0];
    q.w[1] = reinterpret_cast<const float4 *>(weight + e0)[1];
    return q;
}

// The quarter's bytes (8 a lane) and scales (fp16 bits) into LDS.
__device__ __forceinline__ void quarter_q8(const float *row, const NormQuarter &q, double scale, uint8_t *qBytes,
                                           uint16_t *qScales)
{
    float n[8];
    float amax = 0.f;
    const int e0 = q.live ? q.block * kBlock + q.part * 8 : 0;
    const float4 x0 = reinterpret_cast<const float4 *>(row + e0)[0];
    const float4 x1 = reinterpret_cast<const float4 *>(row + e0)[1];
    const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const float w[8] = {q.w[0].x, q.w[0].y, q.w[0].z, q.w[0].w, q.w[1].x, q.w[1].y, q.w[1].z, q.w[1].w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        n[k] = q.live ? norm_value(x[k], scale, w[k]) : 0.f;
        amax = fmaxf(amax, fabsf(n[k]));
    }
    amax = max_lanes<2>(amax); // the four lanes of the block
    const uint16_t bits = scale_bits_from_amax(amax);
    const float s = half_value(bits);
    const float inverse = bits ? quantize_hint(s) : 0.f;
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int k = 0; k < 8; ++k)
        packed[k / 4] |= (uint32_t) (quantize_in_block(n[k], bits, s, inverse) & 0xFF) << (8 * (k % 4));
    if (q.live) {
        *reinterpret_cast<uint2 *>(qBytes + e0) = make_uint2(packed[0], packed[1]);
        if (q.part == 0)
            qScales[q.block] = bits;
    }
}

// Lane l's 32-block of the Q8 row in LDS (a0, a1 the bytes, sa the scale);
// zero past the row.
__device__ __forceinline__ void lane_block(const uint8_t *qBytes, const uint16_t *qScales, int nb, int4 &a0,
                                           int4 &a1, double &sa)
{
    const int lane = opaque_lane();
    const int b = lane < nb ? lane : 0;
    a0 = reinterpret_cast<const int4 *>(qBytes + b * kBlock)[0];
    a1 = reinterpret_cast<const int4 *>(qBytes + b * kBlock)[1];
    sa = lane < nb ? (double) half_value(qScales[b]) : 0.0;
}

// The Q8 row's place in the row buffer, after the fp32 row.
constexpr int kRowQ8Offset = kMaxWidth * 4;
static_assert(kRowQ8Offset + kMaxWidth + kMaxWidth / kBlock * 2 <= kRowBufBytes, "the Q8 row fits");

// The staged row's norm (every wave sums the squares itself, in
// norm_q8_finish's order for 64 V threads of E elements) and this wave's
// quarter of its Q8 row, into the row buffer after the fp32 row.  One copy for
// every norm of the step.
__device__ __attribute__((noinline)) void norm_q8_quarter(NormQuarter q, int width, float epsilon, int E, int V)
{
    const float *row = reinterpret_cast<const float *>(g_sh.row);
    const int lane = opaque_lane();
    // a lane's 32 elements in 8 loads issued together: thread 64 vw + lane of
    // E = 4 owns float4 vw; of E = 8, float4s 2 vw and 2 vw + 1
    float4 x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int e0 = E == 4 ? (64 * i + lane) * 4 : (64 * (i / 2) + lane) * 8 + 4 * (i % 2);
        x[i] = e0 < width ? *reinterpret_cast<const float4 *>(row + e0) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    double total = 0.0;
    if (E == 4) {
#pragma unroll
        for (int vw = 0; vw < 8; ++vw) {
            const float4 v = x[vw];
            const double squares = (((0.0 + (double) v.x * (double) v.x) + (double) v.y * (double) v.y)
                                    + (double) v.z * (double) v.z) + (double) v.w * (double) v.w;
            total += wave_sum_d(squares);
        }
    } else {
        // a thread's eight squares in order: its first float4's, then its second's
#pragma unroll
        for (int vw = 0; vw < 4; ++vw) {
            const float4 v = x[2 * vw], u = x[2 * vw + 1];
            const double squares =
                (((((((0.0 + (double) v.x * (double) v.x) + (double) v.y * (double) v.y) + (double) v.z * (double) v.z)
                     + (double) v.w * (double) v.w) + (double) u.x * (double) u.x) + (double) u.y * (double) u.y)
                  + (double) u.z * (double) u.z) + (double) u.w * (double) u.w;
            total += wave_sum_d(squares);
        }
    }
    (void) V;
    const double scale = norm_scale(total, width, epsilon);
    uint8_t *qBytes = g_sh.row + kRowQ8Offset;
    quarter_q8(row, q, scale, qBytes, reinterpret_cast<uint16_t *>(qBytes + kMaxWidth));
}

// The norm and Q8 row of the staged row (E elements a thread over V waves, as
// the fused kernel of the same norm), ending with lane l's block in registers.
__device__ __forceinline__ bool norm_q8_row(const PersistArgs &a, Shared &sh, const NormQuarter &q, int nb, int E,
                                            int V, int &bar, int4 &a0, int4 &a1, double &sa)
{
    norm_q8_quarter(q, a.width, a.epsilon, E, V);
    if (!compute_sync(sh, bar, a.error))
        return false;
    const uint8_t *qBytes = sh.row + kRowQ8Offset;
    lane_block(qBytes, reinterpret_cast<const uint16_t *>(qBytes + kMaxWidth), nb, a0, a1, sa);
    return true;
}

// A product term whose weight block and scale sit in LDS.
__device__ __forceinline__ double lds_term(const uint8_t *bytes, const uint16_t *scale, const int4 &a0, const int4 &a1,
                                  double sa)
{
    const int4 w0 = reinterpret_cast<const int4 *>(bytes)[0];
    const int4 w1 = reinterpret_cast<const int4 *>(bytes)[1];
    return (double) dot32(w0, w1, a0, a1) * ((double) half_value(*scale) * sa);
}

// ---- the prefetch program ----------------------------------------------------------
// A stage is at most 32 KB of weight bytes (whole rows, in at most two
// regions) and 2 KB of their fp16 scales (at most two regions), laid out in
// its slot as bytes from offset 0 and scales from kSlotScales.  A prefetch wave
// loads the next stage of its slot into registers (32 16-byte pieces and 8
// scale words a lane) while the slot's current stage is being consumed, then
// writes it into the slot: two stages a wave in hand, eight a workgroup.  Its
// loads go out kLoadBurst at a time, which keeps the HBM busy while leaving the
// memory queues short for the compute waves' latency-bound loads.
constexpr int kStagePieces = 32;
constexpr int kStageScaleWords = 8;
constexpr int kLoadBurst = 8;

struct StageRegions {
    const uint8_t *bytes[2];
    int byteLen[2];
    const uint8_t *scales[2];
    int scaleLen[2];
};

__device__ __forceinline__ StageRegions stage_regions(const PersistArgs &a, const Plan &p, int s)
{
    const int W = a.width, F = a.intermediate;
    StageRegions r;
    if (s < a.layers * p.perLayer) {
        const int l = s / p.perLayer, j = s % p.perLayer;
        if (j < p.nG) {
            // gate rows [o0, o0 + 8) and up rows [F + o0, F + o0 + 8)
            const int o0 = (p.gb0 + j / (kBlock / kGateActs)) * kBlock + (j % (kBlock / kGateActs)) * kGateActs;
            const uint8_t *base = a.gate_up + (int64_t) l * a.gate_up_stride;
            const uint8_t *scales = base + (int64_t) 2 * F * W;
            r.bytes[0] = base + (int64_t) o0 * W;
            r.bytes[1] = base + (int64_t) (F + o0) * W;
            r.byteLen[0] = r.byteLen[1] = kGateActs * W;
            r.scales[0] = scales + (int64_t) o0 * p.nb * 2;
            r.scales[1] = scales + (int64_t) (F + o0) * p.nb * 2;
            r.scaleLen[0] = r.scaleLen[1] = kGateActs * p.nb * 2;
        } else {
            const int q0 = p.r0 + (j - p.nG) * kDownStageRows;
            const int nr = min(kDownStageRows, p.r1 - q0);
            const uint8_t *base = a.down + (int64_t) l * a.down_stride;
            r.bytes[0] = r.bytes[1] = base + (int64_t) q0 * F;
            r.byteLen[0] = nr * F;
            r.byteLen[1] = 0;
            r.scales[0] = r.scales[1] = base + (int64_t) W * F + (int64_t) q0 * p.nbF * 2;
            r.scaleLen[0] = nr * p.nbF * 2;
            r.scaleLen[1] = 0;
        }
    } else {
        const int q0 = p.hr0 + (s - a.layers * p.perLayer) * kHeadStageRows;
        const int nr = min(kHeadStageRows, p.hr1 - q0);
        const int64_t V = a.vocab;
        r.bytes[0] = r.bytes[1] = a.embedding + (int64_t) q0 * W;
        r.byteLen[0] = nr * W;
        r.byteLen[1] = 0;
        r.scales[0] = r.scales[1] = a.embedding + V * W + (int64_t) q0 * p.nb * 2;
        r.scaleLen[0] = nr * p.nb * 2;
        r.scaleLen[1] = 0;
    }
    return r;
}

struct StageRegs {
    int4 piece[kStagePieces];
    uint32_t scale[kStageScaleWords];
};

// A region as a raw buffer: loads past its end read as zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t region_buffer(const uint8_t *base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, bytes, 0x00020000);
}

// Stage regions into registers.  Byte piece i is slot bytes [1024 i + 16 lane,
// + 16): whole-row regions are multiples of 1024 bytes, so a piece lies in one
// region (a uniform choice).  A scale word may straddle the two scale regions
// (rows of fewer than 16 blocks), so it is the OR of both regions' reads, one
// of which is past its region and reads zero.
__device__ __forceinline__ void load_stage(const StageRegions &r, StageRegs &g)
{
    const int lane = opaque_lane();
    const __amdgpu_buffer_rsrc_t b0 = region_buffer(r.bytes[0], r.byteLen[0]);
    const __amdgpu_buffer_rsrc_t b1 = region_buffer(r.bytes[1], r.byteLen[1]);
    const __amdgpu_buffer_rsrc_t s0 = region_buffer(r.scales[0], r.scaleLen[0]);
    const __amdgpu_buffer_rsrc_t s1 = region_buffer(r.scales[1], r.scaleLen[1]);
    typedef int v4i __attribute__((ext_vector_type(4)));
    int issued = 0;
#pragma unroll
    for (int i = 0; i < kStagePieces; ++i) {
        const bool first = 1024 * i < r.byteLen[0];
        const v4i v = __builtin_amdgcn_raw_buffer_load_b128(first ? b0 : b1, 16 * lane,
                                                            first ? 1024 * i : 1024 * i - r.byteLen[0], 0);
        g.piece[i] = make_int4(v.x, v.y, v.z, v.w);
        if (++issued % kLoadBurst == 0)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
#pragma unroll
    for (int j = 0; j < kStageScaleWords; ++j) {
        const int off = 256 * j + 4 * lane;
        // an offset before the second region becomes its length: past its end
        const int off1 = off >= r.scaleLen[0] ? off - r.scaleLen[0] : r.scaleLen[1];
        g.scale[j] = __builtin_amdgcn_raw_buffer_load_b32(s0, off, 0, 0)
                     | __builtin_amdgcn_raw_buffer_load_b32(s1, off1, 0, 0);
        if (++issued % kLoadBurst == 0)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

__device__ __forceinline__ void write_stage(const StageRegions &r, const StageRegs &g, uint8_t *slot)
{
    const int lane = opaque_lane();
    const int bytes = r.byteLen[0] + r.byteLen[1], scales = r.scaleLen[0] + r.scaleLen[1];
#pragma unroll
    for (int i = 0; i < kStagePieces; ++i) {
        const int off = 1024 * i + 16 * lane;
        if (off < bytes)
            *reinterpret_cast<int4 *>(slot + off) = g.piece[i];
    }
#pragma unroll
    for (int j = 0; j < kStageScaleWords; ++j) {
        const int off = 256 * j + 4 * lane;
        if (off < scales)
            *reinterpret_cast<uint32_t *>(slot + kSlotScales + off) = g.scale[j];
    }
}

__device__ __forceinline__ void prefetch_program(const PersistArgs &a, const Plan &p, Shared &sh, int pw)
{
    const int stages = a.layers * p.perLayer + p.nH;
    StageRegs g;
    for (int s = pw, k = 0; s < stages; s += kSlots, ++k) {
        const StageRegions r = stage_regions(a, p, s);
        load_stage(r, g);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // stage s is in registers
        if (!lds_wait(&sh.consumed[pw], k, a.error))    // its slot has given back stage s - 4
            return;
        write_stage(r, g, sh.ring[pw]);
        lds_release(&sh.ready[pw], k + 1);
    }
}

// ---- the compute program -------------------------------------------------------------
struct Ring {
    Shared &sh;
    int cw;
    // The slot holding stage s (s mod 4 == cw), once it has arrived.
    __device__ const uint8_t *wait(int s, const int *error)
    {
        return lds_wait(&sh.ready[cw], s / kSlots + 1, error) ? sh.ring[cw] : nullptr;
    }
    // Gives stage s's slot back (its LDS reads have completed).
    __device__ void release(int s)
    {
        lds_release(&sh.consumed[cw], s / kSlots + 1);
    }
};

// q|k|v + RoPE of layer l: the fused qkv_rope_kernel's arithmetic, a wave
// taking pairsPerWave rotate pairs; k and v also go to the cache row.
__device__ __forceinline__ bool phase_qkv(const PersistArgs &a, const Plan &p, Shared &sh, int cw, int l, int pos,
                          uint32_t epoch, int &bar)
{
    const int lane = opaque_lane();
    const int W = a.width, hd = a.head_dim, half = hd / 2;
    const int qWidth = a.heads * hd, kvWidth = a.kv_heads * hd, outputs = qWidth + 2 * kvWidth;
    const uint8_t *wq = a.qkv + (int64_t) l * a.qkv_stride;
    const int firstPair = (p.g * kComputeWaves + cw) * p.pairsPerWave;
    const bool wgWork = p.g * kComputeWaves * p.pairsPerWave < p.pairs;
    const bool waveWork = firstPair < p.pairs;

    WeightBlock lo[kMaxPairsPerWave], hi[kMaxPairsPerWave];
    int rowLo[kMaxPairsPerWave];
#pragma unroll
    for (int k = 0; k < kMaxPairsPerWave; ++k) {
        const int pair = firstPair + k;
        const int head = pair / half, i = pair % half;
        rowLo[k] = head * hd + i; // q heads, then k heads, then v heads
        const bool valid = k < p.pairsPerWave && pair < p.pairs && lane < p.nb;
        lo[k] = load_block(wq, outputs, W, rowLo[k], lane, valid);
        hi[k] = load_block(wq, outputs, W, rowLo[k] + half, lane, valid);
    }
    const NormQuarter nq = load_norm_quarter(a.input_norm + (int64_t) l * a.norm_stride, p.nb, cw);
    // the rotary rows of this wave's pairs (the position is known at the start)
    float cosine[kMaxPairsPerWave], sine[kMaxPairsPerWave];
#pragma unroll
    for (int k = 0; k < kMaxPairsPerWave; ++k) {
        const int64_t angle = (int64_t) pos * half + (firstPair + k) % half;
        cosine[k] = a.cosines[angle];
        sine[k] = a.sines[angle];
    }

    float *row = reinterpret_cast<float *>(sh.row);
    if (l == 0) {
        // the embedding row of sequence[pos] (Embed.h:45-82), a quarter a wave
        uint32_t id = a.sequence[pos];
        if (id >= (uint32_t) a.vocab) // ids are validated on the host; a guard, not a rule
            id = 0;
        const int64_t V = a.vocab;
        const uint8_t *table = a.embedding + (int64_t) id * W;
        const uint16_t *scales = reinterpret_cast<const uint16_t *>(a.embedding + V * W) + (int64_t) id * p.nb;
        const int q = W / kComputeWaves;
        for (int e = cw * q + 4 * lane; e < (cw + 1) * q; e += 4 * 64) {
            const int packed = *reinterpret_cast<const int *>(table + e);
            const float sc = half_value(scales[e / kBlock]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float b = (float) (int8_t) (packed >> (8 * k));
                row[e + k] = (float) ((double) a.embed_scale * (double) (sc * b));
            }
        }
    } else if (wgWork) {
        int w0, w1;
        quarter(W, cw, w0, w1);
        if (!stage_words(a.hid_ll, W, w0, w1, word_tag(epoch, 2 * l), a.error))
            return false;
    }
    if (l == 0 || wgWork) {
        if (!compute_sync(sh, bar, a.error))
            return false;
    }
    if (l == 0) {
        // the workgroup's rows of the residual stream: the embedding row
        for (int i = lane; i < p.r1 - p.r0; i += 64)
            if (i >= 2 * cw && i < 2 * cw + 2)
                sh.resid[i] = row[p.r0 + i];
    }
    if (!wgWork)
        return true;
    int4 a0, a1;
    double sa;
    if (!norm_q8_row(a, sh, nq, p.nb, 8, 4, bar, a0, a1, sa))
        return false;
    if (!waveWork)
        return true;
    constexpr int kRows = 2 * kMaxPairsPerWave;
    double y[kRows];
#pragma unroll
    for (int k = 0; k < kMaxPairsPerWave; ++k) {
        y[2 * k] = block_term(lo[k], a0, a1, sa);
        y[2 * k + 1] = block_term(hi[k], a0, a1, sa);
    }
    const double total = reduce_rows<kRows>(y, lane);
    double rowTotal[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
        rowTotal[r] = lane_value(total, lane_of_row<kRows>(r));
    const uint32_t tag = word_tag(epoch, l);
    const size_t layerCache = (size_t) l * a.max_positions * kvWidth;
#pragma unroll
    for (int k = 0; k < kMaxPairsPerWave; ++k) {
        const int pair = firstPair + k;
        if (lane != 0 || k >= p.pairsPerWave || pair >= p.pairs)
            continue;
        const int r = rowLo[k];
        const float fLo = (float) rowTotal[2 * k], fHi = (float) rowTotal[2 * k + 1];
        if (r < qWidth) {
            float outLo, outHi;
            rotate_pair(fLo, fHi, cosine[k], sine[k], &outLo, &outHi);
            ll_put(a.q_ll + r, __float_as_uint(outLo), tag);
            ll_put(a.q_ll + r + half, __float_as_uint(outHi), tag);
        } else if (r < qWidth + kvWidth) {
            float outLo, outHi;
            rotate_pair(fLo, fHi, cosine[k], sine[k], &outLo, &outHi);
            const int c = r - qWidth;
            const uint16_t bLo = half_bits(outLo), bHi = half_bits(outHi);
            uint16_t *keys = a.key_cache + layerCache + (size_t) pos * kvWidth + c;
            keys[0] = bLo;
            keys[half] = bHi;
            ll_put(a.kv_ll + c, bLo, tag);
            ll_put(a.kv_ll + c + half, bHi, tag);
        } else {
            const int c = r - qWidth - kvWidth;
            const uint16_t bLo = half_bits(fLo), bHi = half_bits(fHi);
            uint16_t *values = a.value_cache + layerCache + (size_t) pos * kvWidth + c;
            values[0] = bLo;
            values[half] = bHi;
            ll_put(a.kv_ll + kvWidth + c, bLo, tag);
            ll_put(a.kv_ll + kvWidth + c + half, bHi, tag);
        }
    }
    return true;
}

// C consecutive fp16 values of a cache row, packed two a word.
template <int C>
struct HalfRow {
    uint32_t w[(C + 1) / 2];
};

template <int C>
__device__ __forceinline__ HalfRow<C> load_half_row(const uint16_t *p)
{
    HalfRow<C> r;
    if constexpr (C == 4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        r.w[0] = v.x;
        r.w[1] = v.y;
    } else if constexpr (C == 2) {
        r.w[0] = *reinterpret_cast<const uint32_t *>(p);
    } else {
        r.w[0] = *p;
    }
    return r;
}

template <int C>
__device__ __forceinline__ float half_at(const HalfRow<C> &r, int i)
{
    return half_value((uint16_t) (r.w[i / 2] >> (16 * (i & 1))));
}

template <int C>
__device__ __forceinline__ void set_half(HalfRow<C> &r, int i, uint16_t bits)
{
    const int shift = 16 * (i & 1);
    r.w[i / 2] = (r.w[i / 2] & ~(0xFFFFu << shift)) | ((uint32_t) bits << shift);
}

// Attention split plan: kChunkKeys keys a split while at most
// kPersistMaxSplits splits cover the keys, else longer splits.
struct AttnPlan {
    int splits, perSplit;
};

__device__ __forceinline__ AttnPlan attn_plan(int keyCount)
{
    const int chunks = ceil_div(keyCount, kChunkKeys * kPersistMaxSplits);
    const int perSplit = chunks * kChunkKeys;
    return {ceil_div(keyCount, perSplit), perSplit};
}

// The tasks of the attention phase: (split, query head), one wave each.  Task
// u covers head (u / 8) % H of split (u % 8) + 8 (u / 8H), so that the heads
// of one split sit on workgroups of one XCD (workgroup u mod P) and share
// their keys through its L2.
__device__ __forceinline__ int attn_tasks(int splits, int heads)
{
    return 8 * heads * ceil_div(splits, 8);
}

// Split sp of head h over C channels a lane: keys [sp n, sp n + n) of the
// pos + 1 attended, scored kChunkKeys at a time with an online softmax
// (MultiQueryAttention.h:43-49, 138-260; the scores, weights and sums in
// double); its partial (the value sums, the maximum and the sum of weights)
// goes out in tagged words.
template <int C>
__device__ __forceinline__ bool attention_task(const PersistArgs &a, int l, int pos, int sp, int h, const AttnPlan &plan,
                               uint32_t epoch)
{
    const int lane = opaque_lane();
    const int hd = a.head_dim, kvWidth = a.kv_heads * hd, qWidth = a.heads * hd;
    const int perKv = a.heads / a.kv_heads;
    const int kvh = h / perKv;
    const bool active = lane * C < hd;
    const int c0 = active ? lane * C : 0;
    const int k0 = sp * plan.perSplit;
    const int n = min(plan.perSplit, pos + 1 - k0);
    const size_t layerCache = (size_t) l * a.max_positions * kvWidth;
    const uint16_t *keys = a.key_cache + layerCache + kvh * hd + c0;
    const uint16_t *values = a.value_cache + layerCache + kvh * hd + c0;
    const uint32_t tag = word_tag(epoch, l);

    double m = -INFINITY, sum = 0.0;
    double acc[C];
#pragma unroll
    for (int i = 0; i < C; ++i)
        acc[i] = 0.0;
    // the first chunk's cached keys and values are loaded before q arrives
    HalfRow<C> kh[kChunkKeys], vh[kChunkKeys];
    auto load_chunk = [&](int j0) {
#pragma unroll
        for (int jj = 0; jj < kChunkKeys; ++jj) {
            const int key = min(k0 + j0 + jj, max(pos - 1, 0));
            kh[jj] = load_half_row<C>(keys + (size_t) key * kvWidth);
            vh[jj] = load_half_row<C>(values + (size_t) key * kvWidth);
        }
    };
    load_chunk(0);
    // q, and this step's key and value if the split holds the position (from
    // the q|k|v phase's tagged rows): one batch of polls
    const bool freshHere = pos >= k0 && pos < k0 + n;
    Words<C> qw, kw, vw;
    qw.at(h * hd + c0);
    kw.at(kvh * hd + c0);
    vw.at(kvWidth + kvh * hd + c0);
    constexpr int P = Words<C>::kPieces;
    int word[3 * P];
    uint32_t lo[3 * P], hi[3 * P];
#pragma unroll
    for (int k = 0; k < P; ++k) {
        word[k] = qw.piece[k];
        word[P + k] = kw.piece[k];
        word[2 * P + k] = vw.piece[k];
    }
    double q[C];
    HalfRow<C> fk = kh[0], fv = vh[0];
    if (freshHere) {
        const uint64_t *rows[3 * P];
        int sizes[3 * P];
#pragma unroll
        for (int k = 0; k < 3 * P; ++k) {
            rows[k] = k < P ? a.q_ll : a.kv_ll;
            sizes[k] = k < P ? qWidth : 2 * kvWidth;
        }
        if (!get_pieces<3 * P>(rows, word, sizes, tag, a.error, lo, hi))
            return false;
    } else {
        int wq[P];
        uint32_t ql[P], qh[P];
#pragma unroll
        for (int k = 0; k < P; ++k)
            wq[k] = word[k];
        if (!get_pairs<P>(a.q_ll, wq, qWidth, tag, a.error, ql, qh))
            return false;
#pragma unroll
        for (int k = 0; k < P; ++k) {
            lo[k] = ql[k];
            hi[k] = qh[k];
        }
    }
    {
        uint32_t ql[P], qh[P], kl[P], khi[P], vl[P], vhi[P];
#pragma unroll
        for (int k = 0; k < P; ++k) {
            ql[k] = lo[k];
            qh[k] = hi[k];
            kl[k] = lo[P + k];
            khi[k] = hi[P + k];
            vl[k] = lo[2 * P + k];
            vhi[k] = hi[2 * P + k];
        }
#pragma unroll
        for (int i = 0; i < C; ++i) {
            q[i] = active ? (double) __uint_as_float(qw.value(h * hd + c0, i, ql, qh)) : 0.0;
            if (freshHere) {
                set_half<C>(fk, i, (uint16_t) kw.value(kvh * hd + c0, i, kl, khi));
                set_half<C>(fv, i, (uint16_t) vw.value(kvWidth + kvh * hd + c0, i, vl, vhi));
            }
        }
    }
    for (int j0 = 0; j0 < n; j0 += kChunkKeys) {
        if (j0 > 0)
            load_chunk(j0);
        const int fresh = pos - k0 - j0; // its place in the chunk, if any
        if (fresh >= 0 && fresh < kChunkKeys) {
#pragma unroll
            for (int jj = 0; jj < kChunkKeys; ++jj)
                if (jj == fresh) {
                    kh[jj] = fk;
                    vh[jj] = fv;
                }
        }
        double y[kChunkKeys];
#pragma unroll
        for (int jj = 0; jj < kChunkKeys; ++jj) {
            double d = 0.0;
#pragma unroll
            for (int i = 0; i < C; ++i)
                d += q[i] * (double) half_at<C>(kh[jj], i);
            y[jj] = d;
        }
        const double total = reduce_rows<kChunkKeys>(y, lane);
        const int mine = row_of_lane<kChunkKeys>(lane);
        const bool live = j0 + mine < n;
        const double score = live ? (double) a.attn_scale * total : -INFINITY;
        const double chunkMax = wave_max_d(score);
        const double mNew = fmax(m, chunkMax);
        const double e = live ? exp(score - mNew) : 0.0;
        const double chunkSum = wave_sum_d(stores_row<kChunkKeys>(lane) ? e : 0.0);
        const double factor = m == -INFINITY ? 0.0 : exp(m - mNew);
        sum = sum * factor + chunkSum;
#pragma unroll
        for (int i = 0; i < C; ++i)
            acc[i] *= factor;
#pragma unroll
        for (int jj = 0; jj < kChunkKeys; ++jj) {
            const double w = lane_value(e, lane_of_row<kChunkKeys>(jj));
#pragma unroll
            for (int i = 0; i < C; ++i)
                acc[i] += w * (double) half_at<C>(vh[jj], i);
        }
        m = mNew;
    }
    const int64_t part = ((int64_t) sp * a.heads + h) * hd;
    if (active)
#pragma unroll
        for (int i = 0; i < C; ++i)
            put_double(a.part_ll + (part + c0 + i) * 2, acc[i], tag);
    // the partials have completed before their (max, sum) is put, so a
    // merge that sees the (max, sum) finds the partials tagged
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) {
        uint64_t *ml = a.ml_ll + ((int64_t) sp * a.heads + h) * 4;
        put_double(ml, m, tag);
        put_double(ml + 2, sum, tag);
    }
    return true;
}

// The merge of one head's splits for one 32-channel block of the attention
// row (MultiQueryAttention.h:43-49: each split rescaled to the row maximum,
// the sums divided by the total), and the block's Q8.  Lane sp polls split
// sp's (max, sum); every split's partials completed before it, so then one
// batch of loads finds them: lanes c and c + 32 take channel c's first and
// second half of the splits (in split order), added in that order.
constexpr int kMergeBatch = 24;

__device__ __forceinline__ bool merge_task(const PersistArgs &a, int l, int h, int cb, const AttnPlan &plan,
                                           uint32_t epoch)
{
    const int lane = opaque_lane();
    const int hd = a.head_dim, qWidth = a.heads * hd;
    const uint32_t tag = word_tag(epoch, l);
    const int splits = plan.splits;
    const int mlWords = kPersistMaxSplits * a.heads * 4;
    const int partWords = kPersistMaxSplits * qWidth * 2;
    const int sp = lane < splits ? lane : 0;
    const int mlWord[2] = {(sp * a.heads + h) * 4, (sp * a.heads + h) * 4 + 2};
    uint32_t mlLo[2], mlHi[2];
    if (!get_pairs<2>(a.ml_ll, mlWord, mlWords, tag, a.error, mlLo, mlHi))
        return false;
    const uint32_t m0 = mlLo[0], m1 = mlHi[0], s0 = mlLo[1], s1 = mlHi[1];
    double total;
    const double f = merge_factor(join_double(m0, m1), join_double(s0, s1), lane < splits, total);
    const int c = lane & (kBlock - 1);
    const int ch = h * hd + cb * kBlock + c;
    const int firstHalf = (splits + 1) / 2;
    const int sBegin = lane < kBlock ? 0 : firstHalf;
    const int sEnd = lane < kBlock ? firstHalf : splits;
    double weighted = 0.0;
    for (int s = 0; s < firstHalf; s += kMergeBatch) {
        int word[kMergeBatch];
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u)
            word[u] = (int) (((int64_t) min(sBegin + s + u, splits - 1) * qWidth + ch) * 2);
        uint32_t lo[kMergeBatch], hi[kMergeBatch];
        if (!get_pairs<kMergeBatch>(a.part_ll, word, partWords, tag, a.error, lo, hi))
            return false;
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            // split s + u's factor for the first half, firstHalf + s + u's for
            // the second (cross-lane reads at wave-uniform lanes)
            const double fFirst = lane_value(f, min(s + u, splits - 1));
            const double fSecond = lane_value(f, min(firstHalf + s + u, splits - 1));
            if (sBegin + s + u < sEnd)
                weighted += join_double(lo[u], hi[u]) * (lane < kBlock ? fFirst : fSecond);
        }
    }
    // the first half's sum, then the second's: the same value in lanes c, c + 32
    const double other = xor_lane<32>(weighted);
    const double sum = lane < kBlock ? weighted + other : other + weighted;
    const float v = (float) (sum / total);
    float amax = fabsf(v);
    amax = max_lanes<16>(amax);
    const uint16_t bits = scale_bits_from_amax(amax);
    const float sc = half_value(bits);
    const int byte = quantize_in_block(v, bits, sc, quantize_hint(sc));
    put_q8(a.attn_ll, qWidth, ch, byte, bits, lane < kBlock, tag);
    return true;
}

// o (+ residual) for this wave's two rows of the workgroup's rows.
__device__ __forceinline__ bool phase_o(const PersistArgs &a, const Plan &p, Shared &sh, int cw, int l, uint32_t epoch)
{
    const int lane = opaque_lane();
    const int qWidth = a.heads * a.head_dim;
    const int rBase = p.r0 + 2 * cw;
    if (rBase >= p.r1)
        return true;
    // the weights first: they stream while the attention row is polled
    WeightBlock w[2];
    const uint8_t *wOut = a.out + (int64_t) l * a.out_stride;
#pragma unroll
    for (int k = 0; k < 2; ++k)
        w[k] = load_block(wOut, a.width, qWidth, rBase + k, lane, lane < p.nbQ && rBase + k < p.r1);
    const uint32_t tag = word_tag(epoch, l);
    const int words = qWidth / 4 + p.nbQ;
    const int b = lane < p.nbQ ? lane : 0;
    // the block's eight byte words and the piece holding its scale word: one batch
    const int scaleWord = qWidth / 4 + b;
    const int word[5] = {b * 8, b * 8 + 2, b * 8 + 4, b * 8 + 6, scaleWord & ~1};
    uint32_t lo[5], hi[5];
    if (!get_pairs<5>(a.attn_ll, word, words, tag, a.error, lo, hi))
        return false;
    const uint32_t bw[8] = {lo[0], hi[0], lo[1], hi[1], lo[2], hi[2], lo[3], hi[3]};
    const uint32_t scaleBits = (scaleWord & 1) ? hi[4] : lo[4];
    const int4 a0 = make_int4((int) bw[0], (int) bw[1], (int) bw[2], (int) bw[3]);
    const int4 a1 = make_int4((int) bw[4], (int) bw[5], (int) bw[6], (int) bw[7]);
    const double sa = lane < p.nbQ ? (double) half_value((uint16_t) scaleBits) : 0.0;
    double y[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
        y[k] = block_term(w[k], a0, a1, sa);
    const double total = reduce_rows<2>(y, lane);
    const int r = rBase + row_of_lane<2>(lane);
    if (stores_row<2>(lane) && r < p.r1) {
        const float updated = (float) (total + (double) sh.resid[r - p.r0]);
        sh.resid[r - p.r0] = updated;
        lds_writes_done();
        ll_put(a.hid_ll + r, __float_as_uint(updated), word_tag(epoch, 2 * l + 1));
    }
    return true;
}

// gate|up + GeGLU of layer l: the post-attention norm of the residual row,
// then this wave's stages, each 8 gate rows and their 8 up rows; the last
// wave of a 32-block quantizes it (gateup_geglu_kernel's arithmetic).
__device__ __forceinline__ bool phase_gateup(const PersistArgs &a, const Plan &p, Shared &sh, Ring &ring, int cw, int l,
                             int stageBase, uint32_t epoch, int &bar)
{
    if (p.nG == 0)
        return true;
    const int W = a.width, F = a.intermediate;
    const NormQuarter nq = load_norm_quarter(a.post_norm + (int64_t) l * a.norm_stride, p.nb, cw);
    int w0, w1;
    quarter(W, cw, w0, w1);
    if (!stage_words(a.hid_ll, W, w0, w1, word_tag(epoch, 2 * l + 1), a.error))
        return false;
    if (!compute_sync(sh, bar, a.error))
        return false;
    int4 a0, a1;
    double sa;
    if (!norm_q8_row(a, sh, nq, p.nb, 4, 8, bar, a0, a1, sa))
        return false;
    const uint32_t tag = word_tag(epoch, l);
    constexpr int kStagesPerBlock = kBlock / kGateActs;
    constexpr int kRows = 2 * kGateActs;
    for (int j = 0; j < p.nG; ++j) {
        const int s = stageBase + j;
        if ((s & (kSlots - 1)) != cw)
            continue;
        const uint8_t *slot = ring.wait(s, a.error);
        if (!slot)
            return false;
        const int lane = opaque_lane(); // stage addresses recomputed, not kept across stages
        const uint16_t *scales = reinterpret_cast<const uint16_t *>(slot + kSlotScales);
        const int b = lane < p.nb ? lane : 0;
        double y[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            y[r] = lds_term(slot + r * W + b * kBlock, scales + r * p.nb + b, a0, a1, sa); // sa = 0 past the row
            if (r % 4 == 3) // four rows' loads at a time
                __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        ring.release(s);
        const double total = reduce_rows<kRows>(y, lane);
        float gate = 0.f, up = 0.f;
#pragma unroll
        for (int i = 0; i < kGateActs; ++i) {
            const float gi = (float) lane_value(total, lane_of_row<kRows>(i));
            const float ui = (float) lane_value(total, lane_of_row<kRows>(kGateActs + i));
            if (lane == i) {
                gate = gi;
                up = ui;
            }
        }
        const int blk = j / kStagesPerBlock, sub = j % kStagesPerBlock;
        if (lane < kGateActs)
            sh.act[blk][sub * kGateActs + lane] = geglu(gate, up);
        int last = 0;
        if (lane == 0)
            last = __hip_atomic_fetch_add(&sh.blockArrivals[blk], 1, __ATOMIC_ACQ_REL,
                                          __HIP_MEMORY_SCOPE_WORKGROUP) == kStagesPerBlock * (l + 1) - 1;
        if (__builtin_amdgcn_readfirstlane(last)) {
            const int o = (p.gb0 + blk) * kBlock + (lane & (kBlock - 1));
            const float v = sh.act[blk][lane & (kBlock - 1)];
            float amax = fabsf(v);
            amax = max_lanes<16>(amax);
            const uint16_t bits = scale_bits_from_amax(amax);
            const float sc = half_value(bits);
            const int byte = quantize_in_block(v, bits, sc, quantize_hint(sc));
            put_q8(a.act_ll, F, o, byte, bits, lane < kBlock, tag);
        }
    }
    return true;
}

// down (+ residual) of layer l: the GeGLU Q8 row staged in LDS, then this
// wave's stages of two rows (q8_matvec_kernel<1, 4, 2>'s order: part p of a
// lane is blocks lane + 64 p and lane + 64 (p + 4), the four parts added in
// order after the wave sums).
__device__ __forceinline__ bool phase_down(const PersistArgs &a, const Plan &p, Shared &sh, Ring &ring, int cw, int l,
                           int stageBase, uint32_t epoch, int &bar)
{
    if (p.nD == 0)
        return true;
    const int F = a.intermediate;
    const int words = F / 4 + p.nbF;
    int w0, w1;
    quarter(words, cw, w0, w1);
    uint32_t *staged = reinterpret_cast<uint32_t *>(sh.row);
    if (!stage_words(a.act_ll, words, w0, w1, word_tag(epoch, l), a.error))
        return false;
    if (!compute_sync(sh, bar, a.error))
        return false;
    const uint8_t *act = sh.row;
    const uint32_t *actScales = staged + F / 4;
    const uint32_t tag = word_tag(epoch, 2 * l + 2);
    for (int i = 0; i < p.nD; ++i) {
        const int s = stageBase + p.nG + i;
        if ((s & (kSlots - 1)) != cw)
            continue;
        const uint8_t *slot = ring.wait(s, a.error);
        if (!slot)
            return false;
        const int lane = opaque_lane(); // stage addresses recomputed, not kept across stages
        const uint16_t *scales = reinterpret_cast<const uint16_t *>(slot + kSlotScales);
        const int q0 = p.r0 + i * kDownStageRows;
        const int nr = min(kDownStageRows, p.r1 - q0);
        double y[kDownStageRows * 4];
#pragma unroll
        for (int rr = 0; rr < kDownStageRows; ++rr)
#pragma unroll
            for (int part = 0; part < 4; ++part)
                y[rr * 4 + part] = 0.0;
        // a part's two activation blocks serve both rows; one part's loads at a
        // time keeps the registers of the stage's 16 terms from being live at once
#pragma unroll
        for (int part = 0; part < 4; ++part) {
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int b = lane + 64 * (part + 4 * jj);
                const bool live = b < p.nbF;
                const int bb = live ? b : 0;
                const int4 x0 = reinterpret_cast<const int4 *>(act + bb * kBlock)[0];
                const int4 x1 = reinterpret_cast<const int4 *>(act + bb * kBlock)[1];
#pragma unroll
                for (int rr = 0; rr < kDownStageRows; ++rr) {
                    const bool valid = live && rr < nr;
                    const double sx = valid ? (double) half_value((uint16_t) actScales[bb]) : 0.0;
                    const int row = valid ? rr : 0;
                    y[rr * 4 + part] += lds_term(slot + row * F + bb * kBlock, scales + row * p.nbF + bb,
                                                 x0, x1, sx);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        ring.release(s);
        const double total = reduce_rows<kDownStageRows * 4>(y, lane);
#pragma unroll
        for (int rr = 0; rr < kDownStageRows; ++rr) {
            double sum = 0.0;
#pragma unroll
            for (int part = 0; part < 4; ++part)
                sum += lane_value(total, lane_of_row<kDownStageRows * 4>(rr * 4 + part));
            const int r = q0 + rr;
            if (lane == 0 && rr < nr) {
                const float updated = (float) (sum + (double) sh.resid[r - p.r0]);
                sh.resid[r - p.r0] = updated;
                lds_writes_done();
                ll_put(a.hid_ll + r, __float_as_uint(updated), tag);
            }
        }
    }
    return true;
}

// The final norm, the workgroup's lm_head rows (logits and their first
// maximum) and, in workgroup 0, the id: lmhead_argmax_kernel's arithmetic and
// head_finalize_kernel's rule.
__device__ __forceinline__ bool phase_head(const PersistArgs &a, const Plan &p, Shared &sh, Ring &ring, int cw, int pos,
                           uint32_t epoch, int &bar)
{
    const int lane = opaque_lane();
    const int W = a.width;
    const NormQuarter nq = load_norm_quarter(a.final_norm, p.nb, cw);
    int w0, w1;
    quarter(W, cw, w0, w1);
    if (!stage_words(a.hid_ll, W, w0, w1, word_tag(epoch, 2 * a.layers), a.error))
        return false;
    if (!compute_sync(sh, bar, a.error))
        return false;
    int4 a0, a1;
    double sa;
    if (!norm_q8_row(a, sh, nq, p.nb, 8, 4, bar, a0, a1, sa))
        return false;
    const int headBase = a.layers * p.perLayer;
    unsigned long long best = 0;
    for (int i = 0; i < p.nH; ++i) {
        const int s = headBase + i;
        if ((s & (kSlots - 1)) != cw)
            continue;
        const uint8_t *slot = ring.wait(s, a.error);
        if (!slot)
            return false;
        const int lane = opaque_lane(); // stage addresses recomputed, not kept across stages
        const uint16_t *scales = reinterpret_cast<const uint16_t *>(slot + kSlotScales);
        const int q0 = p.hr0 + i * kHeadStageRows;
        const int nr = min(kHeadStageRows, p.hr1 - q0);
        const int b = lane < p.nb ? lane : 0;
        double y[kHeadStageRows];
#pragma unroll
        for (int r = 0; r < kHeadStageRows; ++r) {
            const int rr = r < nr ? r : 0; // rows past the stage read row 0 and are never stored
            y[r] = lds_term(slot + rr * W + b * kBlock, scales + rr * p.nb + b, a0, a1, sa);
            if (r % 4 == 3) // four rows' loads at a time
                __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        ring.release(s);
        const double total = reduce_rows<kHeadStageRows>(y, lane);
        const int r = row_of_lane<kHeadStageRows>(lane);
        if (stores_row<kHeadStageRows>(lane) && r < nr) {
            const float logit = (float) total;
            a.logits[q0 + r] = logit;
            const unsigned long long c = candidate_key(logit, (uint32_t) (q0 + r));
            best = c > best ? c : best;
        }
    }
    best = fold_wave_max(best);
    if (lane == 0)
        sh.best[cw] = best;
    int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(&sh.bestArrivals, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP)
               == kComputeWaves - 1;
    if (!__builtin_amdgcn_readfirstlane(last))
        return true;
    unsigned long long c = sh.best[0];
#pragma unroll
    for (int k = 1; k < kComputeWaves; ++k)
        c = sh.best[k] > c ? sh.best[k] : c;
    const uint32_t tag = word_tag(epoch, 0);
    if (lane == 0) {
        ll_put(a.cand_ll + 2 * p.g, (uint32_t) c, tag);
        ll_put(a.cand_ll + 2 * p.g + 1, (uint32_t) (c >> 32), tag);
    }
    if (p.g != 0)
        return true;
    // workgroup 0: every workgroup's candidate, the id, the position, the epoch
    unsigned long long winner = 0;
    for (int k0 = 0; k0 < p.P; k0 += 4 * 64) {
        int word[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            word[j] = 2 * min(k0 + lane + 64 * j, p.P - 1);
        uint32_t lo[4], hi[4];
        if (!get_pairs<4>(a.cand_ll, word, 2 * p.P, tag, a.error, lo, hi))
            return false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const unsigned long long v = ((unsigned long long) hi[j] << 32) | lo[j];
            winner = v > winner ? v : winner; // repeats of the last candidate change nothing
        }
    }
    winner = fold_wave_max(winner);
    if (lane == 0) {
        const uint32_t token = winner == 0 ? 0u : 0xFFFFFFFFu - (uint32_t) (winner & 0xFFFFFFFFull);
        if (a.sample)
            a.sequence[pos + 1] = token;
        *a.position = pos + 1;
        uint32_t next = (epoch + 1) & 0xFFFFFFu;
        *a.epoch = next == 0 ? 1u : next;
    }
    return true;
}

template <int C>
__device__ __forceinline__ void compute_program(const PersistArgs &a, const Plan &p, Shared &sh, int cw)
{
    const uint32_t epoch = *a.epoch;
    const int pos = *a.position;
    const AttnPlan plan = attn_plan(pos + 1);
    const int tasks = attn_tasks(plan.splits, a.heads);
    const int merges = a.heads * (a.head_dim / kBlock);
    Ring ring{sh, cw};
    int bar = 0;
    for (int l = 0; l < a.layers; ++l) {
        const int stageBase = l * p.perLayer;
        if (!phase_qkv(a, p, sh, cw, l, pos, epoch, bar))
            return;
        for (int u = p.g + p.P * cw; u < tasks; u += p.P * kComputeWaves) {
            const int sp = (u % 8) + 8 * (u / (8 * a.heads));
            const int h = (u / 8) % a.heads;
            if (sp < plan.splits && !attention_task<C>(a, l, pos, sp, h, plan, epoch))
                return;
        }
        for (int u = p.g + p.P * cw; u < merges; u += p.P * kComputeWaves)
            if (!merge_task(a, l, u / (a.head_dim / kBlock), u % (a.head_dim / kBlock), plan, epoch))
                return;
        if (!phase_o(a, p, sh, cw, l, epoch))
            return;
        if (!phase_gateup(a, p, sh, ring, cw, l, stageBase, epoch, bar))
            return;
        if (!phase_down(a, p, sh, ring, cw, l, stageBase, epoch, bar))
            return;
    }
    phase_head(a, p, sh, ring, cw, pos, epoch, bar);
}

template <int C>
__global__ __launch_bounds__(kPersistThreads, 1) void persist_step_kernel(PersistArgs a)
{
    Shared &sh = g_sh;
    if (threadIdx.x < kSlots) {
        sh.ready[threadIdx.x] = 0;
        sh.consumed[threadIdx.x] = 0;
    }
    if (threadIdx.x < kMaxWgBlocks)
        sh.blockArrivals[threadIdx.x] = 0;
    if (threadIdx.x == 0) {
        sh.bar = 0;
        sh.bestArrivals = 0;
    }
    __syncthreads();
    const Plan p = make_plan(a, blockIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: a scalar register
    if (wave >= kComputeWaves)
        prefetch_program(a, p, sh, wave - kComputeWaves);
    else
        compute_program<C>(a, p, sh, wave);
}

int host_ceil_div(int a, int b)
{
    return (a + b - 1) / b;
}

} // namespace

PersistWords persist_words(int width, int heads, int kv_heads, int head_dim, int intermediate, int grid)
{
    const int64_t qWidth = (int64_t) heads * head_dim, kvWidth = (int64_t) kv_heads * head_dim;
    const auto q8Words = [](int64_t n) { return n / 4 + n / kBlock; };
    PersistWords w;
    w.hid = width;
    w.q = qWidth;
    w.kv = 2 * kvWidth;
    w.part = (int64_t) kPersistMaxSplits * qWidth * 2;
    w.ml = (int64_t) kPersistMaxSplits * heads * 4;
    w.attn = q8Words(qWidth);
    w.act = q8Words(intermediate);
    w.cand = 2 * (int64_t) grid;
    return w;
}

bool persist_decode_supported(int layers, int width, int heads, int kv_heads, int head_dim,
                              int intermediate, int vocab, int max_positions, int grid)
{
    if (grid < 1 || layers < 1 || layers > kPersistMaxLayers || heads < 1 || kv_heads < 1
        || heads % kv_heads != 0 || vocab < 1)
        return false;
    // whole-row byte regions of a stage are multiples of 1024 bytes (eight rows)
    if (width % 128 != 0 || width > kMaxWidth || intermediate % 64 != 0 || intermediate > kMaxInner)
        return false;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return false;
    const int qWidth = heads * head_dim;
    if (qWidth > kMaxWidth)
        return false;
    const int pairs = (heads + 2 * kv_heads) * (head_dim / 2);
    if (host_ceil_div(pairs, kComputeWaves * grid) > kMaxPairsPerWave)
        return false;
    if (host_ceil_div(width, grid) > kMaxWgRows || host_ceil_div(width, grid) > 2 * kComputeWaves)
        return false;
    if (host_ceil_div(intermediate / kBlock, grid) > kMaxWgBlocks)
        return false;
    // attention: at most kPersistMaxSplits splits of at most kMaxSplitKeys keys
    if (max_positions < 1 || max_positions > kPersistMaxSplits * kMaxSplitKeys)
        return false;
    return true;
}

int persist_grid(int device)
{
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return 0;
    int perUnit = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&perUnit, persist_step_kernel<4>, kPersistThreads, 0)
            != hipSuccess
        || perUnit < 1)
        return 0;
    return prop.multiProcessorCount;
}

hipError_t launch_persist_step(const PersistArgs &a, hipStream_t stream)
{
    if (!persist_decode_supported(a.layers, a.width, a.heads, a.kv_heads, a.head_dim, a.intermediate,
                                  a.vocab, a.max_positions, a.grid))
        return hipErrorInvalidValue;
    const int C = a.head_dim / 64;
    if (C == 4)
        hipLaunchKernelGGL(persist_step_kernel<4>, dim3(a.grid), dim3(kPersistThreads), 0, stream, a);
    else if (C == 2)
        hipLaunchKernelGGL(persist_step_kernel<2>, dim3(a.grid), dim3(kPersistThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(persist_step_kernel<1>, dim3(a.grid), dim3(kPersistThreads), 0, stream, a);
    return hipGetLastError();
}

} // namespace gq8
