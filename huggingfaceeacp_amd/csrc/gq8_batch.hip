// gq8_batch.hip -- the lockstep step of up to 16 independent sequences over
// one weight set: the product of the sequences' activation rows on int8 MFMA
// and the step's epilogue.
//
// The reference decodes one sequence per HF::Decoder (Decoder.h:69-319; its
// products are Linear.h:284-298 over Int8Blocks rows); a lockstep batch is S
// such decoders sharing the weights.  Each sequence's row goes through the
// same arithmetic as a one-sequence step: every block's integer dot is exact,
// is scaled by the product of the two fp16 scales (exact in fp32: 11 x 11
// significant bits) and accumulated in double.  Only the order of the double
// sums differs from the one-row kernels, which leaves the fp32 outputs
// identical but for values within an ulp of a rounding boundary.
//
// q8_rows_kernel: one v_mfma_i32_16x16x32_i8 per block covers 16 sequences x
// 16 weight rows.  Lane l supplies 8 bytes of sequence (l % 16)'s block and 8
// bytes of weight row (l % 16)'s block, both at byte 8 (l / 16) of the block;
// the result D[m][n] lands in lane 16 (m / 4) + n, element m % 4.  A
// workgroup stages its range of the activation blocks in LDS in that fragment
// order (and their scales as fp32), so each wave streams only weight rows
// from HBM, two chunks of 8 blocks in flight.  Products with too few tiles to
// fill the chip split the blocks over several workgroups: each stores its
// double tile, and the last of a column's workgroups (a ticket each) adds
// them in split order.
//
// attention_rows_kernel: one workgroup per (sequence, key split) scores all
// the query heads against one read of the split's keys (the single KV head of
// multi-query attention), so every key and value row is read once a layer.
// It also takes the step's RoPE and cache append: each workgroup rotates the
// sequence's query row itself, and the workgroup whose split holds the new
// position rotates the new key, appends it (and the value) to the cache and
// uses it for that position.  A second launch merges each row's splits
// (MultiQueryAttention.h:43-49) and quantizes the row for o_proj.
#include "gq8_device.hpp"
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"

#include <algorithm>

namespace gq8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kRowsThreads = 256;
constexpr int kRowsWaves = kRowsThreads / 64;
constexpr int kRowsTile = 16;         // outputs a tile (a wave's MFMA columns)
constexpr int kChunkBlocks = 8;       // blocks a wave's weight loads cover at once
constexpr int kRowsMaxRange = 128;    // blocks of the activation rows a workgroup stages
constexpr int kRowsManyTiles = 1024;  // products this wide give each wave whole rows
constexpr int kRowsPrefetch = 2;      // weight chunks in flight a wave
constexpr int kMergeBatch = 8;
constexpr int kRowsBestSlots = 32;   // a row's greedy-pick slots (atomicMax targets)
constexpr int kRowsBestStride = 16;  // 128 bytes between slots        // split partials a merge requests at once
constexpr int kRowsStreamGroups = 512; // workgroups of a streamed product (two a compute unit)
constexpr int kRowsStreamAhead = 8;    // weight chunks in flight a wave of a streamed product

// A workgroup stages `range` blocks of the activation rows in LDS and its
// waves stream weight rows against them.  Wide products (tiles >= 1024: gate
// | up, the lm_head) give a workgroup four tiles and each wave a tile's whole
// rows (WPT 1).  Narrow ones give a tile's consecutive quarters of the blocks
// to four waves (WPT 4) when those hold every chunk in flight at once (q|k|v,
// o: one workgroup a tile, loading its activation blocks directly); longer
// rows (down) split their blocks over `splits` workgroups until the chip has
// about 512, two tiles a workgroup and two waves a tile (WPT 2).
struct RowsPlan {
    int wpt;    // waves a tile: 1, 2 or 4
    int per;    // blocks a wave takes
    int splits; // workgroups over one tile's blocks
    int range() const { return wpt * per; }
};

RowsPlan rows_plan(int inner, int outputs)
{
    const int nb = inner / kBlock;
    const int tiles = (outputs + kRowsTile - 1) / kRowsTile;
    if (tiles >= kRowsManyTiles) {
        const int per = std::min(nb, kRowsMaxRange);
        return {1, per, (nb + per - 1) / per};
    }
    int per = (nb + kRowsWaves - 1) / kRowsWaves;
    if (per > kChunkBlocks)
        per = (per + kChunkBlocks - 1) / kChunkBlocks * kChunkBlocks;
    // rows short enough that a tile's four waves hold all of its weight
    // chunks in flight at once take no split: one round trip, no merge
    if (per <= kRowsPrefetch * kChunkBlocks)
        return {kRowsWaves, per, 1};
    while (kRowsWaves * per > kRowsMaxRange)
        per /= 2;
    int splits = (nb + kRowsWaves * per - 1) / (kRowsWaves * per);
    while (tiles * splits < 512 && per >= 2 * kChunkBlocks && per % (2 * kChunkBlocks) == 0) {
        per /= 2;
        splits = (nb + kRowsWaves * per - 1) / (kRowsWaves * per);
    }
    if (splits > 1 && tiles % 2 == 0) {
        // split over workgroups: two tiles a workgroup, two waves a tile, so
        // each staged block serves two tiles (the staging, not the weights,
        // had bound these launches)
        const int pairs = 2 * per;
        return {2, per, (nb + pairs - 1) / pairs};
    }
    return {kRowsWaves, per, splits};
}

size_t rows_lds_bytes(const RowsPlan &p)
{
    // fragments [block][lane] 8 bytes and scales [block][row] fp32; the
    // tiles' partial sums later reuse the fragments' space
    const size_t staged = (size_t) p.range() * 64 * 8 + (size_t) p.range() * kBatchRows * 4;
    return std::max(staged, (size_t) kRowsWaves * kBatchRows * (kRowsTile + 1) * 8);
}

struct RowsArgs {
    const uint8_t *x8;
    int x_rows, rows;
    const uint8_t *w8;
    const uint8_t *w8t; // non-null: w8 in fragment order (tile_weights_kernel), read instead
    int inner, outputs, per;
    float *y;
    int y_stride, residual;
    double *partials; // [splits][kBatchRows][outputs]
    int *tickets;     // one a workgroup column
    uint8_t *geglu8;  // non-null: outputs are gate | up rows; GeGLU's Q8 rows land here
    int split_major;  // grid (splits, columns) instead of (columns, splits)
    unsigned long long *best; // streamed only, non-null: each row's greedy pick (see below)
};

__device__ inline void store_agent_d(double *p, double v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline double load_agent_d(const double *p)
{
    return __hip_atomic_load(const_cast<double *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline float half_of(uint32_t word, int upper)
{
    return half_value((uint16_t) (upper ? word >> 16 : word & 0xFFFFu));
}

// One chunk of a wave's weight rows: 8 blocks' bytes at this lane's 8-byte
// slice, and their fp16 scales.
struct WeightChunk {
    long w[kChunkBlocks];
    uint32_t s[kChunkBlocks / 2];
};

// A wave's weight stream: this lane's slice of block 0 of the wave's tile
// (rows 16 tile .. 16 tile + 15; lane l takes row l % 16 at byte 8 (l / 16)
// of a block) and the tile's scales.  Tiled: the fragment-ordered copy, where
// block b of a tile is 512 contiguous bytes (lane l's 8 at 8 l) and chunk c's
// scales 256 (row r's 8 at 16 r); the row-major layout puts a tile's block
// at 16 places 2 KB and more apart, which streams about a third slower.
template <bool Tiled>
struct WeightRows {
    const uint8_t *bytes;
    const uint16_t *scales;
    __device__ WeightRows(const RowsArgs &a, int tile, int lane)
    {
        const int nb = a.inner / kBlock, tiles = (a.outputs + kRowsTile - 1) / kRowsTile;
        if constexpr (Tiled) {
            const int tt = min(tile, tiles - 1); // clamped into range; never stored
            bytes = a.w8t + (int64_t) tt * nb * 512 + lane * 8;
            scales = reinterpret_cast<const uint16_t *>(a.w8t + (int64_t) tiles * kRowsTile * a.inner)
                     + (int64_t) tt * nb * kRowsTile + (lane & 15) * kChunkBlocks;
        } else {
            const int n = min(tile * kRowsTile + (lane & 15), a.outputs - 1);
            bytes = a.w8 + (int64_t) n * a.inner + (lane >> 4) * 8;
            scales = reinterpret_cast<const uint16_t *>(a.w8 + (int64_t) a.outputs * a.inner)
                     + (int64_t) n * nb;
        }
    }
};

// V: whole chunks (the block count and every range a multiple of 8), the
// scales one 16-byte load; else (row-major only) blocks past `end` are
// loaded clamped.
template <bool V, bool Tiled = false>
__device__ inline void load_weight_chunk(WeightChunk &c, const WeightRows<Tiled> &ws, int c0, int end)
{
    static_assert(V || !Tiled, "the fragment-ordered copy is read in whole chunks");
    const uint8_t *wRow = ws.bytes;
    const uint16_t *wScale = ws.scales;
#pragma unroll
    for (int k = 0; k < kChunkBlocks; ++k) {
        const int b = V ? c0 + k : min(c0 + k, end - 1);
        c.w[k] = *reinterpret_cast<const long *>(wRow + (int64_t) b * (Tiled ? 512 : kBlock));
    }
    if constexpr (V) {
        const uint4 v = *reinterpret_cast<const uint4 *>(wScale + (Tiled ? (c0 >> 3) * 128 : c0));
        c.s[0] = v.x; c.s[1] = v.y; c.s[2] = v.z; c.s[3] = v.w;
    } else {
#pragma unroll
        for (int k = 0; k < kChunkBlocks; k += 2) {
            const uint32_t lo = wScale[min(c0 + k, end - 1)];
            const uint32_t hi = wScale[min(c0 + k + 1, end - 1)];
            c.s[k / 2] = lo | (hi << 16);
        }
    }
}

// One chunk of the activation rows for the direct path (no staging): 8
// blocks of sequence (lane % 16)'s row at this lane's 8-byte slice (the MFMA
// A fragment), and the fp16 scales of this lane's four accumulator rows
// 4 (lane / 16) + r over the same 8 blocks.
struct ActChunk {
    long x[kChunkBlocks];
    uint32_t s[4][kChunkBlocks / 2];
};

__device__ inline void load_act_chunk(ActChunk &c, const uint8_t *xRow, const uint16_t *const (&xs)[4],
                                      int c0)
{
#pragma unroll
    for (int k = 0; k < kChunkBlocks; ++k)
        c.x[k] = *reinterpret_cast<const long *>(xRow + (int64_t) (c0 + k) * kBlock);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint4 v = *reinterpret_cast<const uint4 *>(xs[r] + c0);
        c.s[r][0] = v.x; c.s[r][1] = v.y; c.s[r][2] = v.z; c.s[r][3] = v.w;
    }
}

// The weight chunk against the activation chunk, in chunk_products'
// arithmetic (its staged scales are these, converted to fp32 the same way).
__device__ inline void chunk_products_direct(const WeightChunk &c, const ActChunk &x, double (&acc)[4])
{
#pragma unroll
    for (int k = 0; k < kChunkBlocks; ++k) {
        const float sw = half_of(c.s[k / 2], k & 1);
        const v4i zero = {0, 0, 0, 0};
        const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(x.x[k], c.w[k], zero, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[r] = fma((double) d[r], (double) (sw * half_of(x.s[r][k / 2], k & 1)), acc[r]);
        asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The chunk against the staged activation blocks: one MFMA a block, then
// acc[r] (sequence 4 (lane / 16) + r, output lane % 16) += dot * (sw * sx)
// (the scale product exact in fp32, the product exact in double).
template <bool V>
__device__ inline void chunk_products(const WeightChunk &c, const long *sX, const float *sSx,
                                      int rb, int c0, int end, int lane, double (&acc)[4])
{
    const int grp = lane >> 4;
#pragma unroll
    for (int k = 0; k < kChunkBlocks; ++k) {
        const int kb = V ? rb + k : min(rb + k, rb + (end - 1 - c0));
        const long xa = sX[kb * 64 + lane];
        const float4 sx = *reinterpret_cast<const float4 *>(sSx + kb * kBatchRows + 4 * grp);
        const float sw = (V || c0 + k < end) ? half_of(c.s[k / 2], k & 1) : 0.f;
        const v4i zero = {0, 0, 0, 0};
        const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, c.w[k], zero, 0, 0, 0);
        acc[0] = fma((double) d[0], (double) (sw * sx.x), acc[0]);
        acc[1] = fma((double) d[1], (double) (sw * sx.y), acc[1]);
        acc[2] = fma((double) d[2], (double) (sw * sx.z), acc[2]);
        acc[3] = fma((double) d[3], (double) (sw * sx.w), acc[3]);
        // one block at a time: the results of hoisted products would hold
        // accumulation registers that cost occupancy (the sums are pinned
        // here, so they cannot sink to the end of a tile either)
        asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Blocks [r0, rEnd) (at most kMaxRange) of the activation rows, staged in
// LDS in MFMA fragment order (lane l of block b: sequence l % 16, bytes
// 8 (l / 16) .. + 8) with their scales as fp32.  stage_load issues every
// load (clamped into range) and stage_write makes the LDS writes (no
// barrier).  A workgroup issues its first weight loads between the two: the
// staging loads are ahead of them in the memory queues, and the weights are
// in flight while the staged rows arrive and are written.
template <int kMaxRange>
struct StagePieces {
    static constexpr int kPieces = kMaxRange * kBatchRows * 2 / kRowsThreads; // 16-byte pieces
    static constexpr int kScales = (kMaxRange * kBatchRows + kRowsThreads - 1) / kRowsThreads;
    uint4 piece[kPieces];
    uint16_t scaleBits[kScales];
};

template <int kMaxRange>
__device__ inline void stage_load(const RowsArgs &a, int r0, int rEnd, StagePieces<kMaxRange> &sp, int t)
{
    using S = StagePieces<kMaxRange>;
    const int nb = a.inner / kBlock;
    const uint16_t *xScales = reinterpret_cast<const uint16_t *>(a.x8 + (int64_t) a.x_rows * a.inner);
    const int pieces = (rEnd - r0) * kBatchRows * 2, scales = (rEnd - r0) * kBatchRows;
#pragma unroll
    for (int i = 0; i < S::kPieces; ++i) {
        const int p = min(t + i * kRowsThreads, pieces - 1);
        const int rb = p >> 5, m = (p >> 1) & 15, h = p & 1;
        sp.piece[i] = *reinterpret_cast<const uint4 *>(a.x8 + (int64_t) min(m, a.rows - 1) * a.inner
                                                       + (int64_t) (r0 + rb) * kBlock + h * 16);
    }
#pragma unroll
    for (int i = 0; i < S::kScales; ++i) {
        const int e = min(t + i * kRowsThreads, scales - 1);
        sp.scaleBits[i] = xScales[(int64_t) min(e & 15, a.rows - 1) * nb + r0 + (e >> 4)];
    }
}

template <int kMaxRange>
__device__ inline void stage_write(int r0, int rEnd, const StagePieces<kMaxRange> &sp, long *sX,
                                   float *sSx, int t)
{
    using S = StagePieces<kMaxRange>;
    const int pieces = (rEnd - r0) * kBatchRows * 2, scales = (rEnd - r0) * kBatchRows;
#pragma unroll
    for (int i = 0; i < S::kPieces; ++i) {
        const int p = t + i * kRowsThreads;
        if (p < pieces) {
            const int rb = p >> 5, m = (p >> 1) & 15, h = p & 1;
            uint2 *dst = reinterpret_cast<uint2 *>(sX) + rb * 64 + m;
            dst[(2 * h) * 16] = make_uint2(sp.piece[i].x, sp.piece[i].y);
            dst[(2 * h + 1) * 16] = make_uint2(sp.piece[i].z, sp.piece[i].w);
        }
    }
#pragma unroll
    for (int i = 0; i < S::kScales; ++i) {
        const int e = t + i * kRowsThreads;
        if (e < scales)
            sSx[e] = half_value(sp.scaleBits[i]);
    }
}

// NC > 0: every wave takes exactly NC whole chunks (the loop unrolled, so
// each chunk's wait counts only the loads before it); NC == 0: any range.
// Direct (WPT 4, whole chunks): no staging; each wave loads its activation
// blocks next to its weight chunks (L2 hits: a quarter of a tile's blocks is
// read by that tile's wave alone, so staging would buy no reuse).
template <int WPT, int NC, bool Direct = false, bool Tiled = false>
__global__ __launch_bounds__(kRowsThreads) void q8_rows_kernel(RowsArgs a)
{
    constexpr bool V = NC > 0;
    static_assert(!Direct || (WPT == kRowsWaves && NC > 0), "direct: split tiles, whole chunks");
    static_assert(!Tiled || V, "the fragment-ordered copy is read in whole chunks");
    constexpr int kTiles = kRowsWaves / WPT; // tiles a workgroup
    extern __shared__ __attribute__((aligned(16))) unsigned char rowsLds[];
    const int range = WPT * a.per;
    long *sX = reinterpret_cast<long *>(rowsLds);
    float *sSx = reinterpret_cast<float *>(rowsLds + (size_t) range * 64 * 8);
    double *sPart = reinterpret_cast<double *>(rowsLds); // over the fragments, once they are read
    __shared__ int sLast;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nb = a.inner / kBlock;
    const int col = lane & 15;
    // GeGLU's pairing (four tiles a workgroup): waves 0 and 1 take gate
    // tiles 2 x, 2 x + 1, waves 2 and 3 the up tiles of the same outputs
    const int upTiles = a.outputs / (2 * kRowsTile);
    // split products launch split-major (blockIdx.x the split), so each XCD
    // (workgroups go to the eight in turn) takes one block range and its L2
    // holds only that range of the activation rows
    const int colIdx = a.split_major ? (int) blockIdx.y : (int) blockIdx.x;
    const int splitIdx = a.split_major ? (int) blockIdx.x : (int) blockIdx.y;
    const int nSplits = a.split_major ? (int) gridDim.x : (int) gridDim.y;
    const int tile = a.geglu8 ? (wave >> 1) * upTiles + 2 * colIdx + (wave & 1)
                              : colIdx * kTiles + wave / WPT;
    const int part = wave % WPT;
    const int r0 = splitIdx * range;             // the workgroup's first block
    const int rEnd = min(r0 + range, nb);
    const int b0 = r0 + part * a.per;              // this wave's blocks
    const int b1 = min(b0 + a.per, nb);

    // this wave's weight rows (clamped into range; never stored)
    const WeightRows<Tiled> ws(a, tile, lane);
    const uint16_t *xScales = reinterpret_cast<const uint16_t *>(a.x8 + (int64_t) a.x_rows * a.inner);
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    if constexpr (Direct) {
        const int grp = lane >> 4;
        const uint8_t *xRow = a.x8 + (int64_t) min(col, a.rows - 1) * a.inner + grp * 8;
        const uint16_t *const xs[4] = {xScales + (int64_t) min(4 * grp + 0, a.rows - 1) * nb,
                                       xScales + (int64_t) min(4 * grp + 1, a.rows - 1) * nb,
                                       xScales + (int64_t) min(4 * grp + 2, a.rows - 1) * nb,
                                       xScales + (int64_t) min(4 * grp + 3, a.rows - 1) * nb};
        constexpr int P = NC < kRowsPrefetch ? NC : kRowsPrefetch;
        WeightChunk wb[P];
        ActChunk xb[P];
        if (b0 < b1) { // the last split's waves may have no blocks
#pragma unroll
            for (int i = 0; i < P; ++i) {
                load_weight_chunk<true, Tiled>(wb[i], ws, b0 + i * kChunkBlocks, b1);
                load_act_chunk(xb[i], xRow, xs, b0 + i * kChunkBlocks);
            }
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                chunk_products_direct(wb[i % P], xb[i % P], acc);
                __builtin_amdgcn_sched_barrier(0);
                asm volatile("" ::: "memory");
                if (i + P < NC) {
                    load_weight_chunk<true, Tiled>(wb[i % P], ws, b0 + (i + P) * kChunkBlocks, b1);
                    load_act_chunk(xb[i % P], xRow, xs, b0 + (i + P) * kChunkBlocks);
                }
            }
        }
    } else {
    // with whole chunks the range is WPT NC chunks
    // the staging loads, then up to kRowsPrefetch chunks of weights in
    // flight a wave: behind the staging loads, since once the weight stream
    // fills the memory queues a wave's vector memory instructions issue only
    // as fast as loads retire; then the LDS writes
    constexpr int kRange = V ? WPT * NC * kChunkBlocks : kRowsMaxRange;
    StagePieces<kRange> staged;
    stage_load<kRange>(a, r0, rEnd, staged, t);
    constexpr int P = V ? (NC < kRowsPrefetch ? NC : kRowsPrefetch) : 1;
    WeightChunk buf[P];
    if (b0 < b1) {
#pragma unroll
        for (int i = 0; i < P; ++i)
            load_weight_chunk<V, Tiled>(buf[i], ws, V ? b0 + i * kChunkBlocks : b0, b1);
    }
    __builtin_amdgcn_sched_barrier(0);
    stage_write<kRange>(r0, rEnd, staged, sX, sSx, t);
    __syncthreads();

    // two weight buffers: the next chunk's loads are in flight while this
    // one computes
    if constexpr (V) {
        if (b0 < b1) { // the last split's waves may have no blocks
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                // memory clobbers keep each chunk's loads where they are
                // issued (hoisting them all would cost occupancy)
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                chunk_products<true>(buf[i % P], sX, sSx, b0 - r0 + i * kChunkBlocks,
                                     b0 + i * kChunkBlocks, b1, lane, acc);
                __builtin_amdgcn_sched_barrier(0);
                asm volatile("" ::: "memory");
                if (i + P < NC) // the buffer just consumed takes the chunk P ahead
                    load_weight_chunk<true, Tiled>(buf[i % P], ws, b0 + (i + P) * kChunkBlocks, b1);
            }
        }
    } else {
        for (int c0 = b0; c0 < b1; c0 += kChunkBlocks) {
            if (c0 > b0)
                load_weight_chunk<false>(buf[0], WeightRows<false>(a, tile, lane), c0, b1);
            chunk_products<false>(buf[0], sX, sSx, c0 - r0, c0, b1, lane, acc);
        }
    }
    } // staged

    // a tile's sum over its waves (in block order), one (sequence, output)
    // cell a thread; tile k of the workgroup lands in sPart[k]
    const int grp = lane >> 4;
    __syncthreads(); // every wave has read its fragments
    double *mine = sPart + (size_t) wave * kBatchRows * (kRowsTile + 1);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        mine[(4 * grp + r) * (kRowsTile + 1) + col] = acc[r];
    __syncthreads();
    if (WPT == 1 && a.geglu8) {
        // the products' fp32 outputs, GeGLU, and the 32-element block's Q8
        // (a row's 32 outputs in 32 consecutive lanes)
        const int F = a.outputs / 2;
        uint16_t *scales = reinterpret_cast<uint16_t *>(a.geglu8 + (int64_t) a.x_rows * F);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int cell = t + i * kRowsThreads;
            const int m = cell >> 5, jj = cell & 31;
            const double *gate = sPart + (size_t) (jj >> 4) * kBatchRows * (kRowsTile + 1);
            const double *up = sPart + (size_t) (2 + (jj >> 4)) * kBatchRows * (kRowsTile + 1);
            const float v = geglu((float) gate[m * (kRowsTile + 1) + (jj & 15)],
                                  (float) up[m * (kRowsTile + 1) + (jj & 15)]);
            const float amax = max_lanes<16>(fabsf(v));
            const uint16_t bits = scale_bits_from_amax(amax);
            const float sc = half_value(bits);
            const int j = colIdx * 2 * kRowsTile + jj;
            if (m < a.rows) {
                a.geglu8[(int64_t) m * F + j] = (uint8_t) (int8_t) quantize_in_block(v, bits, sc, quantize_hint(sc));
                if (jj == 0)
                    scales[(int64_t) m * (F / kBlock) + j / kBlock] = bits;
            }
        }
        return;
    }
    for (int cell = t; cell < kTiles * kBatchRows * kRowsTile; cell += kRowsThreads) {
        const int k = cell >> 8, m = (cell >> 4) & 15, c = cell & 15;
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < WPT; ++w)
            sum += sPart[((size_t) (k * WPT + w) * kBatchRows + m) * (kRowsTile + 1) + c];
        const int on = (colIdx * kTiles + k) * kRowsTile + c;
        if (m >= a.rows || on >= a.outputs)
            continue;
        if (nSplits == 1) {
            float *dst = a.y + (int64_t) m * a.y_stride + on;
            const double old = a.residual ? (double) *dst : 0.0;
            *dst = (float) (sum + old);
        } else {
            // the blocks are split over nSplits workgroups: agent-scope
            // stores (coherent across the L2s), completed before the ticket
            store_agent_d(a.partials + ((int64_t) splitIdx * kBatchRows + m) * a.outputs + on, sum);
        }
    }
    if (nSplits == 1)
        return;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0)
        sLast = __hip_atomic_fetch_add(a.tickets + colIdx, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == nSplits - 1;
    __syncthreads();
    if (!sLast)
        return;
    // the splits' partials of this thread's cells, kMergeBatch splits
    // requested at once (cells and splits past the ends read a clamped, live
    // slot), added in split order
    constexpr int kCells = kTiles * kBatchRows * kRowsTile / kRowsThreads;
    const int splits = nSplits;
    double total[kCells];
#pragma unroll
    for (int i = 0; i < kCells; ++i)
        total[i] = 0.0;
    for (int s0 = 0; s0 < splits; s0 += kMergeBatch) {
        double part[kCells][kMergeBatch];
#pragma unroll
        for (int i = 0; i < kCells; ++i) {
            const int cell = t + i * kRowsThreads;
            const int k = cell >> 8, m = min((cell >> 4) & 15, a.rows - 1), c = cell & 15;
            const int on = min((colIdx * kTiles + k) * kRowsTile + c, a.outputs - 1);
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j)
                part[i][j] = load_agent_d(a.partials + ((int64_t) min(s0 + j, splits - 1) * kBatchRows + m)
                                                           * a.outputs + on);
        }
#pragma unroll
        for (int i = 0; i < kCells; ++i)
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j)
                if (s0 + j < splits)
                    total[i] += part[i][j];
    }
#pragma unroll
    for (int i = 0; i < kCells; ++i) {
        const int cell = t + i * kRowsThreads;
        const int k = cell >> 8, m = (cell >> 4) & 15, c = cell & 15;
        const int on = (colIdx * kTiles + k) * kRowsTile + c;
        if (m >= a.rows || on >= a.outputs)
            continue;
        float *dst = a.y + (int64_t) m * a.y_stride + on;
        const double old = a.residual ? (double) *dst : 0.0;
        *dst = (float) (total[i] + old);
    }
    if (t == 0) // ready for the next launch
        __hip_atomic_store(a.tickets + colIdx, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wide products with no GeGLU (the lm_head): a workgroup stages the whole
// activation rows (nb = NC chunks) once, starts on group blockIdx.x of four
// tiles (one a wave), then takes groups from a shared counter until none is
// left, so a workgroup that the memory system serves faster takes more of
// them.  Each wave's weight chunks stream across the group boundaries, P
// ahead (the next group is claimed when a group starts and published at the
// workgroup barrier P chunks before its end); a tile's 16 x 16 outputs go
// straight from its accumulators to y.  counters[0] counts the claims (group
// gridDim.x + claim), counters[1] the workgroups done; the last one done
// zeroes both for the next launch.  The arithmetic is q8_rows_kernel's.
template <int NC, bool Tiled>
__global__ __launch_bounds__(kRowsThreads) void q8_rows_stream_kernel(RowsArgs a)
{
    constexpr int nb = NC * kChunkBlocks;
    constexpr int P = NC < kRowsStreamAhead ? NC : kRowsStreamAhead;
    // the next group's chunk i + P - NC lands in buffer i % P and is read
    // from buffer (i + P - NC) % P: the same one only when P divides NC
    static_assert(NC % P == 0, "a whole number of buffer rounds a group");
    __shared__ __attribute__((aligned(16))) long sX[nb * 64];
    __shared__ __attribute__((aligned(16))) float sSx[nb * kBatchRows];
    __shared__ int sGroup[2];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int tiles = (a.outputs + kRowsTile - 1) / kRowsTile;
    const int groups = (tiles + kRowsWaves - 1) / kRowsWaves;
    int *counters = a.tickets;
    auto claim = [&]() {
        return __hip_atomic_fetch_add(counters, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    // the first group is the workgroup's own; later ones are claimed
    StagePieces<nb> staged;
    stage_load<nb>(a, 0, nb, staged, t);
    int g = blockIdx.x;
    WeightChunk buf[P];
    if (g < groups) {
        const WeightRows<Tiled> ws(a, g * kRowsWaves + wave, lane);
#pragma unroll
        for (int i = 0; i < P; ++i)
            load_weight_chunk<true, Tiled>(buf[i], ws, i * kChunkBlocks, nb);
    }
    __builtin_amdgcn_sched_barrier(0);
    stage_write<nb>(0, nb, staged, sX, sSx, t);
    __syncthreads();
    // with a.best: the largest (logit key, complemented column) of each of
    // this lane's accumulator rows 4 grp + r over the workgroup's tiles
    unsigned long long runBest[4] = {0ull, 0ull, 0ull, 0ull};
    int slot = 1;
#pragma nounroll
    while (g < groups) {
        if (t == 0) // the next group, in flight while this one streams
            sGroup[slot] = (int) gridDim.x + claim();
        const WeightRows<Tiled> ws(a, g * kRowsWaves + wave, lane);
        int next = groups;
        double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            chunk_products<true>(buf[i % P], sX, sSx, i * kChunkBlocks, i * kChunkBlocks, nb, lane, acc);
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("" ::: "memory");
            if (i + P < NC) {
                load_weight_chunk<true, Tiled>(buf[i % P], ws, (i + P) * kChunkBlocks, nb);
            } else {
                if (i + P == NC) { // the next group's index, published
                    __syncthreads();
                    next = sGroup[slot];
                }
                if (next < groups)
                    load_weight_chunk<true, Tiled>(buf[i % P],
                                                   WeightRows<Tiled>(a, next * kRowsWaves + wave, lane),
                                                   (i + P - NC) * kChunkBlocks, nb);
            }
        }
        const int on = (g * kRowsWaves + wave) * kRowsTile + col;
        if (on < a.outputs) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * grp + r;
                if (m < a.rows)
                    a.y[(int64_t) m * a.y_stride + on] = (float) acc[r];
            }
        }
        if (a.best) { // uniform
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                unsigned long long key = on < a.outputs ? candidate_key((float) acc[r], (uint32_t) on) : 0ull;
                key = max_lanes<8>(key); // the tile's 16 columns (lanes of one row of 16)
                runBest[r] = key > runBest[r] ? key : runBest[r];
            }
        }
        g = next;
        slot ^= 1;
    }
    if (a.best) { // the workgroup's best of each row into one of the row's slots
        __shared__ unsigned long long sRowBest[kRowsWaves][kBatchRows];
        if (col == 0)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                sRowBest[wave][4 * grp + r] = runBest[r];
        __syncthreads();
        if (t < a.rows) {
            unsigned long long c = sRowBest[0][t];
#pragma unroll
            for (int w = 1; w < kRowsWaves; ++w)
                c = sRowBest[w][t] > c ? sRowBest[w][t] : c;
            if (c != 0)
                atomicMax(a.best + ((int64_t) t * kRowsBestSlots + blockIdx.x % kRowsBestSlots)
                                       * kRowsBestStride, c);
        }
    }
    if (t == 0
        && __hip_atomic_fetch_add(counters + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
               == (int) gridDim.x - 1) {
        // every workgroup has claimed its last group: ready for the next launch
        __hip_atomic_store(counters, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(counters + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The fragment-ordered copy of an Int8Blocks weight (WeightRows<true>'s
// layout): thread i of the bytes writes lane (i % 64)'s 8 bytes of block
// (i / 64) % nb of tile i / (64 nb); rows past `outputs` are zero.  Then the
// scales, 8 (one chunk of one row) a thread.
__global__ __launch_bounds__(kRowsThreads) void tile_weights_kernel(const uint8_t *__restrict__ w8,
                                                                   int outputs, int inner,
                                                                   uint8_t *__restrict__ out)
{
    const int nb = inner / kBlock, tiles = (outputs + kRowsTile - 1) / kRowsTile;
    const int64_t pieces = (int64_t) tiles * nb * 64, chunks = (int64_t) tiles * kRowsTile * (nb / 8);
    const uint16_t *scales = reinterpret_cast<const uint16_t *>(w8 + (int64_t) outputs * inner);
    uint16_t *scalesOut = reinterpret_cast<uint16_t *>(out + (int64_t) tiles * kRowsTile * inner);
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < pieces + chunks;
         i += (int64_t) gridDim.x * blockDim.x) {
        if (i < pieces) {
            const int lane = (int) (i % 64), b = (int) ((i / 64) % nb);
            const int64_t tile = i / (64 * (int64_t) nb);
            const int64_t row = tile * kRowsTile + lane % 16;
            long v = 0;
            if (row < outputs)
                v = *reinterpret_cast<const long *>(w8 + row * inner + (int64_t) b * kBlock
                                                    + (lane / 16) * 8);
            reinterpret_cast<long *>(out)[i] = v;
        } else {
            const int64_t j = i - pieces; // (tile, chunk, row)
            const int r = (int) (j % kRowsTile), c = (int) ((j / kRowsTile) % (nb / 8));
            const int64_t tile = j / (kRowsTile * (int64_t) (nb / 8));
            const int64_t row = tile * kRowsTile + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row < outputs)
                v = *reinterpret_cast<const uint4 *>(scales + row * nb + c * 8);
            reinterpret_cast<uint4 *>(scalesOut)[j] = v;
        }
    }
}

// ---- attention of the lockstep rows ---------------------------------------------
constexpr int kRowsTileKeys = 80;   // keys a tile (a split): five of a lane's 16-lane row
constexpr int kRowsWaveKeys = kRowsTileKeys / kRowsWaves; // a wave's keys of the values
constexpr int kRowsHeadGroup = 4;   // query heads a workgroup

// C consecutive fp16 channels kept packed, two a register.
template <int C>
struct Halves {
    uint32_t w[(C + 1) / 2];
    __device__ float at(int c) const
    {
        return half_value((uint16_t) ((w[c / 2] >> (16 * (c & 1))) & 0xFFFFu));
    }
};

template <int C>
__device__ inline Halves<C> load_channels(const uint16_t *p)
{
    Halves<C> h;
    if constexpr (C == 4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        h.w[0] = v.x;
        h.w[1] = v.y;
    } else if constexpr (C == 2) {
        h.w[0] = *reinterpret_cast<const uint32_t *>(p);
    } else {
        h.w[0] = *p;
    }
    return h;
}

// p[j] += s' x[j], j < K, where s' is the s that lane N of the lane's
// 16-lane row holds: four accumulators an instruction group, then the rest
// one at a time
template <int N, int K>
__device__ inline void row_lane_fmac(double (&p)[K], double s, const double (&x)[K])
{
    static_assert(K >= 4 && K < 8, "four to seven keys a lane");
    fmac_row_bcast4<N, N, N, N>(reinterpret_cast<double (&)[4]>(p), s,
                                reinterpret_cast<const double (&)[4]>(x));
    if constexpr (K > 4)
        fmac_row_bcast1<N>(p[4], s, x[4]);
    if constexpr (K > 5)
        fmac_row_bcast1<N>(p[5], s, x[5]);
    if constexpr (K > 6)
        fmac_row_bcast1<N>(p[6], s, x[6]);
}

// C channels a lane (head width 64 C), H heads, G of them a workgroup
// (blockIdx.z picks the group; the groups of one key tile share the tile's
// rows through the L2), a split of per_split keys in tiles of kRowsTileKeys.
// Scores: wave w takes a quarter of the channels and its lane l keys
// t0 + l % 16 + 16 j (j < kLaneKeys) over the quarter's slice l / 16 of
// 4 C channels, every head of the group; lane c of each 16-lane row holds
// channel c of the slice's query, which the multiply-adds take by DPP
// broadcast; the sixteen slices' dots are added in LDS in channel order.
// Values: lane l takes channels C l .. C l + C - 1 and wave w keys
// t0 + kRowsWaveKeys w .. + kRowsWaveKeys - 1, every head of the group.
template <int C, int H, int G>
__global__ __launch_bounds__(kRowsThreads, 2) void attention_rows_kernel(RowsAttentionArgs a)
{
    static_assert(H % G == 0, "whole head groups");
    constexpr int hd = 64 * C, half = hd / 2, qW = H * hd;
    constexpr int hq = hd / kRowsWaves;        // channels a wave scores
    constexpr int kSlices = 4;                 // channel slices of a wave's quarter
    constexpr int kSliceCh = hq / kSlices;     // channels a lane scores (4 C)
    constexpr int kSliceWords = kSliceCh / 2;  // their fp16 pairs
    constexpr int kLaneKeys = kRowsTileKeys / 16; // keys a lane scores
    constexpr int kParts = kRowsWaves * kSlices;  // partial dots of a score
    constexpr int kAccHeads = G < 4 ? G : 4;   // heads a pass of the waves' LDS sum
    constexpr int kRopePairs = ((G + 1) * half + kRowsThreads - 1) / kRowsThreads;
    __shared__ double sQd[G][hd];
    __shared__ __attribute__((aligned(16))) uint16_t sKnew[hd], sVnew[hd];
    // the partial dots, and after the last tile the waves' value sums
    constexpr int kPartDoubles = kParts * G * kRowsTileKeys;
    constexpr int kAccDoubles = kRowsWaves * kAccHeads * hd;
    __shared__ double sShared[kPartDoubles > kAccDoubles ? kPartDoubles : kAccDoubles];
    double (*sP)[G][kRowsTileKeys] = reinterpret_cast<double (*)[G][kRowsTileKeys]>(sShared);
    double (*sAcc)[kAccHeads * hd] = reinterpret_cast<double (*)[kAccHeads * hd]>(sShared);
    __shared__ double sS[G][kRowsTileKeys];
    __shared__ double sMax[G], sSum[G], sF[G];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int seq = blockIdx.y, split = blockIdx.x, hBase = blockIdx.z * G;
    const int k0 = split * a.per_split;
    // the position first: its wait then counts only the loads before it
    const int pos = a.positions[seq];
    asm volatile("" ::: "memory");
    const int c0 = lane * C;
    const float *row = a.qkv + (int64_t) seq * a.qkv_stride;
    uint16_t *keys = a.key_cache + seq * a.cache_stride;
    uint16_t *values = a.value_cache + seq * a.cache_stride;

    // Loads that do not need the position go first: the group's query and
    // the new key pairs (local head G: global head H, right after the
    // queries), the new value, and the first tile's key and value rows (rows
    // past the position are read inside the cache and never used).  Their
    // round trip overlaps the position's.
    float lo[kRopePairs], hi[kRopePairs], cs[kRopePairs], sn[kRopePairs];
#pragma unroll
    for (int k = 0; k < kRopePairs; ++k) {
        const int idx = min(t + k * kRowsThreads, (G + 1) * half - 1);
        const int head = idx / half, i = idx % half;
        const int global = head < G ? hBase + head : H;
        lo[k] = row[global * hd + i];
        hi[k] = row[global * hd + i + half];
        // the angles of the row's position, copied for the step by its embed
        // launch: no wait on the position
        cs[k] = a.row_angles[(int64_t) seq * 2 * half + i];
        sn[k] = a.row_angles[(int64_t) (seq * 2 + 1) * half + i];
    }
    const float newValue = row[qW + hd + min(t, hd - 1)];
    // this lane's score slice: channels ch0 .. ch0 + kSliceCh - 1 of keys
    // t0 + kg + 16 j
    const int kg = lane & 15, ch0 = wave * hq + (lane >> 4) * kSliceCh;
    uint32_t kq[kLaneKeys][kSliceWords];
    Halves<C> vh[kRowsWaveKeys];
    auto load_key_slice = [&](uint32_t (&dst)[kSliceWords], const uint16_t *src) {
        if constexpr (kSliceWords % 4 == 0) {
#pragma unroll
            for (int v = 0; v < kSliceWords / 4; ++v) {
                const uint4 w = reinterpret_cast<const uint4 *>(src)[v];
                dst[4 * v] = w.x; dst[4 * v + 1] = w.y; dst[4 * v + 2] = w.z; dst[4 * v + 3] = w.w;
            }
        } else {
            const uint2 w = *reinterpret_cast<const uint2 *>(src);
            dst[0] = w.x; dst[1] = w.y;
        }
    };
    auto load_keys = [&](int t0) {
#pragma unroll
        for (int j = 0; j < kLaneKeys; ++j) {
            const int key = min(t0 + kg + 16 * j, a.max_positions - 1);
            load_key_slice(kq[j], keys + (int64_t) key * hd + ch0);
        }
    };
    auto load_values = [&](int t0) {
#pragma unroll
        for (int i = 0; i < kRowsWaveKeys; ++i) {
            const int j = min(t0 + wave * kRowsWaveKeys + i, a.max_positions - 1);
            vh[i] = load_channels<C>(values + (int64_t) j * hd + c0);
        }
    };
    load_keys(k0);
    asm volatile("" ::: "memory"); // keeps the loads above the position-dependent exit

    const int keyCount = pos + 1;
    if (k0 >= keyCount)
        return;
    const int k1 = min(k0 + a.per_split, keyCount);
    const bool holdsNew = k1 == keyCount; // this split ends at the new position

    // RoPE (rope_kv_kernel's arithmetic) of the group's query heads and, in
    // the split holding it, of the new key; the new value rounded to fp16
    {
#pragma unroll
        for (int k = 0; k < kRopePairs; ++k) {
            const int idx = t + k * kRowsThreads;
            if (idx >= (G + 1) * half)
                break;
            const int head = idx / half, i = idx % half;
            float rl, rh;
            rotate_pair(lo[k], hi[k], cs[k], sn[k], &rl, &rh);
            if (head < G) {
                sQd[head][i] = (double) rl;
                sQd[head][i + half] = (double) rh;
            } else {
                sKnew[i] = half_bits(rl);
                sKnew[i + half] = half_bits(rh);
            }
        }
        if (holdsNew && t < hd)
            sVnew[t] = half_bits(newValue);
    }
    if (t < G) {
        sMax[t] = -INFINITY;
        sSum[t] = 0.0;
    }
    __syncthreads();
    if (holdsNew && t < hd && blockIdx.z == 0) { // one group appends the new rows
        keys[(int64_t) pos * hd + t] = sKnew[t];
        values[(int64_t) pos * hd + t] = sVnew[t];
    }

    // this lane's channel of the group's queries: lane c of a 16-lane row holds
    // channel c of the row's slice, for every head of the group
    double qLane[G];
#pragma unroll
    for (int h = 0; h < G; ++h)
        qLane[h] = sQd[h][ch0 + min(kg, kSliceCh - 1)];

    double acc[G][C];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int c = 0; c < C; ++c)
            acc[h][c] = 0.0;

    for (int t0 = k0; t0 < k1; t0 += kRowsTileKeys) {
        const int nk = min(kRowsTileKeys, k1 - t0);
        if (t0 > k0) // the first tile's keys are already in
            load_keys(t0);
        if (holdsNew && t0 + nk == keyCount) { // the new position's rows from LDS
#pragma unroll
            for (int j = 0; j < kLaneKeys; ++j)
                if (t0 + kg + 16 * j == pos)
                    load_key_slice(kq[j], sKnew + ch0);
        }
        // this lane's keys against every head of the group over its slice
        double p[G][kLaneKeys];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < kLaneKeys; ++j)
                p[h][j] = 0.0;
        // channel c of the slice takes its query from lane c of the row
        unrolled<kSliceWords>([&](auto word) {
            constexpr int w = decltype(word)::value;
            double ka[kLaneKeys], kb[kLaneKeys];
#pragma unroll
            for (int j = 0; j < kLaneKeys; ++j) {
                ka[j] = (double) half_value((uint16_t) (kq[j][w] & 0xFFFFu));
                kb[j] = (double) half_value((uint16_t) (kq[j][w] >> 16));
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                row_lane_fmac<2 * w>(p[h], qLane[h], ka);
                row_lane_fmac<2 * w + 1>(p[h], qLane[h], kb);
            }
        });
        const int part = wave * kSlices + (lane >> 4); // the slice's place in channel order
#pragma unroll
        for (int j = 0; j < kLaneKeys; ++j)
#pragma unroll
            for (int h = 0; h < G; ++h)
                sP[part][h][kg + 16 * j] = p[h][j];
        // the tile's value rows: their round trip overlaps the softmax
        load_values(t0);
        __syncthreads();
        // the tile's softmax against the running maximum, a wave a head; the
        // slices' dots added in channel order
        // (keys lane and, past 64, lane + 64 of the tile)
        constexpr int kSoftKeys = (kRowsTileKeys + 63) / 64;
        for (int h = wave; h < G; h += kRowsWaves) {
            double sc[kSoftKeys];
            double laneMax = -INFINITY;
#pragma unroll
            for (int k = 0; k < kSoftKeys; ++k) {
                const int key = min(lane + 64 * k, kRowsTileKeys - 1);
                double dot = sP[0][h][key];
#pragma unroll
                for (int q = 1; q < kParts; ++q)
                    dot += sP[q][h][key];
                sc[k] = lane + 64 * k < nk ? (double) a.scale * dot : -INFINITY;
                laneMax = fmax(laneMax, sc[k]);
            }
            const double tileMax = wave_max_d(laneMax);
            const double previous = sMax[h];
            const double largest = fmax(previous, tileMax);
            double laneSum = 0.0;
#pragma unroll
            for (int k = 0; k < kSoftKeys; ++k) {
                const double w = lane + 64 * k < nk ? exp(sc[k] - largest) : 0.0;
                laneSum += w;
                if (lane + 64 * k < kRowsTileKeys)
                    sS[h][lane + 64 * k] = w;
            }
            const double total = wave_sum_d(laneSum);
            if (lane == 0) {
                const double factor = previous == -INFINITY ? 0.0 : exp(previous - largest);
                sF[h] = factor;
                sSum[h] = sSum[h] * factor + total;
                sMax[h] = largest;
            }
        }
        __syncthreads();
        if (holdsNew && t0 + nk == keyCount) { // the new position's value from LDS
            const Halves<C> vn = load_channels<C>(sVnew + c0);
#pragma unroll
            for (int i = 0; i < kRowsWaveKeys; ++i)
                if (t0 + wave * kRowsWaveKeys + i == pos)
                    vh[i] = vn;
        }
        // rescaled running sums plus this wave's keys in order
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const double f = sF[h];
#pragma unroll
            for (int c = 0; c < C; ++c)
                acc[h][c] *= f;
        }
        // (four channels a lane: lane i of each 16-lane row holds key i's
        // weights, which the multiply-adds take by DPP broadcast)
        // (keys 16 .. 19 of a wave's 20 from a second register: lane i of
        // each row holds key 16 + i)
        static_assert(kRowsWaveKeys <= 32, "two broadcast registers");
        double wLane[G], wLane2[G];
        if constexpr (C == 4)
#pragma unroll
            for (int h = 0; h < G; ++h) {
                wLane[h] = sS[h][wave * kRowsWaveKeys + min(lane & 15, kRowsWaveKeys - 1)];
                wLane2[h] = sS[h][wave * kRowsWaveKeys + min(16 + (lane & 15), kRowsWaveKeys - 1)];
            }
        // (the keys as compile-time indices: a loop with an early exit is not
        // unrolled, and vh would be indexed from scratch memory)
        const int keysHere = nk - wave * kRowsWaveKeys; // rows past the position may hold anything
        unrolled<kRowsWaveKeys>([&](auto key) {
            constexpr int i = decltype(key)::value;
            if (i >= keysHere)
                return;
            double v[C];
#pragma unroll
            for (int c = 0; c < C; ++c)
                v[c] = (double) vh[i].at(c);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                if constexpr (C == 4) {
                    if constexpr (i < 16)
                        fmac_row_bcast4<i, i, i, i>(acc[h], wLane[h], v);
                    else
                        fmac_row_bcast4<i - 16, i - 16, i - 16, i - 16>(acc[h], wLane2[h], v);
                } else {
                    const double wi = sS[h][wave * kRowsWaveKeys + i];
#pragma unroll
                    for (int c = 0; c < C; ++c)
                        acc[h][c] += wi * v[c];
                }
            }
        });
        __syncthreads(); // the next tile rewrites the scores
    }

    // the split's partial of the group's heads: the four waves' sums in wave
    // order, kAccHeads heads a pass
    const int64_t slot = (int64_t) seq * kRowsMaxSplits + split;
#pragma unroll
    for (int h0 = 0; h0 < G; h0 += kAccHeads) {
        if (h0 > 0)
            __syncthreads();
#pragma unroll
        for (int h = 0; h < kAccHeads && h0 + h < G; ++h)
#pragma unroll
            for (int c = 0; c < C; ++c)
                sAcc[wave][h * hd + c0 + c] = acc[h0 + h][c];
        __syncthreads();
        const int width = min(kAccHeads, G - h0) * hd;
        for (int o = t; o < width; o += kRowsThreads) {
            double v = sAcc[0][o];
#pragma unroll
            for (int w = 1; w < kRowsWaves; ++w)
                v += sAcc[w][o];
            a.ws_o[slot * qW + (hBase + h0) * hd + o] = v;
        }
    }
    if (t < G) {
        a.ws_ml[(slot * H + hBase + t) * 2] = sMax[t];
        a.ws_ml[(slot * H + hBase + t) * 2 + 1] = sSum[t];
    }
}

// The merge of a row's key splits, one wave a (64 channels of a head,
// sequence), one channel a lane: every split rescaled to the row maximum, in
// split order, the sum divided by the total (MultiQueryAttention.h:43-49),
// rounded to fp32 and quantized in 32-channel blocks for o_proj.  Every
// split's partial is loaded at once, and each wave computes its head's split
// factors itself, so a workgroup moves 16 KB of partials, not a head's 64 KB.
__global__ __launch_bounds__(64) void attention_merge_rows_kernel(RowsAttentionArgs a)
{
    __shared__ double sF[kRowsMaxSplits];
    __shared__ double sTotal;
    const int hd = a.head_dim, H = a.heads, qW = H * hd;
    const int quarters = hd / 64; // waves a head
    const int head = blockIdx.x / quarters, seq = blockIdx.y, t = threadIdx.x;
    const int splits = (a.positions[seq] + a.per_split) / a.per_split; // keys: position + 1
    const int64_t first = (int64_t) seq * kRowsMaxSplits;
    const int o = head * hd + (blockIdx.x % quarters) * 64 + t;
    double part[kRowsMaxSplits];
#pragma unroll
    for (int u = 0; u < kRowsMaxSplits; ++u)
        part[u] = a.ws_o[(first + min(u, splits - 1)) * qW + o];
    {
        const bool live = t < splits;
        const int sp = live ? t : 0;
        const double m = a.ws_ml[((first + sp) * H + head) * 2];
        const double sum = a.ws_ml[((first + sp) * H + head) * 2 + 1];
        double total;
        const double f = merge_factor(m, sum, live, total);
        if (live)
            sF[sp] = f;
        if (t == 0)
            sTotal = total;
    }
    __syncthreads();
    double weighted = 0.0;
#pragma unroll
    for (int u = 0; u < kRowsMaxSplits; ++u)
        if (u < splits)
            weighted += part[u] * sF[u];
    const float v = (float) (weighted / sTotal);
    const float amax = max_lanes<16>(fabsf(v)); // a 32-block is 32 consecutive lanes
    const uint16_t bits = scale_bits_from_amax(amax);
    const float sc = half_value(bits);
    a.q8[(int64_t) seq * qW + o] = (uint8_t) (int8_t) quantize_in_block(v, bits, sc, quantize_hint(sc));
    if ((t & 31) == 0)
        reinterpret_cast<uint16_t *>(a.q8 + (int64_t) a.q8_rows * qW)[(int64_t) seq * (qW / kBlock)
                                                                      + o / kBlock] = bits;
}

// Row r's greedy pick from its slots (the largest key: the largest logit,
// the lowest column among equal ones, as Sampler.cpp:60-76), stored in
// chosen[r] and in the row's slot after its position, which advances; the
// slots are cleared for the next step.  A wave a row.
__global__ __launch_bounds__(64) void batch_pick_advance_kernel(unsigned long long *best,
                                                                uint32_t *chosen, uint32_t *slots,
                                                                int64_t slot_stride, int *positions)
{
    const int r = blockIdx.x, lane = threadIdx.x;
    unsigned long long *mine = best + ((int64_t) r * kRowsBestSlots + lane) * kRowsBestStride;
    unsigned long long c = lane < kRowsBestSlots ? *mine : 0ull;
    if (lane < kRowsBestSlots)
        *mine = 0ull;
    c = max_lanes<32>(c);
    if (lane == 0) {
        const uint32_t token = c == 0 ? 0u : 0xFFFFFFFFu - (uint32_t) (c & 0xFFFFFFFFull);
        const int p = positions[r];
        chosen[r] = token;
        slots[r * slot_stride + p + 1] = token;
        positions[r] = p + 1;
    }
}

__global__ void batch_advance_kernel(const uint32_t *__restrict__ chosen, uint32_t *slots,
                                     int64_t slot_stride, int *positions, int rows)
{
    const int r = threadIdx.x;
    if (r >= rows)
        return;
    const int p = positions[r];
    slots[r * slot_stride + p + 1] = chosen[r];
    positions[r] = p + 1;
}

} // namespace

size_t rows_workspace_bytes(int inner, int outputs)
{
    if (inner <= 0 || outputs <= 0 || inner % kBlock != 0)
        return 0;
    const RowsPlan plan = rows_plan(inner, outputs);
    return plan.splits > 1 ? (size_t) plan.splits * kBatchRows * outputs * sizeof(double) : 0;
}

int rows_ticket_count(int outputs)
{
    return (outputs + kRowsTile - 1) / kRowsTile;
}

namespace {
hipError_t launch_rows(const RowsArgs &a, const RowsPlan &plan, hipStream_t stream);
}

bool rows_tiled_supported(int inner, int outputs)
{
    return inner > 0 && inner % (kChunkBlocks * kBlock) == 0 && outputs > 0;
}

size_t rows_tiled_bytes(int inner, int outputs)
{
    if (!rows_tiled_supported(inner, outputs))
        return 0;
    const size_t rowsPadded = (size_t) rows_ticket_count(outputs) * kRowsTile;
    return rowsPadded * inner + rowsPadded * (inner / kBlock) * sizeof(uint16_t);
}

hipError_t launch_tile_weights(const uint8_t *w8, int inner, int outputs, uint8_t *out,
                               hipStream_t stream)
{
    if (!w8 || !out || !rows_tiled_supported(inner, outputs)
        || reinterpret_cast<uintptr_t>(w8) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0
        || ((size_t) outputs * inner) % 16 != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(tile_weights_kernel, dim3(4096), dim3(kRowsThreads), 0, stream, w8, outputs,
                       inner, out);
    return hipGetLastError();
}

hipError_t launch_q8_rows(const uint8_t *x8, int x_rows, int rows, const uint8_t *w8, int inner,
                          int outputs, float *y, int y_stride, int residual, double *partials,
                          size_t partial_bytes, int *tickets, hipStream_t stream,
                          const uint8_t *w8_tiled, unsigned long long *best)
{
    if (w8_tiled && !rows_tiled_supported(inner, outputs))
        return hipErrorInvalidValue;
    if (rows <= 0 || rows > kBatchRows || x_rows < rows || inner <= 0 || inner % kBlock != 0
        || outputs <= 0 || y_stride < outputs)
        return hipErrorInvalidValue;
    const RowsPlan plan = rows_plan(inner, outputs);
    if (plan.splits > 1
        && (!partials || !tickets || partial_bytes < rows_workspace_bytes(inner, outputs)))
        return hipErrorInvalidValue;
    RowsArgs a{x8, x_rows, rows, w8, w8_tiled, inner, outputs, plan.per, y, y_stride,
               residual, partials, tickets, nullptr};
    a.best = best;
    return launch_rows(a, plan, stream);
}

bool rows_pick_supported(const uint8_t *w8, const uint8_t *w8_tiled, int inner, int outputs)
{
    if (inner <= 0 || inner % kBlock != 0 || outputs <= 0)
        return false;
    const RowsPlan plan = rows_plan(inner, outputs);
    const int nb = inner / kBlock, nc = plan.per / kChunkBlocks;
    const uintptr_t wScales = reinterpret_cast<uintptr_t>(w8) + (uintptr_t) outputs * inner;
    const bool whole = plan.per % kChunkBlocks == 0 && nb % plan.per == 0 && wScales % 16 == 0
                       && (nc == 1 || nc == 2 || nc == 4 || nc == 8 || nc == 16);
    (void) w8_tiled;
    const int groups = (rows_ticket_count(outputs) + kRowsWaves - 1) / kRowsWaves;
    return plan.wpt == 1 && plan.splits == 1 && whole && plan.per == nb && (nc == 4 || nc == 8)
           && groups > kRowsStreamGroups;
}

size_t rows_pick_bytes()
{
    return (size_t) kBatchRows * kRowsBestSlots * kRowsBestStride * sizeof(unsigned long long);
}

hipError_t launch_batch_pick_advance(unsigned long long *best, uint32_t *chosen, uint32_t *slots,
                                     int64_t slot_stride, int *positions, int rows,
                                     hipStream_t stream)
{
    if (!best || rows <= 0 || rows > kBatchRows || slot_stride <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(batch_pick_advance_kernel, dim3(rows), dim3(64), 0, stream, best, chosen,
                       slots, slot_stride, positions);
    return hipGetLastError();
}

bool rows_geglu_supported(int inner, int intermediate)
{
    if (inner <= 0 || inner % kBlock != 0 || intermediate <= 0 || intermediate % (2 * kRowsTile) != 0)
        return false;
    const RowsPlan plan = rows_plan(inner, 2 * intermediate);
    return plan.wpt == 1 && plan.splits == 1;
}

hipError_t launch_q8_rows_geglu(const uint8_t *x8, int x_rows, int rows, const uint8_t *w8,
                                int inner, int intermediate, uint8_t *geglu8, hipStream_t stream,
                                const uint8_t *w8_tiled)
{
    if (rows <= 0 || rows > kBatchRows || x_rows < rows || !geglu8
        || !rows_geglu_supported(inner, intermediate)
        || (w8_tiled && !rows_tiled_supported(inner, 2 * intermediate)))
        return hipErrorInvalidValue;
    const RowsPlan plan = rows_plan(inner, 2 * intermediate);
    const RowsArgs a{x8, x_rows, rows, w8, w8_tiled, inner, 2 * intermediate, plan.per, nullptr, 0,
                     0, nullptr, nullptr, geglu8};
    return launch_rows(a, plan, stream);
}

namespace {
// Tiled: the whole-chunk kernels read the fragment-ordered copy (a.w8t).
template <bool Tiled>
hipError_t launch_rows_as(const RowsArgs &a, const RowsPlan &plan, int nc, bool whole,
                          hipStream_t stream)
{
    const int inner = a.inner, outputs = a.outputs, nb = inner / kBlock;
    const int tilesPerGroup = kRowsWaves / plan.wpt;
    const int columns = (rows_ticket_count(outputs) + tilesPerGroup - 1) / tilesPerGroup;
    const dim3 grid = a.split_major ? dim3(plan.splits, columns) : dim3(columns, plan.splits);
    const size_t lds = rows_lds_bytes(plan);
    // split tiles of whole chunks with no split over workgroups (every chunk
    // in flight at once) load their activation blocks directly (the scale
    // rows 16-byte aligned: x8 aligned, nb a multiple of 8)
    const bool direct = plan.wpt == kRowsWaves && plan.splits == 1 && whole && !a.geglu8
                        && reinterpret_cast<uintptr_t>(a.x8) % 16 == 0;
    // wide products with whole rows of whole chunks and no GeGLU stream
    // their tiles through about two workgroups a compute unit
    const int groups = (rows_ticket_count(outputs) + kRowsWaves - 1) / kRowsWaves;
    const bool streamed = plan.wpt == 1 && plan.splits == 1 && whole && !a.geglu8 && plan.per == nb
                          && (nc == 4 || nc == 8) && groups > kRowsStreamGroups;
    if (a.best && !streamed) // the pick rides on the streamed product only
        return hipErrorInvalidValue;
    if (streamed) {
        if (!a.tickets)
            return hipErrorInvalidValue;
        const dim3 sgrid(kRowsStreamGroups);
        if (nc == 4)
            hipLaunchKernelGGL((q8_rows_stream_kernel<4, Tiled>), sgrid, dim3(kRowsThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((q8_rows_stream_kernel<8, Tiled>), sgrid, dim3(kRowsThreads), 0, stream, a);
        return hipGetLastError();
    }
    if (direct) {
        const size_t epilogue = (size_t) kRowsWaves * kBatchRows * (kRowsTile + 1) * sizeof(double);
#define GQ8_ROWS_DIRECT(N)                                                                     \
    hipLaunchKernelGGL((q8_rows_kernel<kRowsWaves, N, true, Tiled>), grid, dim3(kRowsThreads),   \
                       epilogue, stream, a)
        switch (nc) {
        case 1: GQ8_ROWS_DIRECT(1); break;
        case 2: GQ8_ROWS_DIRECT(2); break;
        case 4: GQ8_ROWS_DIRECT(4); break;
        case 8: GQ8_ROWS_DIRECT(8); break;
        default: GQ8_ROWS_DIRECT(16); break;
        }
#undef GQ8_ROWS_DIRECT
        return hipGetLastError();
    }
#define GQ8_ROWS(W, N)                                                                         \
    hipLaunchKernelGGL((q8_rows_kernel<W, N, false, Tiled>), grid, dim3(kRowsThreads), lds, stream, a)
#define GQ8_ROWS_NC(W)                                                                         \
    switch (nc) {                                                                              \
    case 1: GQ8_ROWS(W, 1); break;                                                             \
    case 2: GQ8_ROWS(W, 2); break;                                                             \
    case 4: GQ8_ROWS(W, 4); break;                                                             \
    case 8: GQ8_ROWS(W, 8); break;                                                             \
    default: GQ8_ROWS(W, 16); break;                                                           \
    }
    if (!whole) { // row-major, any range
        if constexpr (Tiled)
            return hipErrorInvalidValue;
        if (plan.wpt == 1)
            hipLaunchKernelGGL((q8_rows_kernel<1, 0>), grid, dim3(kRowsThreads), lds, stream, a);
        else if (plan.wpt == 2)
            hipLaunchKernelGGL((q8_rows_kernel<2, 0>), grid, dim3(kRowsThreads), lds, stream, a);
        else
            hipLaunchKernelGGL((q8_rows_kernel<kRowsWaves, 0>), grid, dim3(kRowsThreads), lds, stream, a);
    } else if (plan.wpt == 1) {
        GQ8_ROWS_NC(1);
    } else if (plan.wpt == 2) {
        GQ8_ROWS_NC(2);
    } else {
        GQ8_ROWS_NC(kRowsWaves);
    }
#undef GQ8_ROWS_NC
#undef GQ8_ROWS
    return hipGetLastError();
}

hipError_t launch_rows(const RowsArgs &a, const RowsPlan &plan, hipStream_t stream)
{
    const int inner = a.inner, outputs = a.outputs;
    const int nb = inner / kBlock;
    const uintptr_t wScales = reinterpret_cast<uintptr_t>(a.w8) + (uintptr_t) outputs * inner;
    // whole chunks: every wave's range a multiple of 8 blocks inside the row
    // (the last split's waves may hold fewer, or none: nb a multiple of per)
    const int nc = plan.per / kChunkBlocks;
    const bool whole = plan.per % kChunkBlocks == 0 && nb % plan.per == 0 && wScales % 16 == 0
                       && (nc == 1 || nc == 2 || nc == 4 || nc == 8 || nc == 16);
    RowsArgs b = a;
    b.split_major = plan.splits > 1;
    if (a.w8t && whole)
        return launch_rows_as<true>(b, plan, nc, whole, stream);
    b.w8t = nullptr;
    return launch_rows_as<false>(b, plan, nc, whole, stream);
}
} // namespace

bool rows_attention_supported(int heads, int kv_heads, int head_dim, int max_positions)
{
    return kv_heads == 1 && (head_dim == 64 || head_dim == 128 || head_dim == 256)
           && (heads == 2 || heads == 4 || heads == 8) && max_positions > 0
           && max_positions <= kRowsMaxSplits * kRowsTileKeys * 64;
}

int rows_attention_split_keys(int max_positions)
{
    const int span = kRowsMaxSplits * kRowsTileKeys;
    return kRowsTileKeys * ((max_positions + span - 1) / span);
}

size_t rows_attention_workspace_doubles(int rows, int heads, int head_dim)
{
    return (size_t) rows * kRowsMaxSplits * heads * (head_dim + 2);
}

hipError_t launch_rows_attention(const RowsAttentionArgs &a, int rows, int max_positions,
                                 hipStream_t stream)
{
    if (rows <= 0 || rows > kBatchRows || a.q8_rows < rows || !a.row_angles
        || !rows_attention_supported(a.heads, 1, a.head_dim, max_positions)
        || a.per_split != rows_attention_split_keys(max_positions) || a.max_positions != max_positions)
        return hipErrorInvalidValue;
    const int groups = a.heads > kRowsHeadGroup ? a.heads / kRowsHeadGroup : 1;
    const dim3 grid((max_positions + a.per_split - 1) / a.per_split, rows, groups);
    const int C = a.head_dim / 64;
#define GQ8_ROWS_ATTENTION(CC, HH)                                                              \
    hipLaunchKernelGGL((attention_rows_kernel<CC, HH, (HH > kRowsHeadGroup ? kRowsHeadGroup : HH)>), grid, \
                       dim3(kRowsThreads), 0, stream, a)
    switch (a.heads * 8 + C) {
    case 2 * 8 + 1: GQ8_ROWS_ATTENTION(1, 2); break;
    case 2 * 8 + 2: GQ8_ROWS_ATTENTION(2, 2); break;
    case 2 * 8 + 4: GQ8_ROWS_ATTENTION(4, 2); break;
    case 4 * 8 + 1: GQ8_ROWS_ATTENTION(1, 4); break;
    case 4 * 8 + 2: GQ8_ROWS_ATTENTION(2, 4); break;
    case 4 * 8 + 4: GQ8_ROWS_ATTENTION(4, 4); break;
    case 8 * 8 + 1: GQ8_ROWS_ATTENTION(1, 8); break;
    case 8 * 8 + 2: GQ8_ROWS_ATTENTION(2, 8); break;
    case 8 * 8 + 4: GQ8_ROWS_ATTENTION(4, 8); break;
    default: return hipErrorInvalidValue;
    }
#undef GQ8_ROWS_ATTENTION
    if (hipError_t e = hipGetLastError(); e != hipSuccess)
        return e;
    hipLaunchKernelGGL(attention_merge_rows_kernel, dim3(a.heads * (a.head_dim / 64), rows), dim3(64), 0,
                       stream, a);
    return hipGetLastError();
}

hipError_t launch_batch_advance(const uint32_t *chosen, uint32_t *slots, int64_t slot_stride,
                                int *positions, int rows, hipStream_t stream)
{
    if (rows <= 0 || rows > 64 || slot_stride <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(batch_advance_kernel, dim3(1), dim3(64), 0, stream, chosen, slots,
                       slot_stride, positions, rows);
    return hipGetLastError();
}

} // namespace gq8
