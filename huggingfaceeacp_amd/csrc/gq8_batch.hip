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
// bytes of weight row (l % 16)'s block, both at byte 8 (l / 16) of the block,
// straight from memory (the activation rows stay in L2 across workgroups);
// the result D[m][n] lands in lane 16 (m / 4) + n, element m % 4.  A
// workgroup of four waves owns one 16-row tile of the outputs; its waves take
// consecutive ranges of blocks and add their 16 x 16 double tiles in LDS in
// wave (= block) order.  Products with too few tiles to fill the chip split
// the blocks over several workgroups: each stores its double tile, and the
// last of a tile's workgroups (a ticket per tile) adds them in split order.
//
// attention_rows_kernel: one workgroup per (sequence, key split) scores all
// the query heads against one read of the split's keys (the single KV head of
// multi-query attention), so every key and value row is read once a layer.
// It also takes the step's RoPE and cache append: each workgroup rotates the
// sequence's query row itself, and the workgroup whose split holds the new
// position rotates the new key, appends it (and the value) to the cache and
// uses it for that position.  The last split of a sequence to finish merges
// the splits (MultiQueryAttention.h:43-49) and quantizes the row for o_proj.
#include "gq8_device.hpp"
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"

namespace gq8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kRowsThreads = 256;
constexpr int kRowsWaves = kRowsThreads / 64;
constexpr int kRowsTile = 16;         // outputs a workgroup
constexpr int kChunkBlocks = 8;       // blocks a wave loads at once
constexpr int kTargetWorkgroups = 512;

struct RowsPlan {
    int per;    // blocks a wave takes
    int splits; // workgroups over one tile's blocks
};

// Whole chunks a wave while the tiles alone leave the chip short of
// workgroups; the split count follows.
RowsPlan rows_plan(int inner, int outputs)
{
    const int nb = inner / kBlock;
    const int tiles = (outputs + kRowsTile - 1) / kRowsTile;
    int per = (nb + kRowsWaves - 1) / kRowsWaves;
    if (per > kChunkBlocks)
        per = (per + kChunkBlocks - 1) / kChunkBlocks * kChunkBlocks;
    int splits = 1;
    while ((int64_t) tiles * splits < kTargetWorkgroups && per > kChunkBlocks
           && per % (2 * kChunkBlocks) == 0) {
        per /= 2;
        splits = (nb + kRowsWaves * per - 1) / (kRowsWaves * per);
    }
    return {per, splits};
}

struct RowsArgs {
    const uint8_t *x8;
    int x_rows, rows;
    const uint8_t *w8;
    int inner, outputs, per;
    float *y;
    int y_stride, residual;
    double *partials; // [splits][kBatchRows][outputs]
    int *tickets;     // one a tile
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

// V: the scales of a chunk load as one 16-byte vector per row (the block
// count and every wave's first block are multiples of 8).
template <bool V>
__global__ __launch_bounds__(kRowsThreads) void q8_rows_kernel(RowsArgs a)
{
    __shared__ double sPart[kRowsWaves][kBatchRows][kRowsTile + 1];
    __shared__ int sLast;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nb = a.inner / kBlock;
    const int col = lane & 15, grp = lane >> 4;
    const int n0 = blockIdx.x * kRowsTile;
    // operand rows of this lane, clamped into range (their results are never stored)
    const int n = min(n0 + col, a.outputs - 1);
    const int xr = min(col, a.rows - 1);
    const uint8_t *wRow = a.w8 + (int64_t) n * a.inner + grp * 8;
    const uint8_t *xRow = a.x8 + (int64_t) xr * a.inner + grp * 8;
    const uint16_t *wScale = reinterpret_cast<const uint16_t *>(a.w8 + (int64_t) a.outputs * a.inner)
                             + (int64_t) n * nb;
    const uint16_t *xScales = reinterpret_cast<const uint16_t *>(a.x8 + (int64_t) a.x_rows * a.inner);
    const uint16_t *xScale[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        xScale[r] = xScales + (int64_t) min(4 * grp + r, a.rows - 1) * nb;

    const int b0 = (blockIdx.y * kRowsWaves + wave) * a.per;
    const int b1 = min(b0 + a.per, nb);
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int c0 = b0; c0 < b1; c0 += kChunkBlocks) {
        long wv[kChunkBlocks], xv[kChunkBlocks];
#pragma unroll
        for (int k = 0; k < kChunkBlocks; ++k) {
            const int b = min(c0 + k, b1 - 1);
            wv[k] = *reinterpret_cast<const long *>(wRow + (int64_t) b * kBlock);
            xv[k] = *reinterpret_cast<const long *>(xRow + (int64_t) b * kBlock);
        }
        float sw[kChunkBlocks], sx[4][kChunkBlocks];
        if constexpr (V) {
            const uint4 w4 = *reinterpret_cast<const uint4 *>(wScale + c0);
            const uint32_t ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int k = 0; k < kChunkBlocks; ++k)
                sw[k] = half_of(ww[k / 2], k & 1);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint4 x4 = *reinterpret_cast<const uint4 *>(xScale[r] + c0);
                const uint32_t xw[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                for (int k = 0; k < kChunkBlocks; ++k)
                    sx[r][k] = half_of(xw[k / 2], k & 1);
            }
        } else {
            // blocks past the wave's range were loaded clamped; a zero scale
            // drops them (0 * dot adds an exact zero)
#pragma unroll
            for (int k = 0; k < kChunkBlocks; ++k) {
                const int b = min(c0 + k, b1 - 1);
                sw[k] = c0 + k < b1 ? half_value(wScale[b]) : 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sx[r][k] = half_value(xScale[r][b]);
            }
        }
        // no branch between the loads and the arithmetic, and no arithmetic
        // scheduled among the loads: every load of the chunk is in flight
        // before the first product waits
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < kChunkBlocks; ++k) {
            const v4i zero = {0, 0, 0, 0};
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(xv[k], wv[k], zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) // the scale product is exact in fp32
                acc[r] = fma((double) d[r], (double) (sw[k] * sx[r][k]), acc[r]);
        }
    }

#pragma unroll
    for (int r = 0; r < 4; ++r)
        sPart[wave][4 * grp + r][col] = acc[r];
    __syncthreads();
    const int m = t >> 4, c = t & 15; // 256 threads: one (sequence, output) cell each
    double sum = sPart[0][m][c];
#pragma unroll
    for (int w = 1; w < kRowsWaves; ++w)
        sum += sPart[w][m][c];
    const int on = n0 + c;
    const bool live = m < a.rows && on < a.outputs;
    if (gridDim.y == 1) {
        if (live) {
            float *dst = a.y + (int64_t) m * a.y_stride + on;
            const double old = a.residual ? (double) *dst : 0.0;
            *dst = (float) (sum + old);
        }
        return;
    }

    // the blocks are split over gridDim.y workgroups: agent-scope stores
    // (coherent across the L2s), completed before the ticket is taken
    if (live)
        store_agent_d(a.partials + ((int64_t) blockIdx.y * kBatchRows + m) * a.outputs + on, sum);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0)
        sLast = __hip_atomic_fetch_add(a.tickets + blockIdx.x, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == (int) gridDim.y - 1;
    __syncthreads();
    if (!sLast)
        return;
    if (live) {
        double total = 0.0;
        for (int s = 0; s < (int) gridDim.y; ++s)
            total += load_agent_d(a.partials + ((int64_t) s * kBatchRows + m) * a.outputs + on);
        float *dst = a.y + (int64_t) m * a.y_stride + on;
        const double old = a.residual ? (double) *dst : 0.0;
        *dst = (float) (total + old);
    }
    if (t == 0) // ready for the next launch
        __hip_atomic_store(a.tickets + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- attention of the lockstep rows ---------------------------------------------
constexpr int kRowsTileKeys = 64;   // keys a tile (16 a key wave)
constexpr int kRowsWaveKeys = 16;

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

// C channels a lane (head width 64 C), HW heads a wave, HG head groups: four
// key waves per head group, 256 HG threads.
template <int C, int HW, int HG>
__global__ __launch_bounds__(256 * HG) void attention_rows_kernel(RowsAttentionArgs a)
{
    constexpr int H = HW * HG, kWaves = 4 * HG, kThreadsAll = 256 * HG;
    constexpr int hd = 64 * C, half = hd / 2, qW = H * hd;
    constexpr int R = 16 / HW; // keys a scoring round: 16 (key, head) rows a reduction
    static_assert(HW * R == 16 && kRowsWaveKeys % R == 0, "rounds");
    __shared__ float sQ[qW];
    __shared__ __attribute__((aligned(8))) uint16_t sKnew[hd], sVnew[hd];
    __shared__ double sS[H][kRowsTileKeys];
    __shared__ double sMax[H], sSum[H], sF[H];
    __shared__ double sAcc[kWaves][HW * hd];
    __shared__ double sMerge[H][kRowsMaxSplits];
    __shared__ int sLast;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = wave >> 2, kw = wave & 3;
    const int seq = blockIdx.y, split = blockIdx.x;
    const int pos = a.positions[seq];
    const int keyCount = pos + 1;
    const int k0 = split * a.per_split;
    if (k0 >= keyCount)
        return;
    const int k1 = min(k0 + a.per_split, keyCount);
    const bool holdsNew = k1 == keyCount; // this split ends at the new position
    const float *row = a.qkv + (int64_t) seq * a.qkv_stride;
    uint16_t *keys = a.key_cache + seq * a.cache_stride;
    uint16_t *values = a.value_cache + seq * a.cache_stride;

    // RoPE (rope_kv_kernel's arithmetic): the query heads, and the new key
    // where this split holds it; the new value rounded to fp16
    for (int idx = t; idx < (H + 1) * half; idx += kThreadsAll) {
        const int head = idx / half, i = idx % half;
        if (head == H && !holdsNew)
            break;
        const float *base = row + head * hd; // head H: the key, right after the queries
        const int64_t angle = (int64_t) pos * half + i;
        float lo, hi;
        rotate_pair(base[i], base[i + half], a.cosines[angle], a.sines[angle], &lo, &hi);
        if (head < H) {
            sQ[head * hd + i] = lo;
            sQ[head * hd + i + half] = hi;
        } else {
            sKnew[i] = half_bits(lo);
            sKnew[i + half] = half_bits(hi);
        }
    }
    if (holdsNew)
        for (int i = t; i < hd; i += kThreadsAll)
            sVnew[i] = half_bits(row[qW + hd + i]);
    if (t < H) {
        sMax[t] = -INFINITY;
        sSum[t] = 0.0;
    }
    __syncthreads();
    if (holdsNew)
        for (int i = t; i < hd; i += kThreadsAll) {
            keys[(int64_t) pos * hd + i] = sKnew[i];
            values[(int64_t) pos * hd + i] = sVnew[i];
        }

    const int c0 = lane * C;
    double q[HW][C], acc[HW][C];
#pragma unroll
    for (int h = 0; h < HW; ++h)
#pragma unroll
        for (int c = 0; c < C; ++c) {
            q[h][c] = (double) sQ[(g * HW + h) * hd + c0 + c];
            acc[h][c] = 0.0;
        }

    for (int t0 = k0; t0 < k1; t0 += kRowsTileKeys) {
        const int nk = min(kRowsTileKeys, k1 - t0);
        // this wave's keys t0 + 16 kw + i, clamped into the tile (the
        // duplicates are masked), the new position's row from LDS
        const bool tileHoldsNew = holdsNew && t0 + nk == keyCount;
        Halves<C> kh[kRowsWaveKeys], vh[kRowsWaveKeys];
#pragma unroll
        for (int i = 0; i < kRowsWaveKeys; ++i) {
            const int j = t0 + min(kw * kRowsWaveKeys + i, nk - 1);
            kh[i] = load_channels<C>(keys + (int64_t) j * hd + c0);
        }
        if (tileHoldsNew) {
            const Halves<C> kn = load_channels<C>(sKnew + c0);
#pragma unroll
            for (int i = 0; i < kRowsWaveKeys; ++i)
                if (t0 + min(kw * kRowsWaveKeys + i, nk - 1) == pos)
                    kh[i] = kn;
        }
#pragma unroll
        for (int r0 = 0; r0 < kRowsWaveKeys; r0 += R) {
            double y[16];
#pragma unroll
            for (int i = 0; i < R; ++i)
#pragma unroll
                for (int h = 0; h < HW; ++h) {
                    double p = 0.0;
#pragma unroll
                    for (int c = 0; c < C; ++c)
                        p += q[h][c] * (double) kh[r0 + i].at(c);
                    y[i * HW + h] = p;
                }
            const double total = reduce_rows<16>(y, lane);
            if (stores_row<16>(lane)) {
                const int rr = row_of_lane<16>(lane);
                const int jj = kw * kRowsWaveKeys + r0 + rr / HW;
                sS[g * HW + rr % HW][jj] = jj < nk ? (double) a.scale * total : -INFINITY;
            }
            __builtin_amdgcn_sched_barrier(0); // one round's conversions at a time
        }
        // the values, in flight during the softmax
#pragma unroll
        for (int i = 0; i < kRowsWaveKeys; ++i) {
            const int j = t0 + min(kw * kRowsWaveKeys + i, nk - 1);
            vh[i] = load_channels<C>(values + (int64_t) j * hd + c0);
        }
        if (tileHoldsNew) {
            const Halves<C> vn = load_channels<C>(sVnew + c0);
#pragma unroll
            for (int i = 0; i < kRowsWaveKeys; ++i)
                if (t0 + min(kw * kRowsWaveKeys + i, nk - 1) == pos)
                    vh[i] = vn;
        }
        __syncthreads();
        // the tile's softmax against the running maximum, one wave a head
        if (wave < H) {
            const int h = wave;
            const double sc = lane < nk ? sS[h][lane] : -INFINITY;
            const double tileMax = wave_max_d(sc);
            const double previous = sMax[h];
            const double largest = fmax(previous, tileMax);
            const double w = lane < nk ? exp(sc - largest) : 0.0;
            const double total = wave_sum_d(w);
            sS[h][lane] = w;
            if (lane == 0) {
                const double factor = previous == -INFINITY ? 0.0 : exp(previous - largest);
                sF[h] = factor;
                sSum[h] = sSum[h] * factor + total;
                sMax[h] = largest;
            }
        }
        __syncthreads();
        // this wave's keys in order for every head (weights past the tile are zero)
        double part[HW][C];
#pragma unroll
        for (int h = 0; h < HW; ++h)
#pragma unroll
            for (int c = 0; c < C; ++c)
                part[h][c] = 0.0;
#pragma unroll
        for (int i = 0; i < kRowsWaveKeys; ++i) {
            double v[C];
#pragma unroll
            for (int c = 0; c < C; ++c)
                v[c] = (double) vh[i].at(c);
#pragma unroll
            for (int h = 0; h < HW; ++h) {
                const double wi = sS[g * HW + h][kw * kRowsWaveKeys + i];
#pragma unroll
                for (int c = 0; c < C; ++c)
                    part[h][c] += wi * v[c];
            }
        }
#pragma unroll
        for (int h = 0; h < HW; ++h) {
            const double f = sF[g * HW + h];
#pragma unroll
            for (int c = 0; c < C; ++c)
                acc[h][c] = acc[h][c] * f + part[h][c];
        }
        __syncthreads(); // the next tile rewrites the scores
    }

    // the split's partial: the four key waves of each head in order
#pragma unroll
    for (int h = 0; h < HW; ++h)
#pragma unroll
        for (int c = 0; c < C; ++c)
            sAcc[wave][h * hd + c0 + c] = acc[h][c];
    __syncthreads();
    const int64_t slot = (int64_t) seq * kRowsMaxSplits + split;
    for (int o = t; o < qW; o += kThreadsAll) {
        const int head = o / hd, gg = head / HW, within = o - gg * HW * hd;
        double v = sAcc[gg * 4][within];
#pragma unroll
        for (int w = 1; w < 4; ++w)
            v += sAcc[gg * 4 + w][within];
        store_agent_d(a.ws_o + slot * qW + o, v);
    }
    if (t < H) {
        store_agent_d(a.ws_ml + (slot * H + t) * 2, sMax[t]);
        store_agent_d(a.ws_ml + (slot * H + t) * 2 + 1, sSum[t]);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // the stores have completed
    __syncthreads();
    const int splits = (keyCount + a.per_split - 1) / a.per_split;
    if (t == 0)
        sLast = __hip_atomic_fetch_add(a.tickets + seq, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
    __syncthreads();
    if (!sLast)
        return;

    // the merge: split weights per head (one split a lane), then the row
    const int64_t first = (int64_t) seq * kRowsMaxSplits;
    if (wave < H) {
        const bool live = lane < splits;
        const int sp = live ? lane : 0;
        const double m = load_agent_d(a.ws_ml + ((first + sp) * H + wave) * 2);
        const double sum = load_agent_d(a.ws_ml + ((first + sp) * H + wave) * 2 + 1);
        double total;
        const double f = merge_factor(m, sum, live, total);
        if (live)
            sMerge[wave][sp] = f;
        if (lane == 0)
            sSum[wave] = total;
    }
    __syncthreads();
    uint16_t *scales = reinterpret_cast<uint16_t *>(a.q8 + (int64_t) a.q8_rows * qW)
                       + (int64_t) seq * (qW / kBlock);
    for (int o = t; o < qW; o += kThreadsAll) { // whole waves: qW is a multiple of 64
        const int head = o / hd;
        double weighted = 0.0;
        for (int s0 = 0; s0 < splits; s0 += 8) {
            double part[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                part[u] = s0 + u < splits ? load_agent_d(a.ws_o + (first + s0 + u) * qW + o) : 0.0;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s0 + u < splits)
                    weighted += part[u] * sMerge[head][s0 + u];
        }
        const float v = (float) (weighted / sSum[head]);
        const float amax = max_lanes<16>(fabsf(v));
        const uint16_t bits = scale_bits_from_amax(amax);
        const float sc = half_value(bits);
        a.q8[(int64_t) seq * qW + o] = (uint8_t) (int8_t) (bits ? quantize_value(v, sc, 1.0f / sc) : 0);
        if ((o & 31) == 0)
            scales[o / kBlock] = bits;
    }
    if (t == 0) // ready for the next launch
        __hip_atomic_store(a.tickets + seq, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

hipError_t launch_q8_rows(const uint8_t *x8, int x_rows, int rows, const uint8_t *w8, int inner,
                          int outputs, float *y, int y_stride, int residual, double *partials,
                          size_t partial_bytes, int *tickets, hipStream_t stream)
{
    if (rows <= 0 || rows > kBatchRows || x_rows < rows || inner <= 0 || inner % kBlock != 0
        || outputs <= 0 || y_stride < outputs)
        return hipErrorInvalidValue;
    const RowsPlan plan = rows_plan(inner, outputs);
    if (plan.splits > 1
        && (!partials || !tickets || partial_bytes < rows_workspace_bytes(inner, outputs)))
        return hipErrorInvalidValue;
    RowsArgs a{x8, x_rows, rows, w8, inner, outputs, plan.per, y, y_stride, residual, partials,
               tickets};
    const int nb = inner / kBlock;
    const uintptr_t wScales = reinterpret_cast<uintptr_t>(w8) + (uintptr_t) outputs * inner;
    const uintptr_t xScales = reinterpret_cast<uintptr_t>(x8) + (uintptr_t) x_rows * inner;
    const bool vec = nb % kChunkBlocks == 0 && plan.per % kChunkBlocks == 0 && wScales % 16 == 0
                     && xScales % 16 == 0;
    const dim3 grid(rows_ticket_count(outputs), plan.splits);
    if (vec)
        hipLaunchKernelGGL(q8_rows_kernel<true>, grid, dim3(kRowsThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(q8_rows_kernel<false>, grid, dim3(kRowsThreads), 0, stream, a);
    return hipGetLastError();
}

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
    if (rows <= 0 || rows > kBatchRows || a.q8_rows < rows
        || !rows_attention_supported(a.heads, 1, a.head_dim, max_positions)
        || a.per_split != rows_attention_split_keys(max_positions))
        return hipErrorInvalidValue;
    const dim3 grid((max_positions + a.per_split - 1) / a.per_split, rows);
    const int C = a.head_dim / 64;
#define GQ8_ROWS_ATTENTION(CC, HW, HG)                                                              hipLaunchKernelGGL((attention_rows_kernel<CC, HW, HG>), grid, dim3(256 * HG), 0, stream, a)
    switch (a.heads * 8 + C) {
    case 2 * 8 + 1: GQ8_ROWS_ATTENTION(1, 2, 1); break;
    case 2 * 8 + 2: GQ8_ROWS_ATTENTION(2, 2, 1); break;
    case 2 * 8 + 4: GQ8_ROWS_ATTENTION(4, 2, 1); break;
    case 4 * 8 + 1: GQ8_ROWS_ATTENTION(1, 4, 1); break;
    case 4 * 8 + 2: GQ8_ROWS_ATTENTION(2, 4, 1); break;
    case 4 * 8 + 4: GQ8_ROWS_ATTENTION(4, 4, 1); break;
    case 8 * 8 + 1: GQ8_ROWS_ATTENTION(1, 4, 2); break;
    case 8 * 8 + 2: GQ8_ROWS_ATTENTION(2, 4, 2); break;
    case 8 * 8 + 4: GQ8_ROWS_ATTENTION(4, 4, 2); break;
    default: return hipErrorInvalidValue;
    }
#undef GQ8_ROWS_ATTENTION
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
