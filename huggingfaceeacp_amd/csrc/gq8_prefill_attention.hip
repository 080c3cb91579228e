// gq8_prefill_attention.hip -- causal multi-query attention of a prompt block
// (MultiQueryAttention.h:275-308, MultiQueryPrefillAttention) on fp64 MFMA.
//
// Row r of the block sits at position base + r and attends keys [0, base + r]
// of its KV head (query head h reads KV head h / (heads / kv_heads)).  Scores
// scale * q.k, the softmax and the value sums are double, as in the decode
// kernel and the oracle; the block's rows leave as fp32 and as the Q8 row of
// the o product.
//
// Work split: a workgroup owns 16 consecutive rows of one head; its four
// waves take the key tiles (16 keys) round robin, each keeping an online
// softmax state (row maximum, sum and the 16 x head_dim sums), and the states
// are merged in LDS at the end.  The grid starts the longest row blocks
// first, so the short ones fill in behind them.  A wave requests a tile's
// values (16-byte loads) before its scores and the next tile's keys right
// after them, so no tile's operands wait in registers a whole tile ahead; the
// kernel is held to two waves a SIMD (256 registers a wave), and one wave's
// MFMAs run while the other waits on its loads or works on its softmax.
//
// Per tile a wave computes S^T = K Q^T with v_mfma_f64_16x16x4f64, so the
// result holds row j of the block on lanes j, j + 16, j + 32, j + 48 and is
// already the P operand of O += P V (no transpose through LDS).  The online
// softmax is lazy: a row's reference maximum moves (and its sums are
// rescaled) only when a tile's maximum exceeds it by more than kLazyMargin,
// so most tiles need no rescaling; the weights exp(s - m) stay below
// e^kLazyMargin and every sum stays double.
//
// fp64 MFMA operand layout (checked on gfx950): A 16 x 4 with lane l holding
// A[l % 16][l / 16]; B 4 x 16 with lane l holding B[l / 16][l % 16]; D 16 x 16
// with lane l holding D[l / 16 + 4 r][l % 16], r = 0..3.  With g = l / 16 and
// j = l % 16:
//  - S^T (keys x rows, reduced over channels): lane (g, j) supplies key j's
//    and query row j's channels [g E, g E + E) (E = head_dim / 4), read
//    contiguously, and receives the scores of row j against keys g + 4 r.
//  - O (rows x channels, reduced over 4 keys a step): step st takes keys
//    g + 4 st, so lane (g, j) supplies its own weight p[st]; output tile n
//    holds channels j T + n (T = head_dim / 16), so a lane's value operands
//    are T contiguous channels of one key row and its outputs T contiguous
//    channels of rows g + 4 r.
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"

namespace gq8 {
namespace {

typedef double v4d __attribute__((ext_vector_type(4)));

constexpr int kPaRows = 16;   // query rows a workgroup
constexpr int kPaWaves = 4;
constexpr int kPaThreads = kPaWaves * 64;
constexpr int kPaKeys = 16;   // keys a tile
constexpr double kLazyMargin = 8.0;

struct PrefillArgs {
    const float *queries;
    int q_stride;
    const uint16_t *key_cache, *value_cache;
    int heads, kv_heads, head_dim;
    int rows;
    const int *pos_ptr;
    int pos_value;
    float scale;
    float *out;   // optional [rows, heads * head_dim]
    uint8_t *q8;  // optional Q8 row buffer of rows x heads * head_dim
};

__device__ inline v4d mfma(double a, double b, v4d c)
{
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// N consecutive fp16 values (N a multiple of 4), as N / 2 words
template <int N>
__device__ inline void load_halves(const uint16_t *p, uint32_t (&w)[N / 2])
{
    if constexpr (N % 8 == 0) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            const uint4 v = reinterpret_cast<const uint4 *>(p)[i];
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    } else {
        static_assert(N == 4, "4, 8, 16, ... halves");
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        w[0] = v.x; w[1] = v.y;
    }
}

template <int N>
__device__ inline double half_at(const uint32_t (&w)[N], int i)
{
    return (double) half_value((uint16_t) (w[i >> 1] >> (16 * (i & 1))));
}

// E channels a lane group, T = head_dim / 16 output column tiles.
template <int E>
__global__ __launch_bounds__(kPaThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_attention_kernel(PrefillArgs a)
{
    constexpr int HD = 4 * E, T = HD / 16;
    constexpr int KW = E / 2, VW = T / 2; // words of a lane's key channels / value channels
    constexpr int kBlockLanes = kBlock / T;  // lanes holding one 32-channel block of an output row
    constexpr int kMergeTiles = T < 4 ? T : 4;
    // the merge: every wave's maxima and scaled sums of the rows g + 4 r, and
    // kMergeTiles column tiles of every wave's output sums at a time (over
    // the query rows, which no wave reads once all are past their tiles)
    __shared__ double sMax[kPaWaves][4][64], sSum[kPaWaves][4][64];
    constexpr int kQBytes = kPaRows * (HD + 4) * (int) sizeof(float);
    constexpr int kPartBytes = kPaWaves * kMergeTiles * 4 * 64 * (int) sizeof(double);
    __shared__ __align__(16) unsigned char sQPart[kQBytes > kPartBytes ? kQBytes : kPartBytes];
    // padded: a 16-lane group's rows on distinct banks
    float (*sQ)[HD + 4] = reinterpret_cast<float (*)[HD + 4]>(sQPart);
    double (*sPart)[kMergeTiles][4][64] = reinterpret_cast<double (*)[kMergeTiles][4][64]>(sQPart);

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, j = lane & 15;
    const int blocks = (a.rows + kPaRows - 1) / kPaRows;
    const int rb = blocks - 1 - (int) blockIdx.x / a.heads; // the longest row blocks first
    const int h = (int) blockIdx.x % a.heads;
    const int r0 = rb * kPaRows;
    const int qWidth = a.heads * HD, kvWidth = a.kv_heads * HD;
    const int kvh = h / (a.heads / a.kv_heads);
    const int base = (a.pos_ptr ? *a.pos_ptr : 0) + a.pos_value;
    const int rowsHere = min(kPaRows, a.rows - r0);
    const int lastKey = base + r0 + rowsHere - 1;  // the block's last row attends [0, lastKey]
    const int tiles = lastKey / kPaKeys + 1;
    const int myRow = min(j, rowsHere - 1);        // rows past the block repeat its last row
    const int rowPos = base + r0 + myRow;

    // the block's query rows in LDS (rows past the block repeat its last row);
    // lane (g, j) reads row j's channels [g E, g E + E), the B operand of S^T
#pragma unroll
    for (int i = t; i < kPaRows * HD / 4; i += kPaThreads) {
        const int row = i / (HD / 4), c = (i % (HD / 4)) * 4;
        const float *src = a.queries + (int64_t) (r0 + min(row, rowsHere - 1)) * a.q_stride + h * HD + c;
        *reinterpret_cast<float4 *>(&sQ[row][c]) = *reinterpret_cast<const float4 *>(src);
    }
    __syncthreads();
    const int qAt = j * (HD + 4) + g * E; // lane (g, j)'s first query channel in sQ
    const uint16_t *keys = a.key_cache + kvh * HD + g * E;
    const uint16_t *values = a.value_cache + kvh * HD + j * T;
    // a tile's operands: key k0 + j's channels, and keys k0 + g + 4 st's value channels
    // (keys past the block's last are clamped to it and masked)
    auto load_keys = [&](int tile, uint32_t (&kw)[KW]) {
        const int k0 = tile * kPaKeys;
        load_halves<E>(keys + (int64_t) min(k0 + j, lastKey) * kvWidth, kw);
    };
    auto load_values = [&](int tile, uint32_t (&vw)[4][VW]) {
        const int k0 = tile * kPaKeys;
#pragma unroll
        for (int st = 0; st < 4; ++st)
            load_halves<T>(values + (int64_t) min(k0 + g + 4 * st, lastKey) * kvWidth, vw[st]);
    };

    double m = -INFINITY, l = 0.0; // row j's reference maximum and sum (alike on its 4 lanes)
    v4d o[T];
#pragma unroll
    for (int n = 0; n < T; ++n)
        o[n] = v4d{0.0, 0.0, 0.0, 0.0};

    uint32_t kw[KW], vw[4][VW];
    if (wave < tiles)
        load_keys(wave, kw);
    for (int tile = wave; tile < tiles; tile += kPaWaves) {
        load_values(tile, vw); // arrive while the scores are computed
        const int k0 = tile * kPaKeys;

        // the query is read from LDS every tile: an opaque offset keeps the
        // compiler from holding all E channels as doubles across the loop
        int qOff = qAt;
        asm volatile("" : "+v"(qOff));
        const float *qRow = &sQ[0][0] + qOff;
        v4d s = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int c = 0; c < E; c += 4) {
            const float4 qv = *reinterpret_cast<const float4 *>(qRow + c);
            s = mfma(half_at(kw, c), (double) qv.x, s);
            s = mfma(half_at(kw, c + 1), (double) qv.y, s);
            s = mfma(half_at(kw, c + 2), (double) qv.z, s);
            s = mfma(half_at(kw, c + 3), (double) qv.w, s);
        }

        // the next tile's keys: they arrive during the softmax and O += P V
        load_keys(min(tile + kPaWaves, tiles - 1), kw);

        // row j against keys k0 + g + 4 r
        double sv[4];
        bool live[4];
        double tileMax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            live[r] = k0 + g + 4 * r <= rowPos;
            sv[r] = live[r] ? (double) a.scale * s[r] : -INFINITY;
            tileMax = fmax(tileMax, sv[r]);
        }
        tileMax = fmax(tileMax, __shfl_xor(tileMax, 16));
        tileMax = fmax(tileMax, __shfl_xor(tileMax, 32));
        const bool raise = tileMax > m + kLazyMargin; // false while the tile is all masked
        const bool rescale = raise && m != -INFINITY;
        if (__any(rescale)) {
            const double alpha = rescale ? exp(m - tileMax) : 1.0;
            double alphaO[4]; // the factors of output rows g + 4 r
#pragma unroll
            for (int r = 0; r < 4; ++r)
                alphaO[r] = __shfl(alpha, g + 4 * r);
#pragma unroll
            for (int n = 0; n < T; ++n)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    o[n][r] *= alphaO[r];
            l *= alpha;
        }
        if (raise)
            m = tileMax;
        double p[4], sum = 0.0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = live[r] ? exp(sv[r] - m) : 0.0;
            sum += p[r];
        }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        l += sum;

        // O += P V, four keys a step
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int n = 0; n < T; ++n)
                o[n] = mfma(p[st], half_at(vw[st], n), o[n]);

    }

    // the maximum and sum of output rows g + 4 r
    double mO[4], lO[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        mO[r] = __shfl(m, g + 4 * r);
        lO[r] = __shfl(l, g + 4 * r);
    }

    // merge the waves' states.  Every wave scales its sums to the rows'
    // common maximum (wave 0 holds tile 0, which every row attends, so that
    // maximum is finite; a wave whose keys a row never reached has m = -inf
    // and weighs nothing); then the waves exchange their sums kMergeTiles
    // column tiles at a time, and wave w adds the four waves' sums of its
    // rows g + 4 w in wave order and finishes those rows.
#pragma unroll
    for (int r = 0; r < 4; ++r)
        sMax[wave][r][lane] = mO[r];
    __syncthreads(); // (also: every wave is past its tiles, so sQ is free)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        double common = sMax[0][r][lane];
#pragma unroll
        for (int w = 1; w < kPaWaves; ++w)
            common = fmax(common, sMax[w][r][lane]);
        const double f = mO[r] == -INFINITY ? 0.0 : exp(mO[r] - common);
        lO[r] *= f;
#pragma unroll
        for (int n = 0; n < T; ++n)
            o[n][r] *= f;
        sSum[wave][r][lane] = lO[r];
    }
    double mine[T]; // the four waves' sums of row g + 4 wave, column tile n
#pragma unroll
    for (int n0 = 0; n0 < T; n0 += kMergeTiles) {
        if (n0 > 0)
            __syncthreads(); // the previous tiles have been read
#pragma unroll
        for (int n = 0; n < kMergeTiles; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                sPart[wave][n][r][lane] = o[n0 + n][r];
        __syncthreads();
#pragma unroll
        for (int n = 0; n < kMergeTiles; ++n) {
            double v = sPart[0][n][wave][lane];
#pragma unroll
            for (int w = 1; w < kPaWaves; ++w)
                v += sPart[w][n][wave][lane];
            mine[n0 + n] = v;
        }
    }
    double total = sSum[0][wave][lane];
#pragma unroll
    for (int w = 1; w < kPaWaves; ++w)
        total += sSum[w][wave][lane];

    // row g + 4 wave, channels [j T, j T + T): fp32, then Q8 per 32-block
    // (kBlockLanes neighbouring lanes a block)
    {
        const int row = g + 4 * wave;
        const bool live = row < rowsHere;
        const int64_t at = (int64_t) (r0 + min(row, rowsHere - 1)) * qWidth + h * HD + j * T;
        float v[T];
        float amax = 0.f;
#pragma unroll
        for (int n = 0; n < T; ++n) {
            v[n] = (float) (mine[n] / total);
            amax = fmaxf(amax, fabsf(v[n]));
        }
        if (a.out && live) {
#pragma unroll
            for (int n = 0; n < T; n += 4)
                *reinterpret_cast<float4 *>(a.out + at + n) = float4{v[n], v[n + 1], v[n + 2], v[n + 3]};
        }
        if (a.q8) {
#pragma unroll
            for (int mask = 1; mask < kBlockLanes; mask <<= 1)
                amax = fmaxf(amax, __shfl_xor(amax, mask));
            const uint16_t bits = scale_bits_from_amax(amax);
            const float sc = half_value(bits);
            const float inv = bits ? quantize_hint(sc) : 0.f;
            uint32_t packed[T / 4];
#pragma unroll
            for (int i = 0; i < T / 4; ++i) {
                uint32_t word = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int qv = quantize_in_block(v[4 * i + b], bits, sc, inv);
                    word |= (uint32_t) (uint8_t) (int8_t) qv << (8 * b);
                }
                packed[i] = word;
            }
            if (live) {
                if constexpr (T == 16)
                    *reinterpret_cast<uint4 *>(a.q8 + at) = uint4{packed[0], packed[1], packed[2], packed[3]};
                else if constexpr (T == 8)
                    *reinterpret_cast<uint2 *>(a.q8 + at) = uint2{packed[0], packed[1]};
                else
                    *reinterpret_cast<uint32_t *>(a.q8 + at) = packed[0];
                if (j % kBlockLanes == 0)
                    reinterpret_cast<uint16_t *>(a.q8 + (int64_t) a.rows * qWidth)[at / kBlock] = bits;
            }
        }
    }
}

} // namespace

bool prefill_attention_supported(int head_dim, const float *queries, int q_stride,
                                 const uint16_t *key_cache, const uint16_t *value_cache,
                                 const float *out, const uint8_t *q8)
{
    auto aligned = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && q_stride % 4 == 0
           && aligned(queries) && aligned(key_cache) && aligned(value_cache) && aligned(out)
           && aligned(q8);
}

hipError_t launch_prefill_attention(const float *queries, int q_stride, const uint16_t *key_cache,
                                    const uint16_t *value_cache, int heads, int kv_heads,
                                    int head_dim, int rows, const int *pos_ptr, int pos_value,
                                    float scale, float *out, uint8_t *q8, hipStream_t stream)
{
    if (rows <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0
        || !prefill_attention_supported(head_dim, queries, q_stride, key_cache, value_cache, out, q8)
        || q_stride < heads * head_dim)
        return hipErrorInvalidValue;
    PrefillArgs a{queries, q_stride, key_cache, value_cache, heads, kv_heads, head_dim, rows,
                  pos_ptr, pos_value, scale, out, q8};
    const dim3 grid((unsigned) ((rows + kPaRows - 1) / kPaRows * heads));
    switch (head_dim) {
    case 256:
        hipLaunchKernelGGL(prefill_attention_kernel<64>, grid, dim3(kPaThreads), 0, stream, a);
        break;
    case 128:
        hipLaunchKernelGGL(prefill_attention_kernel<32>, grid, dim3(kPaThreads), 0, stream, a);
        break;
    default:
        hipLaunchKernelGGL(prefill_attention_kernel<16>, grid, dim3(kPaThreads), 0, stream, a);
        break;
    }
    return hipGetLastError();
}

} // namespace gq8
