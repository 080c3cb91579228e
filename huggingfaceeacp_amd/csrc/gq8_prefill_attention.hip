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
// waves take the key tiles (16 keys) round robin and each keeps an online
// softmax state (row maximum, sum and the 16 x head_dim sums); the states are
// merged in LDS at the end.  Per tile a wave computes S = Q K^T with
// v_mfma_f64_16x16x4f64 (the query in registers as fp32, the keys straight
// from the fp16 cache), rescales, and adds P V with the same instruction.
//
// fp64 MFMA operand layout (checked on gfx950): A 16 x 4 with lane l holding
// A[l % 16][l / 16]; B 4 x 16 with lane l holding B[l / 16][l % 16]; D 16 x 16
// with lane l holding D[l / 16 + 4 r][l % 16], r = 0..3.  For S the reduction
// index is the channel, mapped so that lane group g = l / 16 supplies the
// channels [g E, g E + E) (E = head_dim / 4) over the steps: a lane reads its
// E channels of a query row and of a key row contiguously.
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"

namespace gq8 {
namespace {

typedef double v4d __attribute__((ext_vector_type(4)));

constexpr int kPaRows = 16;   // query rows a workgroup
constexpr int kPaWaves = 4;
constexpr int kPaThreads = kPaWaves * 64;
constexpr int kPaKeys = 16;   // keys a tile

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

__device__ inline double shfl_xor_d(double v, int mask)
{
    return __shfl_xor(v, mask);
}

// E channels a lane group, T = head_dim / 16 output column tiles.
template <int E>
__global__ __launch_bounds__(kPaThreads) void prefill_attention_kernel(PrefillArgs a)
{
    constexpr int HD = 4 * E, T = HD / 16;
    // the P tile of each wave (its rows on l % 16 for the P V product), and
    // one wave's state at a time for the merge
    __shared__ double sP[kPaWaves][kPaRows][kPaKeys + 1];
    __shared__ double sState[64][T * 4 + 8 + 1];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, j = lane & 15;
    const int r0 = blockIdx.x * kPaRows, h = blockIdx.y;
    const int qWidth = a.heads * HD, kvWidth = a.kv_heads * HD;
    const int kvh = h / (a.heads / a.kv_heads);
    const int base = (a.pos_ptr ? *a.pos_ptr : 0) + a.pos_value;
    const int rowsHere = min(kPaRows, a.rows - r0);
    const int lastKey = base + r0 + rowsHere - 1;  // the block's last row attends [0, lastKey]
    const int tiles = lastKey / kPaKeys + 1;

    // this lane's query channels: row r0 + j (clamped), channels [g E, g E + E)
    float q[E];
    {
        const float *src = a.queries + (int64_t) (r0 + min(j, rowsHere - 1)) * a.q_stride + h * HD + g * E;
#pragma unroll
        for (int c = 0; c < E; c += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(src + c);
            q[c] = v.x; q[c + 1] = v.y; q[c + 2] = v.z; q[c + 3] = v.w;
        }
    }
    // the rows this lane holds in S and O layouts: g + 4 r, at positions
    int rowPos[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        rowPos[r] = base + r0 + g + 4 * r;

    double m[4], l[4];
    v4d o[T];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.0;
    }
#pragma unroll
    for (int n = 0; n < T; ++n)
        o[n] = v4d{0.0, 0.0, 0.0, 0.0};

    const uint16_t *keys = a.key_cache + kvh * HD;
    const uint16_t *values = a.value_cache + kvh * HD;
    for (int tile = wave; tile < tiles; tile += kPaWaves) {
        const int k0 = tile * kPaKeys;
        // S = Q K^T: lane (g, j) supplies K[k0 + j][g E + c] (a B element)
        uint16_t kh[E];
        {
            const int key = min(k0 + j, lastKey);
            const uint16_t *src = keys + (int64_t) key * kvWidth + g * E;
#pragma unroll
            for (int c = 0; c < E; c += 8) {
                const uint4 v = *reinterpret_cast<const uint4 *>(src + c);
                kh[c] = (uint16_t) (v.x & 0xFFFFu); kh[c + 1] = (uint16_t) (v.x >> 16);
                kh[c + 2] = (uint16_t) (v.y & 0xFFFFu); kh[c + 3] = (uint16_t) (v.y >> 16);
                kh[c + 4] = (uint16_t) (v.z & 0xFFFFu); kh[c + 5] = (uint16_t) (v.z >> 16);
                kh[c + 6] = (uint16_t) (v.w & 0xFFFFu); kh[c + 7] = (uint16_t) (v.w >> 16);
            }
        }
        v4d s = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int c = 0; c < E; ++c)
            s = mfma((double) q[c], (double) half_value(kh[c]), s);

        // online softmax over this tile: row g + 4 r, key k0 + j
        double p[4], alpha[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool live = k0 + j <= rowPos[r];
            const double score = live ? (double) a.scale * s[r] : -INFINITY;
            double tileMax = score;
            for (int mask = 1; mask < 16; mask <<= 1)
                tileMax = fmax(tileMax, shfl_xor_d(tileMax, mask));
            const double newMax = fmax(m[r], tileMax);
            alpha[r] = newMax == -INFINITY ? 1.0 : exp(m[r] - newMax);
            p[r] = live ? exp(score - newMax) : 0.0;
            double sum = p[r];
            for (int mask = 1; mask < 16; mask <<= 1)
                sum += shfl_xor_d(sum, mask);
            l[r] = l[r] * alpha[r] + sum;
            m[r] = newMax;
        }
#pragma unroll
        for (int n = 0; n < T; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                o[n][r] *= alpha[r];
        // P to LDS with its rows on l % 16 for the A operand
#pragma unroll
        for (int r = 0; r < 4; ++r)
            sP[wave][g + 4 * r][j] = p[r];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        double pa[4];
#pragma unroll
        for (int st = 0; st < 4; ++st)
            pa[st] = sP[wave][j][4 * st + g]; // A[row j][key 4 st + g]
        // O += P V: lane (g, j) supplies V[k0 + 4 st + g][16 n + j]
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int key = min(k0 + 4 * st + g, lastKey);
            const uint16_t *vrow = values + (int64_t) key * kvWidth + j;
#pragma unroll
            for (int n = 0; n < T; ++n)
                o[n] = mfma(pa[st], (double) half_value(vrow[16 * n]), o[n]);
        }
        __builtin_amdgcn_wave_barrier(); // sP is rewritten by the next tile
    }

    // merge the waves' states into wave 0, one wave at a time
    for (int w = 1; w < kPaWaves; ++w) {
        __syncthreads();
        if (wave == w) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sState[lane][T * 4 + r] = m[r];
                sState[lane][T * 4 + 4 + r] = l[r];
            }
#pragma unroll
            for (int n = 0; n < T; ++n)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sState[lane][n * 4 + r] = o[n][r];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const double om = sState[lane][T * 4 + r], ol = sState[lane][T * 4 + 4 + r];
                const double newMax = fmax(m[r], om);
                const double fa = newMax == -INFINITY ? 0.0 : exp(m[r] - newMax);
                const double fb = newMax == -INFINITY ? 0.0 : exp(om - newMax);
                l[r] = l[r] * fa + ol * fb;
                m[r] = newMax;
#pragma unroll
                for (int n = 0; n < T; ++n)
                    o[n][r] = o[n][r] * fa + sState[lane][n * 4 + r] * fb;
            }
        }
    }
    if (wave != 0)
        return;

    // rows g + 4 r, channels 16 n + j: fp32, then Q8 per 32-block (tiles 2b, 2b + 1)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = g + 4 * r;
        const bool live = row < rowsHere;
        const int64_t rowBase = (int64_t) (r0 + min(row, rowsHere - 1)) * qWidth + h * HD;
#pragma unroll
        for (int b = 0; b < T / 2; ++b) {
            const float v0 = (float) (o[2 * b][r] / l[r]);
            const float v1 = (float) (o[2 * b + 1][r] / l[r]);
            if (a.out && live) {
                a.out[rowBase + 32 * b + j] = v0;
                a.out[rowBase + 32 * b + 16 + j] = v1;
            }
            float amax = fmaxf(fabsf(v0), fabsf(v1));
            for (int mask = 1; mask < 16; mask <<= 1)
                amax = fmaxf(amax, __shfl_xor(amax, mask));
            if (a.q8 && live) {
                const uint16_t bits = scale_bits_from_amax(amax);
                const float sc = half_value(bits);
                const float inv = bits ? quantize_hint(sc) : 0.f;
                a.q8[rowBase + 32 * b + j] = (uint8_t) (int8_t) (bits ? quantize_value(v0, sc, inv) : 0);
                a.q8[rowBase + 32 * b + 16 + j] =
                    (uint8_t) (int8_t) (bits ? quantize_value(v1, sc, inv) : 0);
                if (j == 0)
                    reinterpret_cast<uint16_t *>(a.q8 + (int64_t) a.rows * qWidth)[(rowBase + 32 * b) / kBlock] = bits;
            }
        }
    }
}

} // namespace

bool prefill_attention_supported(int head_dim)
{
    return head_dim == 64 || head_dim == 128 || head_dim == 256;
}

hipError_t launch_prefill_attention(const float *queries, int q_stride, const uint16_t *key_cache,
                                    const uint16_t *value_cache, int heads, int kv_heads,
                                    int head_dim, int rows, const int *pos_ptr, int pos_value,
                                    float scale, float *out, uint8_t *q8, hipStream_t stream)
{
    if (rows <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0
        || !prefill_attention_supported(head_dim) || q_stride < heads * head_dim)
        return hipErrorInvalidValue;
    PrefillArgs a{queries, q_stride, key_cache, value_cache, heads, kv_heads, head_dim, rows,
                  pos_ptr, pos_value, scale, out, q8};
    const dim3 grid((rows + kPaRows - 1) / kPaRows, heads);
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
