// gq8_kernels.hip -- hand-written gfx950 kernels of the Gemma-2B Int8Blocks
// token loop.  Wave64 throughout; 256-thread workgroups (four waves).
//
// Reference counterparts (Lib/HuggingFaceEACP/Kernels/): Embed.h,
// RMSNorm.h, RoPE.h, Linear.h / TiledMatMul.h (the products),
// MultiQueryAttention.h, GeGLU.h, Argmax.h.  The arithmetic rule shared with
// the CPU oracle is in gq8_numerics.hpp.
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"

#include <algorithm>
#include <cfloat>

namespace gq8 {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kUnchosen = 0xFFFFFFFFu; // Argmax.h:45

__device__ inline float group32_amax(float a)
{
    // fmaxf returns the other operand for a NaN, as std::max(largest, |x|)
    // keeps `largest` (Int8Blocks.cpp:118-119).
    for (int mask = 16; mask >= 1; mask >>= 1)
        a = fmaxf(a, __shfl_xor(a, mask));
    return a;
}

// One element of a 32-element block held by 32 consecutive lanes: the block's
// scale from the group's largest magnitude, the element's byte, and (lane 0
// of the group) the scale's fp16 bits.
__device__ inline void quantize_in_group(float value, int lane32, uint8_t *byte,
                                         uint16_t *scaleSlot)
{
    const float amax = group32_amax(fabsf(value));
    const uint16_t bits = scale_bits_from_amax(amax);
    int q = 0;
    if (bits != 0) {
        const float scale = half_value(bits);
        q = quantize_value(value, scale, 1.0f / scale);
    }
    *byte = (uint8_t) (int8_t) q;
    if (lane32 == 0)
        *scaleSlot = bits;
}

__device__ inline double wave_sum(double v)
{
    for (int mask = 32; mask >= 1; mask >>= 1)
        v += __shfl_xor(v, mask);
    return v;
}

__device__ inline double wave_max(double v)
{
    for (int mask = 32; mask >= 1; mask >>= 1)
        v = fmax(v, __shfl_xor(v, mask));
    return v;
}

// ---- quantization of fp32 rows --------------------------------------------
__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(const float *__restrict__ x,
                                                                 int64_t elements,
                                                                 uint8_t *__restrict__ q,
                                                                 uint16_t *__restrict__ scales)
{
    const int64_t i = (int64_t) blockIdx.x * kThreads + threadIdx.x;
    if (i >= elements) // elements is a whole number of 32-blocks: groups leave together
        return;
    quantize_in_group(x[i], threadIdx.x & 31, q + i, scales + i / kBlock);
}

// ---- embedding gather (Embed.h:45-82) ------------------------------------
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint32_t *__restrict__ tokens,
                                                         const int *pos_ptr,
                                                         const uint8_t *__restrict__ table,
                                                         int64_t vocab, int width, float scale,
                                                         float *__restrict__ out)
{
    const int row = blockIdx.y;
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= width)
        return;
    const int base = pos_ptr ? *pos_ptr : 0;
    uint32_t token = tokens[base + row];
    if (token >= (uint32_t) vocab) // ids are validated on the host; a guard, not a rule
        token = 0;
    const int64_t e = (int64_t) token * width + c;
    const int64_t elements = vocab * width;
    const uint16_t bits = reinterpret_cast<const uint16_t *>(table + elements)[e / kBlock];
    const float gathered = half_value(bits) * (float) (int8_t) table[e];
    out[(int64_t) row * width + c] = (float) ((double) scale * (double) gathered);
}

// ---- RMSNorm, optionally fused with the activation quantization ---------
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ weight,
                                                           int rows, int width, float epsilon,
                                                           float *__restrict__ y,
                                                           uint8_t *__restrict__ q8)
{
    __shared__ double partial[kThreads / 64];
    const int row = blockIdx.x;
    const float *xr = x + (int64_t) row * width;

    double squares = 0.0;
    for (int i = threadIdx.x; i < width; i += kThreads) {
        const double v = (double) xr[i];
        squares += v * v; // the square is exact in double
    }
    squares = wave_sum(squares);
    if ((threadIdx.x & 63) == 0)
        partial[threadIdx.x >> 6] = squares;
    __syncthreads();
    double total = 0.0;
    for (int w = 0; w < kThreads / 64; ++w)
        total += partial[w];
    const double scale = norm_scale(total, width, epsilon);

    const int64_t elements = (int64_t) rows * width;
    for (int i = threadIdx.x; i < width; i += kThreads) {
        const int64_t at = (int64_t) row * width + i;
        const float v = norm_value(xr[i], scale, weight[i]);
        if (y)
            y[at] = v;
        if (q8)
            quantize_in_group(v, threadIdx.x & 31, q8 + at,
                              reinterpret_cast<uint16_t *>(q8 + elements) + at / kBlock);
    }
}

// ---- RoPE (RoPE.h:50-94) ------------------------------------------------------
__global__ __launch_bounds__(kThreads) void rope_kernel(float *__restrict__ x, int row_stride,
                                                        int heads, int head_dim,
                                                        const int *pos_ptr, int pos_value,
                                                        const float *__restrict__ cosines,
                                                        const float *__restrict__ sines)
{
    const int row = blockIdx.x;
    const int half = head_dim / 2;
    const int position = (pos_ptr ? *pos_ptr : 0) + pos_value + row;
    for (int idx = threadIdx.x; idx < heads * half; idx += kThreads) {
        const int head = idx / half, pair = idx % half;
        float *base = x + (int64_t) row * row_stride + head * head_dim;
        const int64_t angle = (int64_t) position * half + pair;
        float lo, hi;
        rotate_pair(base[pair], base[pair + half], cosines[angle], sines[angle], &lo, &hi);
        base[pair] = lo;
        base[pair + half] = hi;
    }
}

// The step's q|k|v rows: q rotated in place, k rotated and stored fp16 in the
// key cache, v stored fp16 in the value cache (Decoder.cpp:459-548).
__global__ __launch_bounds__(kThreads) void rope_kv_kernel(
    float *__restrict__ qkv, int qkv_stride, int heads, int kv_heads, int head_dim,
    const int *pos_ptr, int pos_value, const float *__restrict__ cosines,
    const float *__restrict__ sines, uint16_t *__restrict__ key_cache,
    uint16_t *__restrict__ value_cache)
{
    const int row = blockIdx.x;
    const int half = head_dim / 2;
    const int qWidth = heads * head_dim, kvWidth = kv_heads * head_dim;
    const int position = (pos_ptr ? *pos_ptr : 0) + pos_value + row;
    float *r = qkv + (int64_t) row * qkv_stride;
    uint16_t *keys = key_cache + (int64_t) position * kvWidth;
    uint16_t *values = value_cache + (int64_t) position * kvWidth;

    for (int idx = threadIdx.x; idx < (heads + kv_heads) * half; idx += kThreads) {
        const int head = idx / half, pair = idx % half;
        const int64_t angle = (int64_t) position * half + pair;
        if (head < heads) {
            float *base = r + head * head_dim;
            float lo, hi;
            rotate_pair(base[pair], base[pair + half], cosines[angle], sines[angle], &lo, &hi);
            base[pair] = lo;
            base[pair + half] = hi;
        } else {
            const int kvHead = head - heads;
            const float *base = r + qWidth + kvHead * head_dim;
            float lo, hi;
            rotate_pair(base[pair], base[pair + half], cosines[angle], sines[angle], &lo, &hi);
            keys[kvHead * head_dim + pair] = half_bits(lo);
            keys[kvHead * head_dim + pair + half] = half_bits(hi);
        }
    }
    for (int i = threadIdx.x; i < kvWidth; i += kThreads)
        values[i] = half_bits(r[qWidth + kvWidth + i]);
}

__global__ __launch_bounds__(kThreads) void kv_store_kernel(const float *__restrict__ k,
                                                            const float *__restrict__ v,
                                                            int src_stride, int kv_width,
                                                            uint16_t *__restrict__ key_cache,
                                                            uint16_t *__restrict__ value_cache,
                                                            const int *pos_ptr, int pos_value)
{
    const int row = blockIdx.x;
    const int position = (pos_ptr ? *pos_ptr : 0) + pos_value + row;
    for (int i = threadIdx.x; i < kv_width; i += kThreads) {
        key_cache[(int64_t) position * kv_width + i] = half_bits(k[(int64_t) row * src_stride + i]);
        value_cache[(int64_t) position * kv_width + i] =
            half_bits(v[(int64_t) row * src_stride + i]);
    }
}

// ---- the Q8 x Q8 product ------------------------------------------------------
// y[r, o] = sum_b scale_w[o, b] * scale_x[r, b] * dot8(w[o, b], x[r, b]).
// Lane l of a wave owns the 32-element blocks l, l + 64, ... of an output row
// (32 weight bytes = two 16-byte loads, one fp16 scale), dots them against
// the same blocks of up to B activation rows staged in LDS with sdot4, and
// accumulates scale * dot in double.  Each wave owns U consecutive output
// rows; a workgroup (four waves) loops over the activation rows in groups of
// B, so a multi-row step reads every weight row from HBM once.
template <int B, int U>
__global__ __launch_bounds__(kThreads) void q8_product_kernel(
    const uint8_t *__restrict__ x8, int64_t x_elements, int x_row0, int rows,
    const uint8_t *__restrict__ w8, int inner, int outputs, float *__restrict__ y, int y_stride,
    int residual)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const int nb = inner / kBlock;
    int8_t *sQ = reinterpret_cast<int8_t *>(smem);
    double *sScale = reinterpret_cast<double *>(smem + (size_t) B * inner);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t wElements = (int64_t) outputs * inner;
    const uint16_t *wScales = reinterpret_cast<const uint16_t *>(w8 + wElements);
    const uint16_t *xScales = reinterpret_cast<const uint16_t *>(x8 + x_elements);
    const int out0 = (blockIdx.x * (kThreads / 64) + wave) * U;

    for (int g = 0; g < rows; g += B) {
        const int gb = min(B, rows - g);
        __syncthreads();
        const int vecs = inner / 16;
        for (int idx = threadIdx.x; idx < gb * vecs; idx += kThreads) {
            const int b = idx / vecs, v = idx % vecs;
            reinterpret_cast<int4 *>(sQ)[b * vecs + v] =
                reinterpret_cast<const int4 *>(x8 + (int64_t) (x_row0 + g + b) * inner)[v];
        }
        for (int idx = threadIdx.x; idx < gb * nb; idx += kThreads) {
            const int b = idx / nb, j = idx % nb;
            sScale[b * nb + j] = (double) half_value(xScales[(int64_t) (x_row0 + g + b) * nb + j]);
        }
        __syncthreads();

        double acc[U][B];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int b = 0; b < B; ++b)
                acc[u][b] = 0.0;

        for (int blk = lane; blk < nb; blk += 64) {
            int4 wa[U], wb[U];
            double ws[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int o = out0 + u;
                if (o < outputs) {
                    const int4 *p = reinterpret_cast<const int4 *>(w8 + (int64_t) o * inner
                                                                   + (int64_t) blk * kBlock);
                    wa[u] = p[0];
                    wb[u] = p[1];
                    ws[u] = (double) half_value(wScales[(int64_t) o * nb + blk]);
                } else {
                    wa[u] = make_int4(0, 0, 0, 0);
                    wb[u] = make_int4(0, 0, 0, 0);
                    ws[u] = 0.0;
                }
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                if (b < gb) {
                    const int4 *ap = reinterpret_cast<const int4 *>(sQ + b * inner + blk * kBlock);
                    const int4 a0 = ap[0], a1 = ap[1];
                    const double sa = sScale[b * nb + blk];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        int d = 0;
                        d = __builtin_amdgcn_sdot4(wa[u].x, a0.x, d, false);
                        d = __builtin_amdgcn_sdot4(wa[u].y, a0.y, d, false);
                        d = __builtin_amdgcn_sdot4(wa[u].z, a0.z, d, false);
                        d = __builtin_amdgcn_sdot4(wa[u].w, a0.w, d, false);
                        d = __builtin_amdgcn_sdot4(wb[u].x, a1.x, d, false);
                        d = __builtin_amdgcn_sdot4(wb[u].y, a1.y, d, false);
                        d = __builtin_amdgcn_sdot4(wb[u].z, a1.z, d, false);
                        d = __builtin_amdgcn_sdot4(wb[u].w, a1.w, d, false);
                        acc[u][b] += (double) d * (ws[u] * sa); // all three exact but the sum
                    }
                }
            }
        }

#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const double total = wave_sum(acc[u][b]);
                const int o = out0 + u;
                if (lane == 0 && b < gb && o < outputs) {
                    float *dst = y + (int64_t) (g + b) * y_stride + o;
                    const double old = residual ? (double) *dst : 0.0;
                    *dst = (float) (total + old);
                }
            }
        }
    }
}

// ---- multi-query attention, split over 64-key chunks ----------------------
// Partial: one workgroup per (chunk, query row) holds every head; scores in
// double (sequential over channels, as the oracle sums them), the chunk's
// maximum and exp-sum per head, and the chunk's unnormalised value sums.
constexpr int kChunk = kAttentionChunk;
constexpr int kMaxQueryWidth = 2048;
constexpr int kMaxKvWidth = 256;

__global__ __launch_bounds__(kThreads) void mqa_partial_kernel(
    const float *__restrict__ queries, int q_stride, const uint16_t *__restrict__ key_cache,
    const uint16_t *__restrict__ value_cache, int heads, int kv_heads, int head_dim,
    const int *pos_ptr, int pos_value, float scale, int chunks_cap, double *__restrict__ ws_o,
    double *__restrict__ ws_ml)
{
    __shared__ double sQuery[kMaxQueryWidth];
    __shared__ uint32_t sKeys[kChunk * (kMaxKvWidth / 2 + 1)];
    __shared__ double sWeights[kMaxHeads * kChunk];

    const int chunk = blockIdx.x, row = blockIdx.y;
    const int keyCount = (pos_ptr ? *pos_ptr : 0) + pos_value + row + 1;
    const int k0 = chunk * kChunk;
    if (k0 >= keyCount)
        return;
    const int nkeys = min(kChunk, keyCount - k0);
    const int qWidth = heads * head_dim, kvWidth = kv_heads * head_dim;
    const int perKv = heads / kv_heads;
    const int keyWords = kvWidth / 2, keyStride = kMaxKvWidth / 2 + 1;

    for (int i = threadIdx.x; i < qWidth; i += kThreads)
        sQuery[i] = (double) queries[(int64_t) row * q_stride + i];
    const uint32_t *keyRows = reinterpret_cast<const uint32_t *>(key_cache + (int64_t) k0 * kvWidth);
    for (int i = threadIdx.x; i < nkeys * keyWords; i += kThreads) {
        const int j = i / keyWords, w = i % keyWords;
        sKeys[j * keyStride + w] = keyRows[(int64_t) j * keyWords + w];
    }
    __syncthreads();

    for (int idx = threadIdx.x; idx < heads * kChunk; idx += kThreads) {
        const int head = idx / kChunk, j = idx % kChunk;
        double score = -INFINITY;
        if (j < nkeys) {
            const double *q = sQuery + head * head_dim;
            const uint32_t *k = sKeys + j * keyStride + ((head / perKv) * head_dim) / 2;
            double total = 0.0;
            for (int c = 0; c < head_dim; c += 2) {
                const uint32_t pair = k[c / 2];
                total += q[c] * (double) half_value((uint16_t) (pair & 0xFFFFu));
                total += q[c + 1] * (double) half_value((uint16_t) (pair >> 16));
            }
            score = (double) scale * total;
        }
        sWeights[idx] = score;
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int head = wave; head < heads; head += kThreads / 64) {
        const double s = sWeights[head * kChunk + lane];
        const double m = wave_max(s);
        const double w = lane < nkeys ? exp(s - m) : 0.0;
        const double l = wave_sum(w);
        sWeights[head * kChunk + lane] = w;
        if (lane == 0) {
            double *ml = ws_ml + (((int64_t) row * chunks_cap + chunk) * heads + head) * 2;
            ml[0] = m;
            ml[1] = l;
        }
    }
    __syncthreads();

    double *o = ws_o + ((int64_t) row * chunks_cap + chunk) * qWidth;
    for (int idx = threadIdx.x; idx < qWidth; idx += kThreads) {
        const int head = idx / head_dim, c = idx % head_dim;
        const uint16_t *v = value_cache + (int64_t) k0 * kvWidth + (head / perKv) * head_dim + c;
        double acc = 0.0;
        for (int j = 0; j < nkeys; ++j)
            acc += sWeights[head * kChunk + j] * (double) half_value(v[(int64_t) j * kvWidth]);
        o[idx] = acc;
    }
}

// Merge: per query row, the chunks' maxima and sums rescaled to the row's
// maximum (the exact online-softmax join, MultiQueryAttention.h:43-49), the
// output divided by the total, rounded to fp32 and optionally quantized.
__global__ __launch_bounds__(kThreads) void mqa_merge_kernel(
    int heads, int head_dim, const int *pos_ptr, int pos_value, int chunks_cap,
    const double *__restrict__ ws_o, const double *__restrict__ ws_ml, float *__restrict__ out,
    uint8_t *__restrict__ q8, int rows)
{
    const int row = blockIdx.x;
    const int keyCount = (pos_ptr ? *pos_ptr : 0) + pos_value + row + 1;
    const int chunks = (keyCount + kChunk - 1) / kChunk;
    const int qWidth = heads * head_dim;
    const int64_t elements = (int64_t) rows * qWidth;

    for (int idx = threadIdx.x; idx < qWidth; idx += kThreads) {
        const int head = idx / head_dim;
        double largest = -INFINITY;
        for (int c = 0; c < chunks; ++c)
            largest = fmax(largest, ws_ml[(((int64_t) row * chunks_cap + c) * heads + head) * 2]);
        double total = 0.0, weighted = 0.0;
        for (int c = 0; c < chunks; ++c) {
            const double *ml = ws_ml + (((int64_t) row * chunks_cap + c) * heads + head) * 2;
            const double factor = exp(ml[0] - largest);
            total += ml[1] * factor;
            weighted += ws_o[((int64_t) row * chunks_cap + c) * qWidth + idx] * factor;
        }
        const float v = (float) (weighted / total);
        const int64_t at = (int64_t) row * qWidth + idx;
        if (out)
            out[at] = v;
        if (q8)
            quantize_in_group(v, threadIdx.x & 31, q8 + at,
                              reinterpret_cast<uint16_t *>(q8 + elements) + at / kBlock);
    }
}

// ---- GeGLU (GeGLU.h:50-73) ---------------------------------------------------
__global__ __launch_bounds__(kThreads) void geglu_kernel(const float *__restrict__ fused, int rows,
                                                         int intermediate,
                                                         float *__restrict__ out,
                                                         uint8_t *__restrict__ q8)
{
    const int row = blockIdx.y;
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= intermediate) // whole 32-groups only
        return;
    const float *f = fused + (int64_t) row * 2 * intermediate;
    const float v = geglu(f[i], f[intermediate + i]);
    const int64_t at = (int64_t) row * intermediate + i;
    if (out)
        out[at] = v;
    if (q8)
        quantize_in_group(v, threadIdx.x & 31, q8 + at,
                          reinterpret_cast<uint16_t *>(q8 + (int64_t) rows * intermediate)
                              + at / kBlock);
}

// ---- argmax (Argmax.h:47-200) --------------------------------------------------
struct Candidate {
    float value;
    uint32_t index;
};

__device__ inline Candidate better_of(Candidate a, Candidate b)
{
    if (b.index == kUnchosen)
        return a;
    if (a.index == kUnchosen)
        return b;
    if (b.value > a.value || (b.value == a.value && b.index < a.index))
        return b;
    return a;
}

__device__ inline Candidate fold_workgroup(Candidate c, Candidate *scratch)
{
    for (int mask = 32; mask >= 1; mask >>= 1) {
        Candidate other;
        other.value = __shfl_xor(c.value, mask);
        other.index = __shfl_xor(c.index, mask);
        c = better_of(c, other);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0)
        scratch[wave] = c;
    __syncthreads();
    Candidate best = scratch[0];
    for (int w = 1; w < kThreads / 64; ++w)
        best = better_of(best, scratch[w]);
    return best;
}

constexpr int kArgmaxPerThread = 8;

__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(
    const float *__restrict__ logits, const float *__restrict__ mask, int length,
    float *__restrict__ partValues, uint32_t *__restrict__ partIndices)
{
    __shared__ Candidate scratch[kThreads / 64];
    const int row = blockIdx.y;
    const int groups = gridDim.x;
    const float *r = logits + (int64_t) row * length;
    Candidate best{-FLT_MAX, kUnchosen};
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < length; i += groups * kThreads) {
        const float v = r[i];
        const bool allowed = mask == nullptr || mask[i] == 0.f;
        if (allowed && (best.index == kUnchosen || v > best.value)) {
            best.value = v;
            best.index = (uint32_t) i;
        }
    }
    best = fold_workgroup(best, scratch);
    if (threadIdx.x == 0) {
        partValues[(int64_t) row * groups + blockIdx.x] = best.value;
        partIndices[(int64_t) row * groups + blockIdx.x] = best.index;
    }
}

__global__ __launch_bounds__(kThreads) void argmax_final_kernel(
    const float *__restrict__ partValues, const uint32_t *__restrict__ partIndices, int groups,
    uint32_t *__restrict__ indices, const int *pos_ptr, int index_offset)
{
    __shared__ Candidate scratch[kThreads / 64];
    const int row = blockIdx.x;
    Candidate best{-FLT_MAX, kUnchosen};
    for (int j = threadIdx.x; j < groups; j += kThreads)
        best = better_of(best, Candidate{partValues[(int64_t) row * groups + j],
                                         partIndices[(int64_t) row * groups + j]});
    best = fold_workgroup(best, scratch);
    if (threadIdx.x == 0) {
        const int base = (pos_ptr ? *pos_ptr : 0) + index_offset;
        indices[base + row] = best.index == kUnchosen ? 0u : best.index;
    }
}

__global__ void advance_kernel(int *pos_ptr, int amount)
{
    if (threadIdx.x == 0 && blockIdx.x == 0)
        *pos_ptr += amount;
}

inline unsigned blocks_for(int64_t n, int per)
{
    return (unsigned) ((n + per - 1) / per);
}

int argmax_groups(int length)
{
    const int per = kThreads * kArgmaxPerThread;
    return std::max(1, (length + per - 1) / per);
}

} // namespace

// ============================================================================
// Launchers
// ============================================================================
hipError_t launch_quantize(const float *x, int64_t elements, uint8_t *q, uint16_t *scales,
                           hipStream_t stream)
{
    if (elements <= 0 || elements % kBlock != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(blocks_for(elements, kThreads)), dim3(kThreads),
                       0, stream, x, elements, q, scales);
    return hipGetLastError();
}

hipError_t launch_embed(const uint32_t *tokens, const int *pos_ptr, int rows,
                        const uint8_t *table, int vocab, int width, float scale, float *out,
                        hipStream_t stream)
{
    if (rows <= 0 || width <= 0 || width % kBlock != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_kernel, dim3(blocks_for(width, kThreads), rows), dim3(kThreads), 0,
                       stream, tokens, pos_ptr, table, (int64_t) vocab, width, scale, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *weight, int rows, int width,
                          float epsilon, float *y, uint8_t *q8, hipStream_t stream)
{
    if (rows <= 0 || width <= 0 || width % kBlock != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, weight, rows,
                       width, epsilon, y, q8);
    return hipGetLastError();
}

hipError_t launch_rope(float *x, int row_stride, int heads, int head_dim, const int *pos_ptr,
                       int pos_value, int rows, const float *cosines, const float *sines,
                       hipStream_t stream)
{
    if (rows <= 0 || heads <= 0 || head_dim <= 0 || head_dim % 2 != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_kernel, dim3(rows), dim3(kThreads), 0, stream, x, row_stride, heads,
                       head_dim, pos_ptr, pos_value, cosines, sines);
    return hipGetLastError();
}

hipError_t launch_rope_kv(float *qkv, int qkv_stride, int heads, int kv_heads, int head_dim,
                          const int *pos_ptr, int pos_value, int rows, const float *cosines,
                          const float *sines, uint16_t *key_cache, uint16_t *value_cache,
                          hipStream_t stream)
{
    if (rows <= 0 || heads <= 0 || kv_heads <= 0 || head_dim % 2 != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_kv_kernel, dim3(rows), dim3(kThreads), 0, stream, qkv, qkv_stride,
                       heads, kv_heads, head_dim, pos_ptr, pos_value, cosines, sines, key_cache,
                       value_cache);
    return hipGetLastError();
}

hipError_t launch_kv_store(const float *k, const float *v, int src_stride, int rows,
                           int kv_width, uint16_t *key_cache, uint16_t *value_cache,
                           const int *pos_ptr, int pos_value, hipStream_t stream)
{
    if (rows <= 0 || kv_width <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(kv_store_kernel, dim3(rows), dim3(kThreads), 0, stream, k, v, src_stride,
                       kv_width, key_cache, value_cache, pos_ptr, pos_value);
    return hipGetLastError();
}

namespace {
template <int B, int U>
hipError_t product_with(const uint8_t *x8, int64_t xElements, int xRow0, int rows,
                        const uint8_t *w8, int inner, int outputs, float *y, int yStride,
                        int residual, hipStream_t stream)
{
    const size_t lds = (size_t) B * inner + (size_t) B * (inner / kBlock) * sizeof(double);
    const unsigned grid = blocks_for(outputs, (kThreads / 64) * U);
    hipLaunchKernelGGL((q8_product_kernel<B, U>), dim3(grid), dim3(kThreads), lds, stream, x8,
                       xElements, xRow0, rows, w8, inner, outputs, y, yStride, residual);
    return hipGetLastError();
}

constexpr size_t kProductLdsLimit = 64 * 1024;

size_t product_lds(int b, int inner)
{
    return (size_t) b * inner + (size_t) b * (inner / kBlock) * sizeof(double);
}
} // namespace

hipError_t launch_q8_product(const uint8_t *x8, int x_rows_total, int x_row0, int rows,
                             const uint8_t *w8, int inner, int outputs, float *y, int y_stride,
                             int residual, hipStream_t stream)
{
    if (rows <= 0 || inner <= 0 || outputs <= 0 || inner % kBlock != 0 || y_stride < outputs
        || x_row0 < 0 || x_row0 + rows > x_rows_total || product_lds(1, inner) > kProductLdsLimit)
        return hipErrorInvalidValue;
    const int64_t xElements = (int64_t) x_rows_total * inner;
    int b = 8;
    while (b > 1 && (b > rows || product_lds(b, inner) > kProductLdsLimit))
        b >>= 1;
    // rows per wave: 8 for a vocabulary-wide product, 4 for the feed-forward
    // width, 1 where the matrix is too small to fill the chip otherwise
    const int perWave = inner > 4096 ? 1 : (outputs >= 131072 ? 8 : (outputs >= 16384 ? 4 : 1));
#define GQ8_PRODUCT(BB)                                                                      \
    switch (perWave) {                                                                       \
    case 8: return product_with<BB, 8>(x8, xElements, x_row0, rows, w8, inner, outputs, y,   \
                                       y_stride, residual, stream);                          \
    case 4: return product_with<BB, 4>(x8, xElements, x_row0, rows, w8, inner, outputs, y,   \
                                       y_stride, residual, stream);                          \
    default: return product_with<BB, 1>(x8, xElements, x_row0, rows, w8, inner, outputs, y,  \
                                        y_stride, residual, stream);                         \
    }
    switch (b) {
    case 8: GQ8_PRODUCT(8);
    case 4: GQ8_PRODUCT(4);
    case 2: GQ8_PRODUCT(2);
    default: GQ8_PRODUCT(1);
    }
#undef GQ8_PRODUCT
}

size_t mqa_workspace_bytes(int rows, int heads, int head_dim, int max_keys)
{
    const int64_t chunks = (max_keys + kChunk - 1) / kChunk;
    const int64_t qWidth = (int64_t) heads * head_dim;
    return (size_t) (rows * chunks * qWidth + rows * chunks * heads * 2) * sizeof(double);
}

hipError_t launch_mqa(const float *queries, int q_stride, const uint16_t *key_cache,
                      const uint16_t *value_cache, int heads, int kv_heads, int head_dim,
                      int rows, const int *pos_ptr, int pos_value, int max_keys, float scale,
                      float *out, uint8_t *q8, void *workspace, size_t workspace_bytes,
                      hipStream_t stream)
{
    if (rows <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || heads > kMaxHeads
        || head_dim % 2 != 0 || heads * head_dim > kMaxQueryWidth
        || kv_heads * head_dim > kMaxKvWidth || max_keys <= 0
        || workspace_bytes < mqa_workspace_bytes(rows, heads, head_dim, max_keys))
        return hipErrorInvalidValue;
    if (q8 && (heads * head_dim) % kBlock != 0)
        return hipErrorInvalidValue;
    const int chunksCap = (max_keys + kChunk - 1) / kChunk;
    double *wsO = reinterpret_cast<double *>(workspace);
    double *wsMl = wsO + (int64_t) rows * chunksCap * heads * head_dim;
    hipLaunchKernelGGL(mqa_partial_kernel, dim3(chunksCap, rows), dim3(kThreads), 0, stream,
                       queries, q_stride, key_cache, value_cache, heads, kv_heads, head_dim,
                       pos_ptr, pos_value, scale, chunksCap, wsO, wsMl);
    hipError_t status = hipGetLastError();
    if (status != hipSuccess)
        return status;
    hipLaunchKernelGGL(mqa_merge_kernel, dim3(rows), dim3(kThreads), 0, stream, heads, head_dim,
                       pos_ptr, pos_value, chunksCap, wsO, wsMl, out, q8, rows);
    return hipGetLastError();
}

hipError_t launch_geglu(const float *fused, int rows, int intermediate, float *out,
                        uint8_t *q8, hipStream_t stream)
{
    if (rows <= 0 || intermediate <= 0 || intermediate % kBlock != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(geglu_kernel, dim3(blocks_for(intermediate, kThreads), rows),
                       dim3(kThreads), 0, stream, fused, rows, intermediate, out, q8);
    return hipGetLastError();
}

size_t argmax_workspace_bytes(int rows, int length)
{
    return (size_t) rows * argmax_groups(length) * (sizeof(float) + sizeof(uint32_t));
}

hipError_t launch_argmax(const float *logits, const float *mask, int rows, int length,
                         uint32_t *indices, const int *pos_ptr, int index_offset,
                         void *workspace, size_t workspace_bytes, hipStream_t stream)
{
    if (rows <= 0 || length <= 0 || workspace_bytes < argmax_workspace_bytes(rows, length))
        return hipErrorInvalidValue;
    const int groups = argmax_groups(length);
    float *values = reinterpret_cast<float *>(workspace);
    uint32_t *idx = reinterpret_cast<uint32_t *>(values + (int64_t) rows * groups);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(groups, rows), dim3(kThreads), 0, stream,
                       logits, mask, length, values, idx);
    hipError_t status = hipGetLastError();
    if (status != hipSuccess)
        return status;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(kThreads), 0, stream, values, idx,
                       groups, indices, pos_ptr, index_offset);
    return hipGetLastError();
}

hipError_t launch_advance(int *pos_ptr, int amount, hipStream_t stream)
{
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, stream, pos_ptr, amount);
    return hipGetLastError();
}

} // namespace gq8
