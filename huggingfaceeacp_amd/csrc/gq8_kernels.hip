// gq8_kernels.hip -- hand-written gfx950 kernels of the Gemma-2B Int8Blocks
// token loop.  Wave64 throughout; 256-thread workgroups (four waves).
//
// Reference counterparts (Lib/HuggingFaceEACP/Kernels/): Embed.h,
// RMSNorm.h, RoPE.h, Linear.h / TiledMatMul.h (the products),
// MultiQueryAttention.h, GeGLU.h, Argmax.h.  The arithmetic rule shared with
// the CPU oracle is in gq8_numerics.hpp.
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"
#include "gq8_lanes.hpp"

#include <algorithm>
#include <cfloat>

namespace gq8 {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kUnchosen = 0xFFFFFFFFu; // Argmax.h:45

// The largest magnitude of a 32-lane group (lanes 32 g .. 32 g + 31); lanes
// of the wave outside the group may be inactive.  fmaxf returns the other
// operand for a NaN, as std::max(largest, |x|) keeps `largest`
// (Int8Blocks.cpp:29-30).
__device__ inline float group32_amax(float a)
{
    for (int mask = 16; mask >= 1; mask >>= 1)
        a = fmaxf(a, __shfl_xor(a, mask));
    return a;
}

// One element of a 32-element block held by 32 consecutive lanes: the block's
// scale from the group's largest magnitude, the element's byte, and (lane 0
// of the group) the scale's fp16 bits.  Without branches, so a thread's
// elements interleave.
__device__ inline void quantize_in_group(float value, int lane32, uint8_t *byte,
                                         uint16_t *scaleSlot)
{
    const float amax = group32_amax(fabsf(value));
    const uint16_t bits = scale_bits_from_amax(amax);
    const float scale = half_value(bits);
    *byte = (uint8_t) (int8_t) quantize_in_block(value, bits, scale, quantize_hint(scale));
    if (lane32 == 0)
        *scaleSlot = bits;
}

// whole-wave butterflies (every caller is a whole wave)
__device__ inline double wave_sum(double v)
{
    return sum_lanes<32>(v);
}

__device__ inline double wave_max(double v)
{
    return max_lanes<32>(v);
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
// Row r embeds tokens[*pos_ptr + r] (one sequence), or with row_positions
// tokens[r * slot_stride + row_positions[r]] (row r of a lockstep batch, each
// sequence's slots slot_stride apart).  With row_angles, the first workgroup
// of row r also copies the RoPE table rows of its position (RoPE.cpp:7-34):
// cosines to row_angles[2 r half ..], sines to row_angles[(2 r + 1) half ..].
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint32_t *__restrict__ tokens,
                                                         const int *pos_ptr,
                                                         const int *row_positions,
                                                         int64_t slot_stride,
                                                         const uint8_t *__restrict__ table,
                                                         int64_t vocab, int width, float scale,
                                                         float *__restrict__ out,
                                                         const float *__restrict__ cosines,
                                                         const float *__restrict__ sines, int half,
                                                         float *__restrict__ row_angles)
{
    const int row = blockIdx.y;
    if (row_angles && blockIdx.x == 0 && (int) threadIdx.x < 2 * half) {
        const int i = threadIdx.x % half;
        const int64_t angle = (int64_t) row_positions[row] * half + i;
        row_angles[(int64_t) row * 2 * half + threadIdx.x] =
            (int) threadIdx.x < half ? cosines[angle] : sines[angle];
    }
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= width)
        return;
    const int64_t slot = row_positions ? row * slot_stride + row_positions[row]
                                       : (int64_t) (pos_ptr ? *pos_ptr : 0) + row;
    uint32_t token = tokens[slot];
    if (token >= (uint32_t) vocab) // ids are validated on the host; a guard, not a rule
        token = 0;
    const int64_t e = (int64_t) token * width + c;
    const int64_t elements = vocab * width;
    const uint16_t bits = reinterpret_cast<const uint16_t *>(table + elements)[e / kBlock];
    const float gathered = half_value(bits) * (float) (int8_t) table[e];
    out[(int64_t) row * width + c] = (float) ((double) scale * (double) gathered);
}

// ---- RMSNorm, optionally fused with the activation quantization ---------
// The normalized element i of a row and its Int8Blocks byte and block scale
// (lane 0 of its 32-lane group stores the scale).  The whole wave is active:
// the group's largest magnitude is the DPP form of group32_amax, same pairing.
__device__ inline void norm_store(float x, float w, double scale, int64_t at, bool live,
                                  int64_t elements, float *__restrict__ y, uint8_t *__restrict__ q8)
{
    const float v = norm_value(x, scale, w);
    const float amax = max_lanes<16>(fabsf(v));
    const uint16_t bits = scale_bits_from_amax(amax);
    const float sc = half_value(bits);
    const int byte = quantize_in_block(v, bits, sc, quantize_hint(sc));
    if (!live)
        return;
    if (y)
        y[at] = v;
    if (q8) {
        q8[at] = (uint8_t) (int8_t) byte;
        if ((threadIdx.x & 31) == 0)
            reinterpret_cast<uint16_t *>(q8 + elements)[at / kBlock] = bits;
    }
}

// K: elements a thread holds (the row's width rounded up to K x kThreads),
// loaded at once, or 0: rows of any width, streamed from memory twice.  Every
// lane of a wave takes part in the group reductions (elements past the width
// are computed from a clamped index and not stored).  P > 1 (K > 0): the row
// is P workgroups (blockIdx.y); each sums the squares of the whole row and
// normalizes its K / P elements a thread, so a few rows fill more of the
// chip and each thread's chain is shorter.
template <int K, int P>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ weight,
                                                           int rows, int width, float epsilon,
                                                           float *__restrict__ y,
                                                           uint8_t *__restrict__ q8)
{
    __shared__ double partial[kThreads / 64];
    const int row = blockIdx.x;
    const float *xr = x + (int64_t) row * width;

    const int64_t elements = (int64_t) rows * width;
    if constexpr (K == 0) {
        double squares = 0.0;
        for (int i = threadIdx.x; i < width; i += kThreads) {
            const double v = (double) xr[i];
            squares += v * v;
        }
        squares = wave_sum(squares);
        if ((threadIdx.x & 63) == 0)
            partial[threadIdx.x >> 6] = squares;
        __syncthreads();
        double total = 0.0;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w)
            total += partial[w];
        const double scale = norm_scale(total, width, epsilon);
        for (int base = 0; base < width; base += kThreads) { // uniform: whole waves
            const int i = base + threadIdx.x;
            const bool live = i < width;
            const int c = live ? i : width - 1;
            norm_store(xr[c], weight[c], scale, (int64_t) row * width + c, live, elements, y, q8);
        }
    } else {
        static_assert(K % P == 0, "whole parts of a row");
        constexpr int KP = K / P;
        const int k0 = (int) blockIdx.y * KP; // this workgroup's part: elements t + k kThreads, k >= k0
        float xv[K], xn[KP], wv[KP];
#pragma unroll
        for (int k = 0; k < K; ++k)
            xv[k] = xr[min((int) threadIdx.x + k * kThreads, width - 1)]; // clamped; masked below
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            const int i = min((int) threadIdx.x + (k0 + k) * kThreads, width - 1);
            if constexpr (P == 1)
                xn[k] = xv[k];
            else
                xn[k] = xr[i];
            wv[k] = weight[i];
        }
        double squares = 0.0;
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (threadIdx.x + k * kThreads < width)
                squares += (double) xv[k] * (double) xv[k]; // the square is exact in double
        squares = wave_sum(squares);
        if ((threadIdx.x & 63) == 0)
            partial[threadIdx.x >> 6] = squares;
        __syncthreads();
        double total = 0.0;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w)
            total += partial[w];
        const double scale = norm_scale(total, width, epsilon);
        if constexpr (P == 1 && K == 8) {
            // Many rows (a prefill): the normalized row goes through LDS so
            // that a thread holds 8 consecutive elements, a 32-element
            // block's four threads find its largest magnitude in two lane
            // exchanges and compute its scale once, and the bytes leave in
            // one 8-byte store.  The same values, maximum, scale and bytes
            // as the per-element form below.
            __shared__ __align__(16) float sRow[K * kThreads];
#pragma unroll
            for (int k = 0; k < K; ++k)
                sRow[threadIdx.x + k * kThreads] = norm_value(xn[k], scale, wv[k]);
            __syncthreads();
            const int e0 = 8 * (int) threadIdx.x; // elements e0 .. e0 + 7, block e0 / 32
            const float4 lo4 = *reinterpret_cast<const float4 *>(&sRow[e0]);
            const float4 hi4 = *reinterpret_cast<const float4 *>(&sRow[e0 + 4]);
            const float v[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
            float amax = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                amax = fmaxf(amax, fabsf(v[i]));
            amax = fmaxf(amax, xor_lane<1>(amax));
            amax = fmaxf(amax, xor_lane<2>(amax));
            const uint16_t bits = scale_bits_from_amax(amax);
            const float sc = half_value(bits);
            const float inv = quantize_hint(sc);
            uint32_t packed[2] = {0u, 0u};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                packed[i / 4] |= (uint32_t) (uint8_t) (int8_t) quantize_in_block(v[i], bits, sc, inv)
                                 << (8 * (i % 4));
            if (e0 < width) { // whole 32-element blocks are live together
                const int64_t at = (int64_t) row * width + e0;
                if (y) {
                    *reinterpret_cast<float4 *>(y + at) = lo4;
                    *reinterpret_cast<float4 *>(y + at + 4) = hi4;
                }
                if (q8) {
                    *reinterpret_cast<uint2 *>(q8 + at) = make_uint2(packed[0], packed[1]);
                    if ((threadIdx.x & 3) == 0)
                        reinterpret_cast<uint16_t *>(q8 + elements)[at / kBlock] = bits;
                }
            }
            return;
        }
        // every element's value, block scale and byte first (no branches, so
        // the K chains interleave), then the stores
        float v[KP], amax[KP];
        uint16_t bits[KP];
        int bytes[KP];
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            v[k] = norm_value(xn[k], scale, wv[k]);
            amax[k] = fabsf(v[k]);
        }
        max_lanes_each<16>(amax); // each 32-lane group's largest magnitude
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            bits[k] = scale_bits_from_amax(amax[k]);
            const float sc = half_value(bits[k]);
            bytes[k] = quantize_in_block(v[k], bits[k], sc, quantize_hint(sc));
        }
        uint16_t *scales = q8 ? reinterpret_cast<uint16_t *>(q8 + elements) : nullptr;
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            const int i = threadIdx.x + (k0 + k) * kThreads;
            if (i >= width) // whole 32-element groups are live together
                continue;
            const int64_t at = (int64_t) row * width + i;
            if (y)
                y[at] = v[k];
            if (q8) {
                q8[at] = (uint8_t) (int8_t) bytes[k];
                if ((threadIdx.x & 31) == 0)
                    scales[at / kBlock] = bits[k];
            }
        }
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

// ---- the one-row product of a decode step --------------------------------
// Same arithmetic as q8_product_kernel for a single activation row, without
// LDS or barriers on the common shapes: the activation blocks a lane needs sit
// in its registers, and every weight load of the wave is issued before any
// arithmetic.  A row of `inner` elements is split into 64-block segments;
// WPR waves share a row group (segments dealt round-robin), each wave owns U
// consecutive rows and S segments of each.
template <int U, int WPR, int S>
__global__ __launch_bounds__(kThreads) void q8_matvec_kernel(
    const uint8_t *__restrict__ x8, int64_t x_elements, int x_row, const uint8_t *__restrict__ w8,
    int inner, int outputs, float *__restrict__ y, int residual)
{
    GQ8_ARGS_EARLY("s"(y), "s"(residual));
    __shared__ double sPartial[kThreads / 64][U];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int group = wave / WPR, part = wave % WPR;
    const int row0 = (blockIdx.x * (4 / WPR) + group) * U;
    const int nb = inner / kBlock;
    const int64_t wElements = (int64_t) outputs * inner;
    const uint16_t *wScales = reinterpret_cast<const uint16_t *>(w8 + wElements);

    // Branch-free loads: an invalid (row, block) reads block 0 of row 0 and
    // its scale is zeroed at use; the scales come in their aligned 32-bit
    // words.  Every load of the wave is then in flight before the first wait.
    int4 wa[U][S], wb[U][S];
    uint32_t wsPair[U][S];
    bool wsHigh[U][S];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int o = row0 + u;
#pragma unroll
        for (int j = 0; j < S; ++j) {
            const int b = lane + 64 * (part + WPR * j);
            const bool valid = o < outputs && b < nb;
            const int64_t r = valid ? o : 0;
            const int c = valid ? b : 0;
            const int4 *p = reinterpret_cast<const int4 *>(w8 + r * inner + (int64_t) c * kBlock);
            wa[u][j] = p[0];
            wb[u][j] = p[1];
            const int64_t index = r * nb + c;
            // masking (not selecting) the word keeps the load unconditional
            wsPair[u][j] = reinterpret_cast<const uint32_t *>(wScales)[index >> 1]
                           & (valid ? 0xFFFFFFFFu : 0u);
            wsHigh[u][j] = (index & 1) != 0;
        }
    }
    int4 a0[S], a1[S];
    uint16_t saBits[S];
    const uint16_t *xScales = reinterpret_cast<const uint16_t *>(x8 + x_elements);
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const int b = lane + 64 * (part + WPR * j);
        const bool valid = b < nb;
        const int c = valid ? b : 0;
        const int4 *p = reinterpret_cast<const int4 *>(x8 + (int64_t) x_row * inner + (int64_t) c * kBlock);
        a0[j] = p[0];
        a1[j] = p[1];
        saBits[j] = xScales[(int64_t) x_row * nb + c] & (valid ? 0xFFFFu : 0u);
    }
    // the residual of the wave's rows, issued last: it arrives behind the
    // weights, so the store at the end does not wait for a fresh round trip
    float old[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        old[u] = y[min(row0 + u, outputs - 1)];
    __builtin_amdgcn_sched_barrier(0);
    double sa[S];
#pragma unroll
    for (int j = 0; j < S; ++j)
        sa[j] = (double) half_value(saBits[j]);
    uint16_t wsBits[U][S];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < S; ++j)
            wsBits[u][j] = (uint16_t) (wsHigh[u][j] ? wsPair[u][j] >> 16 : wsPair[u][j] & 0xFFFFu);

    double acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        acc[u] = 0.0;
#pragma unroll
        for (int j = 0; j < S; ++j) {
            int d = 0;
            d = __builtin_amdgcn_sdot4(wa[u][j].x, a0[j].x, d, false);
            d = __builtin_amdgcn_sdot4(wa[u][j].y, a0[j].y, d, false);
            d = __builtin_amdgcn_sdot4(wa[u][j].z, a0[j].z, d, false);
            d = __builtin_amdgcn_sdot4(wa[u][j].w, a0[j].w, d, false);
            d = __builtin_amdgcn_sdot4(wb[u][j].x, a1[j].x, d, false);
            d = __builtin_amdgcn_sdot4(wb[u][j].y, a1[j].y, d, false);
            d = __builtin_amdgcn_sdot4(wb[u][j].z, a1[j].z, d, false);
            d = __builtin_amdgcn_sdot4(wb[u][j].w, a1[j].w, d, false);
            acc[u] += (double) d * ((double) half_value(wsBits[u][j]) * sa[j]);
        }
        acc[u] = wave_sum(acc[u]);
    }

    if (WPR > 1) {
        if (lane == 0)
#pragma unroll
            for (int u = 0; u < U; ++u)
                sPartial[wave][u] = acc[u];
        __syncthreads();
        if (part != 0)
            return;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            double total = 0.0;
            for (int w = 0; w < WPR; ++w)
                total += sPartial[wave + w][u];
            acc[u] = total;
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int o = row0 + u;
            if (o < outputs)
                y[o] = (float) (acc[u] + (residual ? (double) old[u] : 0.0));
        }
    }
}

// ---- multi-query attention, split over the keys ------------------------------
// Partial: a workgroup per (split, query row) owns a contiguous range of keys
// (a whole number of 32-key tiles, at most kMaxSplits splits per row) and all
// heads; it walks its range a tile at a time through LDS with an online
// softmax (running maximum and sum per head, the value sums rescaled when the
// maximum moves: the exact streaming fold of MultiQueryAttention.h:43-49).
// Scores and sums are in double; each score is its channel sum in four
// interleaved partial sums.
constexpr int kTile = 32;
constexpr int kMaxSplits = kAttentionSplits;
constexpr int kMaxQueryWidth = 2048;
constexpr int kMaxKvWidth = 256;
constexpr int kOutPerThread = kMaxQueryWidth / kThreads; // 8

__device__ inline int keys_per_split(int keyCount)
{
    const int tiles = (keyCount + kTile - 1) / kTile;
    return ((tiles + kMaxSplits - 1) / kMaxSplits) * kTile;
}

__global__ __launch_bounds__(kThreads) void mqa_partial_kernel(
    const float *__restrict__ queries, int q_stride, const uint16_t *__restrict__ key_cache,
    const uint16_t *__restrict__ value_cache, int heads, int kv_heads, int head_dim,
    const int *pos_ptr, int pos_value, float scale, double *__restrict__ ws_o,
    double *__restrict__ ws_ml)
{
    __shared__ double sQuery[kMaxQueryWidth];
    __shared__ uint32_t sKeys[kTile * (kMaxKvWidth / 2 + 1)];
    __shared__ uint32_t sValues[kTile * (kMaxKvWidth / 2)];
    __shared__ double sWeights[kMaxHeads * kTile];
    __shared__ double sMax[kMaxHeads], sSum[kMaxHeads], sFactor[kMaxHeads];

    const int split = blockIdx.x, row = blockIdx.y;
    const int keyCount = (pos_ptr ? *pos_ptr : 0) + pos_value + row + 1;
    const int perSplit = keys_per_split(keyCount);
    const int k0 = split * perSplit;
    if (k0 >= keyCount)
        return;
    const int k1 = min(k0 + perSplit, keyCount);
    const int qWidth = heads * head_dim, kvWidth = kv_heads * head_dim;
    const int perKv = heads / kv_heads;
    const int keyWords = kvWidth / 2, keyStride = kMaxKvWidth / 2 + 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    for (int i = threadIdx.x; i < qWidth; i += kThreads)
        sQuery[i] = (double) queries[(int64_t) row * q_stride + i];
    if (threadIdx.x < heads) {
        sMax[threadIdx.x] = -INFINITY;
        sSum[threadIdx.x] = 0.0;
    }
    double acc[kOutPerThread];
#pragma unroll
    for (int i = 0; i < kOutPerThread; ++i)
        acc[i] = 0.0;

    for (int t0 = k0; t0 < k1; t0 += kTile) {
        const int nk = min(kTile, k1 - t0);
        __syncthreads(); // the previous tile's reads are done
        const uint32_t *keyRows = reinterpret_cast<const uint32_t *>(key_cache + (int64_t) t0 * kvWidth);
        const uint32_t *valueRows = reinterpret_cast<const uint32_t *>(value_cache + (int64_t) t0 * kvWidth);
        for (int i = threadIdx.x; i < nk * keyWords; i += kThreads) {
            const int j = i / keyWords, w = i % keyWords;
            sKeys[j * keyStride + w] = keyRows[i];
            sValues[i] = valueRows[i];
        }
        __syncthreads();

        for (int idx = threadIdx.x; idx < heads * kTile; idx += kThreads) {
            const int head = idx / kTile, j = idx % kTile;
            double score = -INFINITY;
            if (j < nk) {
                const double *q = sQuery + head * head_dim;
                const uint32_t *k = sKeys + j * keyStride + ((head / perKv) * head_dim) / 2;
                double p0 = 0.0, p1 = 0.0, p2 = 0.0, p3 = 0.0;
                int c = 0;
                for (; c + 4 <= head_dim; c += 4) {
                    const uint32_t a = k[c / 2], b = k[c / 2 + 1];
                    p0 += q[c] * (double) half_value((uint16_t) (a & 0xFFFFu));
                    p1 += q[c + 1] * (double) half_value((uint16_t) (a >> 16));
                    p2 += q[c + 2] * (double) half_value((uint16_t) (b & 0xFFFFu));
                    p3 += q[c + 3] * (double) half_value((uint16_t) (b >> 16));
                }
                for (; c < head_dim; c += 2) {
                    const uint32_t a = k[c / 2];
                    p0 += q[c] * (double) half_value((uint16_t) (a & 0xFFFFu));
                    p1 += q[c + 1] * (double) half_value((uint16_t) (a >> 16));
                }
                score = (double) scale * ((p0 + p1) + (p2 + p3));
            }
            sWeights[idx] = score;
        }
        __syncthreads();

        // per head: the tile's weights against the running maximum
        for (int head = wave; head < heads; head += kThreads / 64) {
            const double s = lane < kTile ? sWeights[head * kTile + lane] : -INFINITY;
            const double tileMax = wave_max(s);
            const double previous = sMax[head];
            const double largest = fmax(previous, tileMax);
            const double w = (lane < nk) ? exp(s - largest) : 0.0;
            const double total = wave_sum(w);
            if (lane < kTile)
                sWeights[head * kTile + lane] = w;
            if (lane == 0) {
                const double factor = previous == -INFINITY ? 0.0 : exp(previous - largest);
                sFactor[head] = factor;
                sSum[head] = sSum[head] * factor + total;
                sMax[head] = largest;
            }
        }
        __syncthreads();

#pragma unroll
        for (int i = 0; i < kOutPerThread; ++i) {
            const int idx = threadIdx.x + i * kThreads;
            if (idx < qWidth) {
                const int head = idx / head_dim, c = idx % head_dim;
                const int column = (head / perKv) * head_dim + c;
                const uint16_t *v = reinterpret_cast<const uint16_t *>(sValues) + column;
                const double *w = sWeights + head * kTile;
                double sum = 0.0;
                for (int j = 0; j < nk; ++j)
                    sum += w[j] * (double) half_value(v[j * kvWidth]);
                acc[i] = acc[i] * sFactor[head] + sum;
            }
        }
    }

    double *o = ws_o + ((int64_t) row * kMaxSplits + split) * qWidth;
#pragma unroll
    for (int i = 0; i < kOutPerThread; ++i) {
        const int idx = threadIdx.x + i * kThreads;
        if (idx < qWidth)
            o[idx] = acc[i];
    }
    if (threadIdx.x < heads) {
        double *ml = ws_ml + (((int64_t) row * kMaxSplits + split) * heads + threadIdx.x) * 2;
        ml[0] = sMax[threadIdx.x];
        ml[1] = sSum[threadIdx.x];
    }
}

// Merge: per query row, each split's maximum and sum rescaled to the row's
// maximum, the factors computed once per (head, split) in LDS, the output
// divided by the total, rounded to fp32 and optionally quantized.
__global__ __launch_bounds__(kThreads) void mqa_merge_kernel(
    int heads, int head_dim, const int *pos_ptr, int pos_value, const double *__restrict__ ws_o,
    const double *__restrict__ ws_ml, float *__restrict__ out, uint8_t *__restrict__ q8, int rows)
{
    __shared__ double sFactor[kMaxHeads * kMaxSplits];
    __shared__ double sLargest[kMaxHeads], sTotal[kMaxHeads];
    const int row = blockIdx.x;
    const int keyCount = (pos_ptr ? *pos_ptr : 0) + pos_value + row + 1;
    const int perSplit = keys_per_split(keyCount);
    const int splits = (keyCount + perSplit - 1) / perSplit;
    const int qWidth = heads * head_dim;
    const int64_t elements = (int64_t) rows * qWidth;
    const double *ml = ws_ml + (int64_t) row * kMaxSplits * heads * 2;

    if (threadIdx.x < heads) {
        double largest = -INFINITY;
        for (int s = 0; s < splits; ++s)
            largest = fmax(largest, ml[((int64_t) s * heads + threadIdx.x) * 2]);
        sLargest[threadIdx.x] = largest;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < heads * splits; idx += kThreads) {
        const int head = idx / splits, s = idx % splits;
        sFactor[head * kMaxSplits + s] = exp(ml[((int64_t) s * heads + head) * 2] - sLargest[head]);
    }
    __syncthreads();
    if (threadIdx.x < heads) {
        double total = 0.0;
        for (int s = 0; s < splits; ++s)
            total += ml[((int64_t) s * heads + threadIdx.x) * 2 + 1]
                     * sFactor[threadIdx.x * kMaxSplits + s];
        sTotal[threadIdx.x] = total;
    }
    __syncthreads();

    const double *o = ws_o + (int64_t) row * kMaxSplits * qWidth;
    for (int idx = threadIdx.x; idx < qWidth; idx += kThreads) {
        const int head = idx / head_dim;
        const double *factor = sFactor + head * kMaxSplits;
        double weighted = 0.0;
        for (int s = 0; s < splits; ++s)
            weighted += o[(int64_t) s * qWidth + idx] * factor[s];
        const float v = (float) (weighted / sTotal[head]);
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
                       stream, tokens, pos_ptr, nullptr, (int64_t) 0, table, (int64_t) vocab, width,
                       scale, out, nullptr, nullptr, 0, nullptr);
    return hipGetLastError();
}

hipError_t launch_embed_slots(const uint32_t *slots, int64_t slot_stride, const int *positions,
                              int rows, const uint8_t *table, int vocab, int width, float scale,
                              float *out, const float *cosines, const float *sines, int half,
                              float *row_angles, hipStream_t stream)
{
    if (rows <= 0 || width <= 0 || width % kBlock != 0 || !positions || slot_stride <= 0
        || (row_angles && (!cosines || !sines || half <= 0 || 2 * half > kThreads)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_kernel, dim3(blocks_for(width, kThreads), rows), dim3(kThreads), 0,
                       stream, slots, nullptr, positions, slot_stride, table, (int64_t) vocab,
                       width, scale, out, cosines, sines, half, row_angles);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *weight, int rows, int width,
                          float epsilon, float *y, uint8_t *q8, hipStream_t stream)
{
    if (rows <= 0 || width <= 0 || width % kBlock != 0)
        return hipErrorInvalidValue;
    const int held = (width + kThreads - 1) / kThreads;
    // a few rows (a lockstep step's) take a workgroup for each element a
    // thread holds
    const bool split = rows <= 64;
#define GQ8_RMSNORM(KK)                                                                          \
    do {                                                                                         \
        if (split)                                                                               \
            hipLaunchKernelGGL((rmsnorm_kernel<KK, KK>), dim3(rows, KK), dim3(kThreads), 0, stream, \
                               x, weight, rows, width, epsilon, y, q8);                          \
        else                                                                                     \
            hipLaunchKernelGGL((rmsnorm_kernel<KK, 1>), dim3(rows), dim3(kThreads), 0, stream, x,  \
                               weight, rows, width, epsilon, y, q8);                             \
    } while (0)
    if (held <= 1)
        GQ8_RMSNORM(1);
    else if (held <= 2)
        GQ8_RMSNORM(2);
    else if (held <= 4)
        GQ8_RMSNORM(4);
    else if (held <= 8)
        GQ8_RMSNORM(8);
    else if (held <= 16)
        GQ8_RMSNORM(16);
    else
        hipLaunchKernelGGL((rmsnorm_kernel<0, 1>), dim3(rows), dim3(kThreads), 0, stream, x, weight,
                           rows, width, epsilon, y, q8);
#undef GQ8_RMSNORM
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

template <int U, int WPR, int S>
hipError_t matvec_with(const uint8_t *x8, int64_t xElements, int xRow, const uint8_t *w8,
                       int inner, int outputs, float *y, int residual, hipStream_t stream)
{
    const unsigned grid = blocks_for(outputs, (4 / WPR) * U);
    hipLaunchKernelGGL((q8_matvec_kernel<U, WPR, S>), dim3(grid), dim3(kThreads), 0, stream, x8,
                       xElements, xRow, w8, inner, outputs, y, residual);
    return hipGetLastError();
}

// The one-row product: rows per wave by the output count, waves per row by
// the number of 64-block segments in a row.  Rows of 5-8 segments (the
// feed-forward down product) take four rows a workgroup, so the activation
// blocks a wave holds serve four rows (512 workgroups for 2048 outputs: 191.6
// against 197 us for 18 launches at one row a workgroup).
hipError_t launch_matvec(const uint8_t *x8, int64_t xElements, int xRow, const uint8_t *w8,
                         int inner, int outputs, float *y, int residual, hipStream_t stream)
{
    const int segments = (inner / kBlock + 63) / 64;
    if (segments <= 1) {
        if (outputs >= 131072)
            return matvec_with<8, 1, 1>(x8, xElements, xRow, w8, inner, outputs, y, residual, stream);
        if (outputs >= 16384)
            return matvec_with<4, 1, 1>(x8, xElements, xRow, w8, inner, outputs, y, residual, stream);
        return matvec_with<1, 1, 1>(x8, xElements, xRow, w8, inner, outputs, y, residual, stream);
    }
    if (segments == 2)
        return matvec_with<1, 2, 1>(x8, xElements, xRow, w8, inner, outputs, y, residual, stream);
    if (segments <= 4)
        return matvec_with<1, 4, 1>(x8, xElements, xRow, w8, inner, outputs, y, residual, stream);
    if (segments <= 8)
        return matvec_with<4, 4, 2>(x8, xElements, xRow, w8, inner, outputs, y, residual, stream);
    return hipErrorInvalidValue;
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
    if (rows == 1)
        return launch_matvec(x8, xElements, x_row0, w8, inner, outputs, y, residual, stream);
    if (q8_gemm_supported(rows, inner, outputs))
        return launch_q8_gemm(x8, xElements, x_row0, rows, w8, inner, outputs, y, y_stride,
                              residual, stream);
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
    (void) max_keys; // the split count is fixed, so a captured step fits every length
    const int64_t qWidth = (int64_t) heads * head_dim;
    return (size_t) ((int64_t) rows * kMaxSplits * (qWidth + 2 * heads)) * sizeof(double);
}

hipError_t launch_mqa(const float *queries, int q_stride, const uint16_t *key_cache,
                      const uint16_t *value_cache, int heads, int kv_heads, int head_dim,
                      int rows, const int *pos_ptr, int pos_value, int max_keys, float scale,
                      float *out, uint8_t *q8, void *workspace, size_t workspace_bytes,
                      hipStream_t stream)
{
    if (rows <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || heads > kMaxHeads
        || head_dim % 4 != 0 || heads * head_dim > kMaxQueryWidth
        || kv_heads * head_dim > kMaxKvWidth || max_keys <= 0
        || workspace_bytes < mqa_workspace_bytes(rows, heads, head_dim, max_keys))
        return hipErrorInvalidValue;
    if (q8 && (heads * head_dim) % kBlock != 0)
        return hipErrorInvalidValue;
    if (rows >= kPrefillAttentionMinRows
        && prefill_attention_supported(head_dim, queries, q_stride, key_cache, value_cache, out, q8))
        return launch_prefill_attention(queries, q_stride, key_cache, value_cache, heads, kv_heads,
                                        head_dim, rows, pos_ptr, pos_value, scale, out, q8, stream);
    double *wsO = reinterpret_cast<double *>(workspace);
    double *wsMl = wsO + (int64_t) rows * kMaxSplits * heads * head_dim;
    hipLaunchKernelGGL(mqa_partial_kernel, dim3(kMaxSplits, rows), dim3(kThreads), 0, stream,
                       queries, q_stride, key_cache, value_cache, heads, kv_heads, head_dim,
                       pos_ptr, pos_value, scale, wsO, wsMl);
    hipError_t status = hipGetLastError();
    if (status != hipSuccess)
        return status;
    hipLaunchKernelGGL(mqa_merge_kernel, dim3(rows), dim3(kThreads), 0, stream, heads, head_dim,
                       pos_ptr, pos_value, wsO, wsMl, out, q8, rows);
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
