// gq8_gemm.hip -- the multi-row Int8Blocks product on int8 MFMA (prefill).
//
// y[m, n] (+)= sum over 32-element blocks b of
//                  dot_i8(x[m, b], w[n, b]) * (scale_w[n, b] * scale_x[m, b])
//
// the reference's product (Linear.h:10-34, 284-298; the prefill's
// SimdTiledMatMul.h / TiledMatMul.h) with both operands in Int8Blocks: the
// activation rows quantized by the reference's own weight rule.  One
// v_mfma_i32_16x16x32_i8 covers exactly one block of a 16 x 16 tile, so every
// block's integer dot is exact; it is then scaled and accumulated in double,
// block by block in order, exactly as the one-row kernels and the oracle do
// -- so a prompt row computed here equals the same row computed alone.
//
// Tiling: a workgroup of eight waves owns a 128 x 64 tile of y (rows x
// outputs), a wave 32 x 32 (2 x 2 MFMA tiles).  K goes in chunks of eight
// blocks (256 bytes).  A chunk of both operands and its fp16 scales (as
// doubles) is staged in LDS with 16-byte loads (66 KB), so two workgroups
// share a CU and one's loads overlap the other's arithmetic.  The double
// epilogue (a conversion, a product with the weight scale and a fused
// multiply-add with the activation scale per element and block) bounds the
// kernel, not the MFMA.  The activation scales of a 16-lane row's four rows
// reach its lanes by DPP broadcast inside that multiply-add, so a chunk reads
// them from LDS once (four blocks a load) rather than per element.
//
// MFMA operand layout (checked on gfx950): for A 16 x 32 and B given as
// B[j][k] 16 x 32, lane l supplies A[l % 16][8 (l / 16) .. + 8) and
// B[l % 16][8 (l / 16) .. + 8); D[i][j] lands in lane 16 (i / 4) + j,
// element i % 4.
#include "gq8_kernels.hpp"
#include "gq8_lanes.hpp"
#include "gq8_numerics.hpp"

namespace gq8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kTileM = 128, kTileN = 64;
constexpr int kGemmThreads = 512;
constexpr int kChunk = 8;                       // blocks a chunk
constexpr int kChunkBytes = kChunk * kBlock;    // 256
constexpr int kRowBytes = kChunkBytes + 16;     // padded LDS row: conflict-free fragment reads
constexpr int kStageRows = kTileM + kTileN;     // 192 operand rows a chunk
constexpr int kStageVectors = kStageRows * kChunkBytes / 16 / kGemmThreads; // 6 a thread
constexpr int kStageScales = kStageRows * kChunk;                           // 1536

constexpr int kScalePieces = (kStageScales + kGemmThreads - 1) / kGemmThreads; // 3 a thread

// acc[j][r] += part[j][r] * s', r = 0..3, where s' is the s held by lane
// 4 Q + r of this lane's 16-lane row (a DPP broadcast inside the
// multiply-add).  It rounds acc + part * s' once, as acc + d * (sw * sx)
// does: both products are exact in double.
template <int Q>
__device__ inline void fmac_row_scales(double (&acc)[2][4], double s, const double (&part)[2][4])
{
    fmac_row_bcast4<4 * Q, 4 * Q + 1, 4 * Q + 2, 4 * Q + 3>(acc[0], s, part[0]);
    fmac_row_bcast4<4 * Q, 4 * Q + 1, 4 * Q + 2, 4 * Q + 3>(acc[1], s, part[1]);
}

// kGeglu: the gate|up product of a fused [2 F, inner] weight (gate rows
// first) with GeGLU and its Q8 folded in.  Tile column block bx stages gate
// rows [32 bx, 32 bx + 32) as B rows 0..31 and the matching up rows as B rows
// 32..63, so a tile holds both halves of 32 GeGLU outputs of 128 rows: the
// epilogue rounds both to fp32 (the stores the unfused product makes), takes
// the GeGLU of each pair and quantizes each row's 32 outputs as one block into
// q8_out ([rows, F] Q8 row buffer), with the fp32 outputs to debug_out if set.
template <bool kGeglu>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(4)))
void q8_gemm_kernel(
    const uint8_t *__restrict__ x8, int64_t xElements, int xRow0, int rows,
    const uint8_t *__restrict__ w8, int inner, int outputs, float *__restrict__ y, int yStride,
    int residual, uint8_t *__restrict__ q8_out, float *__restrict__ debug_out)
{
    // rows [0, 128) of a buffer are A (activation rows), [128, 192) B (weight rows)
    __shared__ __attribute__((aligned(16))) uint8_t sOps[1][kStageRows * kRowBytes];
    __shared__ double sScales[1][kStageRows][kChunk + 1];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int m0 = blockIdx.y * kTileM, n0 = blockIdx.x * kTileN;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int nb = inner / kBlock;
    const uint16_t *xScales = reinterpret_cast<const uint16_t *>(x8 + xElements);
    const uint16_t *wScales = reinterpret_cast<const uint16_t *>(w8 + (int64_t) outputs * inner);

    // the global source of the staged pieces this thread moves: row r of the
    // stage (clamped into range; rows past the end are computed, never stored)
    // 32-bit byte offsets from the two operand bases: the first kStageVectors
    // / 3 pieces of every thread are A rows (128 rows x 16 pieces = 2048 =
    // 4 x 512), the rest B rows
    const uint8_t *aBase = x8 + (int64_t) xRow0 * inner;
    const uint16_t *aScales = xScales + (int64_t) xRow0 * nb;
    // the weight row of B stage row j (0..63) of this tile
    const int F = outputs / 2;
    auto weight_row = [&](int j) {
        if constexpr (kGeglu)
            return (j < 32 ? 0 : F) + min((int) blockIdx.x * 32 + (j & 31), F - 1);
        else
            return min(n0 + j, outputs - 1);
    };
    uint32_t srcOff[kStageVectors];
#pragma unroll
    for (int i = 0; i < kStageVectors; ++i) {
        const int piece = t + i * kGemmThreads;     // 16-byte pieces, 16 a row
        const int r = piece >> 4, col = (piece & 15) * 16;
        srcOff[i] = r < kTileM ? (uint32_t) min(m0 + r, rows - 1) * (uint32_t) inner + col
                               : (uint32_t) weight_row(r - kTileM) * (uint32_t) inner + col;
    }
    uint32_t scaleOff[kScalePieces];
#pragma unroll
    for (int i = 0; i < kScalePieces; ++i) {
        const int e = t + i * kGemmThreads;
        const int r = e / kChunk, b = e % kChunk;
        scaleOff[i] = (r < kTileM ? (uint32_t) min(m0 + r, rows - 1)
                                  : (uint32_t) weight_row(r - kTileM)) * (uint32_t) nb + b;
    }
    static_assert(kTileM * 16 == 4 * kGemmThreads && kStageVectors == 6, "piece split");
    static_assert(kTileM * kChunk == 2 * kGemmThreads && kScalePieces == 3, "scale split");
    double acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[i][j][r] = 0.0;

    // this lane's fragment offsets in a stage
    const int kg = (lane >> 4) * 8;
    int aOff[2], bOff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        aOff[i] = (wm + i * 16 + (lane & 15)) * kRowBytes + kg;
        bOff[i] = (kTileM + wn + i * 16 + (lane & 15)) * kRowBytes + kg;
    }

    const int chunks = nb / kChunk;
    // a chunk's pieces go global -> registers one chunk ahead, so their loads
    // are in flight while the previous chunk is computed
    // (native vectors in plain unrolled loops: HIP's int4 carried across the
    // loop, or arrays captured by a lambda, are left in scratch memory)
    v4i v[kStageVectors];
    uint16_t sc[kScalePieces];
#pragma unroll
    for (int i = 0; i < kStageVectors; ++i)
        v[i] = *reinterpret_cast<const v4i *>((i < 4 ? aBase : w8) + srcOff[i]);
#pragma unroll
    for (int i = 0; i < kScalePieces; ++i)
        sc[i] = (i < 2 ? aScales : wScales)[scaleOff[i]];
    for (int c = 0; c < chunks; ++c) {
        __syncthreads(); // the previous chunk has been read
        {
#pragma unroll
            for (int i = 0; i < kStageVectors; ++i) {
                const int piece = t + i * kGemmThreads;
                *reinterpret_cast<v4i *>(&sOps[0][(piece >> 4) * kRowBytes + (piece & 15) * 16]) = v[i];
            }
#pragma unroll
            for (int i = 0; i < kScalePieces; ++i) {
                const int e = t + i * kGemmThreads;
                sScales[0][e / kChunk][e % kChunk] = (double) half_value(sc[i]);
            }
        }
        __syncthreads();
        {
            // the next chunk (the last is a repeat, never stored); its offset
            // joins the uniform bases, so each piece's address is a 32-bit
            // offset from a scalar base.  The chunk index and the offsets pass
            // through empty asm statements: otherwise the loop keeps a stepped
            // 64-bit address a piece (twelve registers) or the offsets'
            // 64-bit extensions.
            int next = min(c + 1, chunks - 1);
            asm volatile("" : "+s"(next));
            const int64_t c0 = (int64_t) next * kChunk;
            const uint8_t *aChunk = aBase + c0 * kBlock, *wChunk = w8 + c0 * kBlock;
            const uint16_t *aScaleChunk = aScales + c0, *wScaleChunk = wScales + c0;
#pragma unroll
            for (int i = 0; i < kStageVectors; ++i) {
                uint32_t off = srcOff[i];
                asm volatile("" : "+v"(off));
                v[i] = *reinterpret_cast<const v4i *>((i < 4 ? aChunk : wChunk) + off);
            }
#pragma unroll
            for (int i = 0; i < kScalePieces; ++i) {
                uint32_t off = scaleOff[i];
                asm volatile("" : "+v"(off));
                sc[i] = (i < 2 ? aScaleChunk : wScaleChunk)[off];
            }
        }
        const uint8_t *ops = sOps[0];
        // the activation scales of the wave's rows, four blocks a load: lane
        // (g, j) holds row 4 g + (j & 3)'s scale of block 4 h + (j >> 2) (the
        // rows of MFMA tile i), and every lane of the 16-lane row g takes the
        // one it needs by DPP
        double sxRow[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                sxRow[i][h] = sScales[0][wm + i * 16 + (lane >> 4) * 4 + (lane & 3)]
                                     [h * 4 + ((lane >> 2) & 3)];
        // a block's four MFMAs go out together, then their double epilogue, so
        // the later MFMAs run while the first one's results are scaled; the
        // blocks are unrolled (LDS offsets as immediates) with a scheduling
        // barrier between them, so no block's loads are hoisted into another's
        // registers
#pragma unroll
        for (int kb = 0; kb < kChunk; ++kb) {
            long af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                af[i] = *reinterpret_cast<const long *>(ops + aOff[i] + kb * kBlock);
                bf[i] = *reinterpret_cast<const long *>(ops + bOff[i] + kb * kBlock);
            }
            double sw[2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                sw[j] = sScales[0][kTileM + wn + j * 16 + (lane & 15)][kb];
            v4i d[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v4i zero = {0, 0, 0, 0};
                    d[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[i], bf[j], zero, 0, 0, 0);
                }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                double part[2][4]; // d * sw: exact (a 20-bit integer times an fp16 value)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        part[j][r] = (double) d[i][j][r] * sw[j];
                switch (kb & 3) {
                case 0: fmac_row_scales<0>(acc[i], sxRow[i][kb >> 2], part); break;
                case 1: fmac_row_scales<1>(acc[i], sxRow[i][kb >> 2], part); break;
                case 2: fmac_row_scales<2>(acc[i], sxRow[i][kb >> 2], part); break;
                default: fmac_row_scales<3>(acc[i], sxRow[i][kb >> 2], part); break;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    if constexpr (!kGeglu) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn + j * 16 + (lane & 15);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + wm + i * 16 + (lane >> 4) * 4 + r;
                    if (m < rows && n < outputs) {
                        float *out = y + (int64_t) m * yStride + n;
                        const double old = residual ? (double) *out : 0.0;
                        *out = (float) (acc[i][j][r] + old);
                    }
                }
            }
    } else {
        // the fp32 gate (columns 0..31) and up (32..63) values of the tile in
        // LDS, over the staging buffer (every wave is past its last read)
        __syncthreads();
        float *sOut = reinterpret_cast<float *>(sOps[0]); // [128][65]
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int c = wn + j * 16 + (lane & 15);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sOut[(wm + i * 16 + (lane >> 4) * 4 + r) * 65 + c] = (float) acc[i][j][r];
            }
        __syncthreads();
        // thread t: row t / 4, outputs 8 (t % 4) .. + 8 (four lanes a 32-block)
        const int row = t >> 2, c0 = (t & 3) * 8;
        const int m = m0 + row;
        float v[8];
        float amax = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v[k] = geglu(sOut[row * 65 + c0 + k], sOut[row * 65 + 32 + c0 + k]);
            amax = fmaxf(amax, fabsf(v[k]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 1));
        amax = fmaxf(amax, __shfl_xor(amax, 2));
        const int o0 = blockIdx.x * 32 + c0;
        if (m < rows && o0 < F) {
            const uint16_t bits = scale_bits_from_amax(amax);
            const float sc = half_value(bits);
            const float inv = bits ? quantize_hint(sc) : 0.f;
            uint32_t packed[2] = {0u, 0u};
#pragma unroll
            for (int k = 0; k < 8; ++k)
                packed[k / 4] |= (uint32_t) (uint8_t) (int8_t) quantize_in_block(v[k], bits, sc, inv)
                                 << (8 * (k % 4));
            *reinterpret_cast<uint2 *>(q8_out + (int64_t) m * F + o0) = make_uint2(packed[0], packed[1]);
            if ((t & 3) == 0)
                reinterpret_cast<uint16_t *>(q8_out + (int64_t) rows * F)[(int64_t) m * (F / kBlock) + blockIdx.x] = bits;
            if (debug_out)
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    debug_out[(int64_t) m * F + o0 + k] = v[k];
        }
    }
}

} // namespace

bool q8_gemm_supported(int rows, int inner, int outputs)
{
    return rows >= kGemmMinRows && inner % kChunkBytes == 0 && outputs > 0;
}

hipError_t launch_q8_gemm(const uint8_t *x8, int64_t x_elements, int x_row0, int rows,
                          const uint8_t *w8, int inner, int outputs, float *y, int y_stride,
                          int residual, hipStream_t stream)
{
    if (rows <= 0 || outputs <= 0 || inner <= 0 || inner % kChunkBytes != 0 || y_stride < outputs)
        return hipErrorInvalidValue;
    const dim3 grid((outputs + kTileN - 1) / kTileN, (rows + kTileM - 1) / kTileM);
    hipLaunchKernelGGL(q8_gemm_kernel<false>, grid, dim3(kGemmThreads), 0, stream, x8, x_elements,
                       x_row0, rows, w8, inner, outputs, y, y_stride, residual, nullptr, nullptr);
    return hipGetLastError();
}

bool q8_gemm_geglu_supported(int rows, int inner, int intermediate)
{
    return q8_gemm_supported(rows, inner, 2 * intermediate) && intermediate % kBlock == 0;
}

hipError_t launch_q8_gemm_geglu(const uint8_t *x8, int64_t x_elements, int x_row0, int rows,
                                const uint8_t *w8, int inner, int intermediate, uint8_t *q8_out,
                                float *debug_out, hipStream_t stream)
{
    if (rows <= 0 || !q8_gemm_geglu_supported(rows, inner, intermediate) || !q8_out)
        return hipErrorInvalidValue;
    const dim3 grid(intermediate / kBlock, (rows + kTileM - 1) / kTileM);
    hipLaunchKernelGGL(q8_gemm_kernel<true>, grid, dim3(kGemmThreads), 0, stream, x8, x_elements,
                       x_row0, rows, w8, inner, 2 * intermediate, nullptr, 0, 0, q8_out, debug_out);
    return hipGetLastError();
}

} // namespace gq8
