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
// Tiling: a workgroup of four waves owns a 64 x 64 tile of y, a wave 32 x 32
// (2 x 2 MFMA tiles).  K goes in chunks of eight blocks: each lane loads its
// eight-byte fragments of the chunk straight from global memory (they are
// contiguous 8-byte pieces of 32-byte blocks; a row of A and B is shared by
// two waves, which L1 serves), and the chunk's fp16 scales are staged in LDS
// as doubles.  The double epilogue (three fp64 operations an element and
// block) bounds the kernel, not the MFMA.
//
// MFMA operand layout (checked on gfx950): for A 16 x 32 and B given as
// B[j][k] 16 x 32, lane l supplies A[l % 16][8 (l / 16) .. + 8) and
// B[l % 16][8 (l / 16) .. + 8); D[i][j] lands in lane 16 (i / 4) + j,
// element i % 4.
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"

namespace gq8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmTile = 64;
constexpr int kGemmThreads = 256;
constexpr int kGemmChunk = 8; // blocks a chunk

__global__ __launch_bounds__(kGemmThreads) void q8_gemm_kernel(
    const uint8_t *__restrict__ x8, int64_t xElements, int xRow0, int rows,
    const uint8_t *__restrict__ w8, int inner, int outputs, float *__restrict__ y, int yStride,
    int residual)
{
    __shared__ double sScaleX[kGemmTile][kGemmChunk + 1];
    __shared__ double sScaleW[kGemmTile][kGemmChunk + 1];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int m0 = blockIdx.y * kGemmTile, n0 = blockIdx.x * kGemmTile;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int nb = inner / kBlock;
    const uint16_t *xScales = reinterpret_cast<const uint16_t *>(x8 + xElements);
    const uint16_t *wScales = reinterpret_cast<const uint16_t *>(w8 + (int64_t) outputs * inner);

    // this lane's fragment rows (clamped into range: the rows past the end
    // are computed and never stored)
    const int kg = (lane >> 4) * 8;
    const uint8_t *aRow[2], *bRow[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = min(m0 + wm + i * 16 + (lane & 15), rows - 1);
        const int n = min(n0 + wn + i * 16 + (lane & 15), outputs - 1);
        aRow[i] = x8 + (int64_t) (xRow0 + m) * inner + kg;
        bRow[i] = w8 + (int64_t) n * inner + kg;
    }
    // the scale rows this thread stages
    const int stageRow = t / kGemmChunk, stageBlock = t % kGemmChunk; // 32 rows a pass
    double acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[i][j][r] = 0.0;

    for (int c0 = 0; c0 < nb; c0 += kGemmChunk) {
        const int nc = min(kGemmChunk, nb - c0);
        // the chunk's fragments, all loads in flight (a block past the end
        // re-reads the last one and is not used)
        long af[kGemmChunk][2], bf[kGemmChunk][2];
#pragma unroll
        for (int kb = 0; kb < kGemmChunk; ++kb) {
            const int64_t at = (int64_t) (c0 + min(kb, nc - 1)) * kBlock;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                af[kb][i] = *reinterpret_cast<const long *>(aRow[i] + at);
                bf[kb][i] = *reinterpret_cast<const long *>(bRow[i] + at);
            }
        }
        // the chunk's scales as doubles
        __syncthreads(); // the previous chunk's scales are read
#pragma unroll
        for (int pass = 0; pass < kGemmTile / (kGemmThreads / kGemmChunk); ++pass) {
            const int r = stageRow + pass * (kGemmThreads / kGemmChunk);
            const int b = c0 + min(stageBlock, nc - 1);
            const int m = min(m0 + r, rows - 1), n = min(n0 + r, outputs - 1);
            sScaleX[r][stageBlock] = (double) half_value(xScales[(int64_t) (xRow0 + m) * nb + b]);
            sScaleW[r][stageBlock] = (double) half_value(wScales[(int64_t) n * nb + b]);
        }
        __syncthreads();
#pragma unroll
        for (int kb = 0; kb < kGemmChunk; ++kb) {
            if (kb >= nc)
                break;
            double sw[2], sx[2][4];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                sw[j] = sScaleW[wn + j * 16 + (lane & 15)][kb];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sx[i][r] = sScaleX[wm + i * 16 + (lane >> 4) * 4 + r][kb];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v4i zero = {0, 0, 0, 0};
                    const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[kb][i], bf[kb][j], zero,
                                                                      0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[i][j][r] += (double) d[r] * (sw[j] * sx[i][r]);
                }
        }
    }

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
}

} // namespace

hipError_t launch_q8_gemm(const uint8_t *x8, int64_t x_elements, int x_row0, int rows,
                          const uint8_t *w8, int inner, int outputs, float *y, int y_stride,
                          int residual, hipStream_t stream)
{
    if (rows <= 0 || outputs <= 0 || inner <= 0 || inner % kBlock != 0 || y_stride < outputs)
        return hipErrorInvalidValue;
    const dim3 grid((outputs + kGemmTile - 1) / kGemmTile, (rows + kGemmTile - 1) / kGemmTile);
    hipLaunchKernelGGL(q8_gemm_kernel, grid, dim3(kGemmThreads), 0, stream, x8, x_elements, x_row0,
                       rows, w8, inner, outputs, y, y_stride, residual);
    return hipGetLastError();
}

} // namespace gq8
