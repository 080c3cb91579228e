// gq8_runtime.hip -- the C ABI of include/gemma_q8.h: the op-level entry
// points, the decoder (HF::Decoder, Lib/HuggingFaceEACP/Decoder/Decoder.cpp)
// and the greedy token loop (HF::Gemma, Lib/HuggingFaceEACP/Generation/
// Gemma.cpp).  Host C++ over the HIP runtime; every device buffer is owned
// here and every refusal is checked before anything is launched.
#include "gemma_q8.h"
#include "gq8_checkpoint.hpp"
#include "gq8_decode.hpp"
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstring>
#include <random>
#include <string>
#include <mutex>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_lastError;

int fail(int status, const std::string &message)
{
    g_lastError = message;
    return status;
}

#define GQ8_HIP(expr)                                                                    \
    do {                                                                                 \
        hipError_t status_ = (expr);                                                     \
        if (status_ != hipSuccess)                                                       \
            return fail(GQ8_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(status_)); \
    } while (0)

#define GQ8_LAUNCH(expr)                                                                 \
    do {                                                                                 \
        hipError_t status_ = (expr);                                                     \
        if (status_ == hipErrorInvalidValue)                                             \
            return fail(GQ8_ERR_ARGUMENT, std::string(#expr) + ": arguments refused");   \
        if (status_ != hipSuccess)                                                       \
            return fail(GQ8_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(status_)); \
    } while (0)

hipStream_t as_stream(void *stream)
{
    return reinterpret_cast<hipStream_t>(stream);
}

int hardware_threads(int requested)
{
    if (requested > 0)
        return requested;
    const unsigned n = std::thread::hardware_concurrency();
    return n == 0 ? 1 : (int) n;
}

template <typename F>
void parallel_for(int64_t count, int threads, F body)
{
    threads = (int) std::max<int64_t>(1, std::min<int64_t>(threads, count));
    if (threads == 1) {
        for (int64_t i = 0; i < count; ++i)
            body(i);
        return;
    }
    std::vector<std::thread> pool;
    std::atomic<int64_t> next{0};
    for (int t = 0; t < threads; ++t)
        pool.emplace_back([&] {
            for (int64_t i = next++; i < count; i = next++)
                body(i);
        });
    for (auto &thread : pool)
        thread.join();
}

// ---- host Int8Blocks (Int8Blocks.cpp:25-124), the same numerics as the GPU
void quantize_block_host(const float *block, uint8_t *bytes, uint16_t *scale)
{
    float largest = 0.f;
    for (int i = 0; i < gq8::kBlock; ++i) {
        const float m = std::fabs(block[i]);
        if (largest < m)
            largest = m;
    }
    const uint16_t bits = gq8::scale_bits_from_amax(largest);
    *scale = bits;
    if (bits == 0) {
        std::memset(bytes, 0, gq8::kBlock);
        return;
    }
    const float s = gq8::half_value(bits);
    const float inverse = 1.0f / s;
    for (int i = 0; i < gq8::kBlock; ++i)
        bytes[i] = (uint8_t) (int8_t) gq8::quantize_value(block[i], s, inverse);
}

// ---- seeded synthetic weights -------------------------------------------
// Box-Muller in double over std::mt19937_64: one engine per 2^20-element
// chunk, seeded (tensor_seed << 32) | chunk; (r cos t, r sin t) fill two
// consecutive elements, r = sqrt(-2 ln(1 - u1)), t = 2 pi u2, u = next() >> 11
// scaled by 2^-53; each value sigma * z narrowed to fp32.
constexpr int64_t kChunk = int64_t(1) << 20;

void normal_chunk(uint64_t tensorSeed, double sigma, int64_t chunk, int64_t count, float *out)
{
    std::mt19937_64 engine((tensorSeed << 32) | (uint64_t) chunk);
    const int64_t begin = chunk * kChunk;
    const int64_t end = std::min(begin + kChunk, count);
    const double twoPi = 6.283185307179586476925286766559;
    for (int64_t at = begin; at < end; at += 2) {
        const double u1 = (double) (engine() >> 11) * (1.0 / 9007199254740992.0);
        const double u2 = (double) (engine() >> 11) * (1.0 / 9007199254740992.0);
        const double radius = std::sqrt(-2.0 * std::log(1.0 - u1));
        const double angle = twoPi * u2;
        out[at - begin] = (float) (sigma * (radius * std::cos(angle)));
        if (at + 1 < end)
            out[at + 1 - begin] = (float) (sigma * (radius * std::sin(angle)));
    }
}

// Sampler::uniform (Sampler.cpp:209-212): the top 53 bits of a 64-bit
// Mersenne Twister output, scaled into [0, 1).
void uniform_draws(uint64_t seed, int count, double *out)
{
    std::mt19937_64 engine(seed);
    for (int i = 0; i < count; ++i)
        out[i] = (double) (engine() >> 11) * 0x1.0p-53;
}

int sampling_error(const gq8_sampling &o)
{
    if (!(o.temperature >= 0.f))
        return fail(GQ8_ERR_ARGUMENT, "A sampling temperature must be zero or positive");
    if (o.top_k < 0)
        return fail(GQ8_ERR_ARGUMENT, "A top-k count cannot be negative");
    if (!(o.top_p > 0.f && o.top_p <= 1.f))
        return fail(GQ8_ERR_ARGUMENT, "A top-p mass must lie inside (0, 1]");
    return GQ8_OK;
}


} // namespace

// ============================================================================
// Status and format helpers
// ============================================================================
int gq8::report(int status, const std::string &message)
{
    return fail(status, message);
}

int gq8::check_sampling(const gq8_sampling &options)
{
    return sampling_error(options);
}

extern "C" const char *gq8_status_string(int status)
{
    switch (status) {
    case GQ8_OK: return "ok";
    case GQ8_ERR_ARGUMENT: return "invalid argument";
    case GQ8_ERR_SHAPE: return "decoder shape refused";
    case GQ8_ERR_CAPACITY: return "rows past the step capacity";
    case GQ8_ERR_WINDOW: return "position past the window";
    case GQ8_ERR_TOKEN: return "token id outside the vocabulary";
    case GQ8_ERR_UNQUANTIZABLE: return "tensor shape not storable as Int8Blocks";
    case GQ8_ERR_NOT_PREPARED: return "weights not loaded";
    case GQ8_ERR_EMPTY: return "no tokens";
    case GQ8_ERR_DEVICE: return "HIP error";
    case GQ8_ERR_MEMORY: return "device allocation failed";
    case GQ8_ERR_FORMAT: return "malformed or mismatched checkpoint file";
    default: return "unknown status";
    }
}

extern "C" const char *gq8_last_error(void)
{
    return g_lastError.c_str();
}

extern "C" const char *gq8_version(void)
{
    return "gemma_q8 0.1.0 gfx950";
}

extern "C" int64_t gq8_int8_block_count(int64_t element_count)
{
    return element_count / gq8::kBlock;
}

extern "C" int64_t gq8_int8_blocks_byte_count(int64_t element_count)
{
    return element_count + 2 * gq8_int8_block_count(element_count);
}

extern "C" int gq8_quantizes_as_int8_blocks(int64_t contiguous_extent, int64_t element_count)
{
    return contiguous_extent > 0 && element_count > 0 && contiguous_extent % gq8::kBlock == 0
           && element_count % (2 * gq8::kBlock) == 0;
}

extern "C" int gq8_quantize_int8_blocks_host(const float *values, int64_t value_count,
                                             int64_t first, int64_t element_count,
                                             uint8_t *destination)
{
    if (!values || !destination || value_count < 0 || first < 0 || first % gq8::kBlock != 0
        || value_count % gq8::kBlock != 0 || first + value_count > element_count)
        return fail(GQ8_ERR_ARGUMENT, "quantize: pieces must be whole blocks inside the tensor");
    uint16_t *scales = reinterpret_cast<uint16_t *>(destination + element_count);
    const int64_t blocks = value_count / gq8::kBlock;
    const int64_t perTask = 4096;
    parallel_for((blocks + perTask - 1) / perTask, hardware_threads(0), [&](int64_t task) {
        const int64_t b0 = task * perTask, b1 = std::min(blocks, b0 + perTask);
        for (int64_t b = b0; b < b1; ++b) {
            const int64_t element = first + b * gq8::kBlock;
            uint16_t bits;
            quantize_block_host(values + b * gq8::kBlock, destination + element, &bits);
            std::memcpy(reinterpret_cast<uint8_t *>(scales) + 2 * (element / gq8::kBlock), &bits, 2);
        }
    });
    return GQ8_OK;
}

extern "C" int gq8_dequantize_int8_blocks_host(const uint8_t *stored, int64_t element_count,
                                               float *values)
{
    if (!stored || !values || element_count < 0)
        return fail(GQ8_ERR_ARGUMENT, "dequantize: null buffer");
    for (int64_t i = 0; i < element_count; ++i) {
        uint16_t bits;
        std::memcpy(&bits, stored + element_count + 2 * (i / gq8::kBlock), 2);
        values[i] = gq8::half_value(bits) * (float) ((int) (stored[i] ^ 0x80u) - 128);
    }
    return GQ8_OK;
}

extern "C" int gq8_rotary_table_host(int max_positions, int head_dim, double theta,
                                     float *cosines, float *sines)
{
    if (max_positions <= 0 || head_dim <= 0 || head_dim % 2 != 0 || !cosines || !sines)
        return fail(GQ8_ERR_ARGUMENT, "rotary table: bad shape");
    // makeRotaryTable (RoPE.cpp:7-34): double inverse frequency and angle,
    // cos/sin narrowed to fp32.
    const int half = head_dim / 2;
    for (int channel = 0; channel < half; ++channel) {
        const double exponent = 2.0 * channel / (double) head_dim;
        const double inverseFrequency = 1.0 / std::pow(theta, exponent);
        for (int position = 0; position < max_positions; ++position) {
            const double angle = (double) position * inverseFrequency;
            cosines[(int64_t) position * half + channel] = (float) std::cos(angle);
            sines[(int64_t) position * half + channel] = (float) std::sin(angle);
        }
    }
    return GQ8_OK;
}

// ============================================================================
// Op-level entry points
// ============================================================================
extern "C" int gq8_quantize_rows(const float *x, int64_t rows, int64_t inner, uint8_t *q8,
                                 void *stream)
{
    if (!x || !q8 || rows <= 0 || inner <= 0 || inner % gq8::kBlock != 0)
        return fail(GQ8_ERR_UNQUANTIZABLE, "quantize_rows: inner must be a positive multiple of 32");
    const int64_t elements = rows * inner;
    GQ8_LAUNCH(gq8::launch_quantize(x, elements, q8,
                                    reinterpret_cast<uint16_t *>(q8 + elements), as_stream(stream)));
    return GQ8_OK;
}

extern "C" int gq8_embed(const uint32_t *tokens, int rows, const uint8_t *table, int vocab,
                         int width, float scale, float *out, void *stream)
{
    if (!tokens || !table || !out || rows <= 0 || vocab <= 0 || width <= 0
        || width % gq8::kBlock != 0)
        return fail(GQ8_ERR_ARGUMENT, "embed: bad arguments");
    GQ8_LAUNCH(gq8::launch_embed(tokens, nullptr, rows, table, vocab, width, scale, out,
                                 as_stream(stream)));
    return GQ8_OK;
}

extern "C" int gq8_rmsnorm(const float *x, const float *weight, int rows, int width,
                           float epsilon, float *y, uint8_t *q8, void *stream)
{
    if (!x || !weight || (!y && !q8) || rows <= 0 || width <= 0 || width % gq8::kBlock != 0)
        return fail(GQ8_ERR_ARGUMENT, "rmsnorm: bad arguments");
    GQ8_LAUNCH(gq8::launch_rmsnorm(x, weight, rows, width, epsilon, y, q8, as_stream(stream)));
    return GQ8_OK;
}

extern "C" int gq8_rope(float *x, int row_stride, int heads, int head_dim, int first_position,
                        int rows, const float *cosines, const float *sines, void *stream)
{
    if (!x || !cosines || !sines || rows <= 0 || heads <= 0 || head_dim <= 0
        || head_dim % 4 != 0 || row_stride < heads * head_dim || first_position < 0)
        return fail(GQ8_ERR_ARGUMENT, "rope: bad arguments");
    GQ8_LAUNCH(gq8::launch_rope(x, row_stride, heads, head_dim, nullptr, first_position, rows,
                                cosines, sines, as_stream(stream)));
    return GQ8_OK;
}

extern "C" int gq8_q8_product(const uint8_t *x8, const uint8_t *w8, int rows, int inner,
                              int outputs, float *y, int y_stride, int residual, void *stream)
{
    if (!x8 || !w8 || !y || rows <= 0 || outputs <= 0 || y_stride < outputs)
        return fail(GQ8_ERR_ARGUMENT, "q8_product: bad arguments");
    if (!gq8_quantizes_as_int8_blocks(inner, (int64_t) inner * outputs)
        || inner % gq8::kBlock != 0 || inner > 16384)
        return fail(GQ8_ERR_UNQUANTIZABLE, "q8_product: inner must be a multiple of 32, <= 16384");
    GQ8_LAUNCH(gq8::launch_q8_product(x8, rows, 0, rows, w8, inner, outputs, y, y_stride, residual,
                                      as_stream(stream)));
    return GQ8_OK;
}

extern "C" int gq8_kv_store_f16(const float *k, const float *v, int src_stride, int rows,
                                int kv_width, uint16_t *key_cache, uint16_t *value_cache,
                                int position, void *stream)
{
    if (!k || !v || !key_cache || !value_cache || rows <= 0 || kv_width <= 0
        || src_stride < kv_width || position < 0)
        return fail(GQ8_ERR_ARGUMENT, "kv_store: bad arguments");
    GQ8_LAUNCH(gq8::launch_kv_store(k, v, src_stride, rows, kv_width, key_cache, value_cache,
                                    nullptr, position, as_stream(stream)));
    return GQ8_OK;
}

static int check_attention_shape(int heads, int kv_heads, int head_dim)
{
    // MultiQueryAttention.cpp:19-39 plus this kernel's own limits
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || head_dim <= 0
        || head_dim % 4 != 0 || head_dim > gq8::kMaxHeadDim || heads > gq8::kMaxHeads
        || heads * head_dim > 2048 || kv_heads * head_dim > 256)
        return fail(GQ8_ERR_SHAPE, "attention: heads a multiple of kv heads, head width a "
                                   "multiple of 4 up to 256, at most 16 heads, query row <= 2048, "
                                   "kv row <= 256");
    return GQ8_OK;
}

extern "C" size_t gq8_mqa_workspace_bytes(int rows, int heads, int head_dim, int max_keys)
{
    return gq8::mqa_workspace_bytes(rows, heads, head_dim, max_keys);
}

extern "C" int gq8_mqa_decode(const float *query, const uint16_t *key_cache,
                              const uint16_t *value_cache, int heads, int kv_heads, int head_dim,
                              int key_count, float scale, float *out, void *workspace,
                              size_t workspace_bytes, void *stream)
{
    if (int s = check_attention_shape(heads, kv_heads, head_dim))
        return s;
    if (!query || !key_cache || !value_cache || !out || !workspace || key_count < 1)
        return fail(GQ8_ERR_ARGUMENT, "mqa_decode: bad arguments");
    if (workspace_bytes < gq8::mqa_workspace_bytes(1, heads, head_dim, key_count))
        return fail(GQ8_ERR_ARGUMENT, "mqa_decode: workspace too small");
    GQ8_LAUNCH(gq8::launch_mqa(query, heads * head_dim, key_cache, value_cache, heads, kv_heads,
                               head_dim, 1, nullptr, key_count - 1, key_count, scale, out, nullptr,
                               workspace, workspace_bytes, as_stream(stream)));
    return GQ8_OK;
}

// ---- mqa_decode without an allocation ------------------------------------
// The split partials of gq8_mqa_decode_noalloc live in this file-scope device
// array: rows 1, at most kMaxHeads heads and a 2048-wide query row, i.e.
// kAttentionSplits x (2048 + 2 x 16) doubles = 1 064 960 bytes per GPU, held
// until the process ends.  The kernels take its device address, which
// hipGetSymbolAddress gives once per device (the array's name is a host-side
// stand-in, not a device address).  The merge reads only the splits the
// partial kernel wrote in the same call, so nothing needs clearing; calls that
// overlap on one GPU share the array and race.
namespace {
constexpr size_t kNoAllocScratchBytes =
    (size_t) gq8::kAttentionSplits * (2048 + 2 * gq8::kMaxHeads) * sizeof(double);
constexpr int kNoAllocMaxDevices = 64;
}

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratchMutex;
void *g_scratchAddress[kNoAllocMaxDevices] = {};

// The calling thread's current device's address of `scratch`, resolved once.
int scratch_address(void **out)
{
    int device = 0;
    GQ8_HIP(hipGetDevice(&device));
    if (device < 0 || device >= kNoAllocMaxDevices)
        return fail(GQ8_ERR_DEVICE, "mqa_decode_noalloc: device ordinal past the table");
    std::lock_guard<std::mutex> lock(g_scratchMutex);
    if (!g_scratchAddress[device]) {
        void *address = nullptr;
        GQ8_HIP(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)));
        if (!address)
            return fail(GQ8_ERR_DEVICE, "mqa_decode_noalloc: no device address for the scratch array");
        g_scratchAddress[device] = address;
    }
    *out = g_scratchAddress[device];
    return GQ8_OK;
}
} // namespace

extern "C" size_t gq8_mqa_decode_noalloc_limit_bytes(void)
{
    return kNoAllocScratchBytes;
}

extern "C" int gq8_mqa_decode_noalloc(const float *query, const uint16_t *key_cache,
                                      const uint16_t *value_cache, int heads, int kv_heads,
                                      int head_dim, int key_count, float scale, float *out,
                                      void *stream)
{
    if (int s = check_attention_shape(heads, kv_heads, head_dim))
        return s;
    if (!query || !key_cache || !value_cache || !out || key_count < 1)
        return fail(GQ8_ERR_ARGUMENT, "mqa_decode_noalloc: bad arguments");
    // check_attention_shape (at most 16 heads, a 2048-wide query row) keeps
    // every accepted shape's partials within the array: a guard, not a rule
    const size_t needed = gq8::mqa_workspace_bytes(1, heads, head_dim, key_count);
    if (needed > kNoAllocScratchBytes)
        return fail(GQ8_ERR_ARGUMENT, "mqa_decode_noalloc: the split partials need "
                                          + std::to_string(needed) + " bytes, past the "
                                          + std::to_string(kNoAllocScratchBytes)
                                          + "-byte static scratch");
    void *workspace = nullptr;
    if (int s = scratch_address(&workspace))
        return s;
    GQ8_LAUNCH(gq8::launch_mqa(query, heads * head_dim, key_cache, value_cache, heads, kv_heads,
                               head_dim, 1, nullptr, key_count - 1, key_count, scale, out, nullptr,
                               workspace, kNoAllocScratchBytes, as_stream(stream)));
    return GQ8_OK;
}

extern "C" int gq8_mqa_prefill(const float *queries, const uint16_t *key_cache,
                               const uint16_t *value_cache, int heads, int kv_heads,
                               int head_dim, int rows, int position_offset, float scale,
                               float *out, void *workspace, size_t workspace_bytes, void *stream)
{
    if (int s = check_attention_shape(heads, kv_heads, head_dim))
        return s;
    if (!queries || !key_cache || !value_cache || !out || !workspace || rows < 1
        || position_offset < 0)
        return fail(GQ8_ERR_ARGUMENT, "mqa_prefill: bad arguments");
    const int maxKeys = position_offset + rows;
    if (workspace_bytes < gq8::mqa_workspace_bytes(rows, heads, head_dim, maxKeys))
        return fail(GQ8_ERR_ARGUMENT, "mqa_prefill: workspace too small");
    GQ8_LAUNCH(gq8::launch_mqa(queries, heads * head_dim, key_cache, value_cache, heads, kv_heads,
                               head_dim, rows, nullptr, position_offset, maxKeys, scale, out,
                               nullptr, workspace, workspace_bytes, as_stream(stream)));
    return GQ8_OK;
}

extern "C" int gq8_geglu(const float *fused, int rows, int intermediate, float *out, uint8_t *q8,
                         void *stream)
{
    if (!fused || (!out && !q8) || rows <= 0 || intermediate <= 0
        || intermediate % gq8::kBlock != 0)
        return fail(GQ8_ERR_ARGUMENT, "geglu: bad arguments");
    GQ8_LAUNCH(gq8::launch_geglu(fused, rows, intermediate, out, q8, as_stream(stream)));
    return GQ8_OK;
}

extern "C" size_t gq8_argmax_workspace_bytes(int rows, int length)
{
    return gq8::argmax_workspace_bytes(rows, length);
}

extern "C" size_t gq8_sample_workspace_bytes(int vocab)
{
    // the sort's buffers, then one draw and its index
    return vocab > 0 ? std::max(gq8::sample_workspace_bytes(vocab) + 256,
                                gq8::argmax_workspace_bytes(1, vocab))
                     : 0;
}

extern "C" int gq8_sample_row(const float *logits, const float *mask, int vocab,
                              const gq8_sampling *options, double uniform, uint32_t *token,
                              void *workspace, size_t workspace_bytes, void *stream)
{
    if (!logits || !options || !token || !workspace)
        return fail(GQ8_ERR_ARGUMENT, "sample_row: null argument");
    if (vocab <= 0)
        return fail(GQ8_ERR_EMPTY, "Cannot sample from an empty row of logits");
    if (int st = sampling_error(*options))
        return st;
    if (workspace_bytes < gq8_sample_workspace_bytes(vocab))
        return fail(GQ8_ERR_ARGUMENT, "sample_row: workspace too small");
    if (!(uniform >= 0.0 && uniform < 1.0))
        return fail(GQ8_ERR_ARGUMENT, "sample_row: the draw lies outside [0, 1)");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (options->temperature == 0.f) { // Sampler.cpp:84-85
        GQ8_LAUNCH(gq8::launch_argmax(logits, mask, 1, vocab, token, nullptr, 0, workspace,
                                      gq8::argmax_workspace_bytes(1, vocab), st));
        return GQ8_OK;
    }
    const size_t sortBytes = gq8::sample_workspace_bytes(vocab);
    auto *tail = reinterpret_cast<uint8_t *>(workspace) + sortBytes;
    auto *draw = reinterpret_cast<double *>(tail);
    auto *index = reinterpret_cast<int *>(tail + sizeof(double));
    struct {
        double u;
        int index;
    } host{uniform, 0};
    GQ8_HIP(hipMemcpyAsync(draw, &host, sizeof(host), hipMemcpyHostToDevice, st));
    gq8::SampleArgs a{};
    a.logits = logits;
    a.mask = mask;
    a.vocab = vocab;
    a.temperature = options->temperature;
    a.top_k = options->top_k;
    a.top_p = options->top_p;
    a.draws = draw;
    a.draw_count = 1;
    a.draw_index = index;
    a.token_out = token;
    GQ8_LAUNCH(gq8::launch_sample(a, workspace, sortBytes, st));
    // the draw is read from host memory that ends with this call
    GQ8_HIP(hipStreamSynchronize(st));
    return GQ8_OK;
}

extern "C" int gq8_argmax_rows(const float *logits, const float *mask, int rows, int length,
                               uint32_t *indices, void *workspace, size_t workspace_bytes,
                               void *stream)
{
    if (!logits || !indices || !workspace || rows <= 0 || length <= 0)
        return fail(GQ8_ERR_ARGUMENT, "argmax: bad arguments");
    if (workspace_bytes < gq8::argmax_workspace_bytes(rows, length))
        return fail(GQ8_ERR_ARGUMENT, "argmax: workspace too small");
    GQ8_LAUNCH(gq8::launch_argmax(logits, mask, rows, length, indices, nullptr, 0, workspace,
                                  workspace_bytes, as_stream(stream)));
    return GQ8_OK;
}

// ============================================================================
// Decoder
// ============================================================================
namespace {
enum Role { kQ = 0, kK, kV, kO, kGate, kUp, kDown, kInputNorm, kPostNorm, kPerLayer };
}

struct gq8_decoder {
    gq8_shape shape{};
    int capacity = 0; // step rows
    int qWidth = 0, kvWidth = 0, qkvWidth = 0, maxInner = 0;
    hipStream_t stream = nullptr;

    uint8_t *embedding = nullptr;
    std::vector<uint8_t *> qkv, out, gateUp, down; // layer l at the kind's base + l * stride
    std::vector<float *> inputNorm, postNorm;
    int64_t qkvStride = 0, outStride = 0, gateUpStride = 0, downStride = 0; // bytes
    int64_t normStride = 0;                                                 // floats
    float *finalNorm = nullptr;
    std::vector<char> present;
    uint64_t weightVersion = 0; // bumped by every weight upload (copies made from them go stale)

    uint16_t *keyCache = nullptr, *valueCache = nullptr;
    float *cosines = nullptr, *sines = nullptr;

    float *hidden = nullptr, *normalisedRows = nullptr, *qkvRows = nullptr, *fused = nullptr;
    uint8_t *x8 = nullptr;
    void *attentionWorkspace = nullptr;
    size_t attentionWorkspaceBytes = 0;
    void *argmaxWorkspace = nullptr;
    size_t argmaxWorkspaceBytes = 0;
    float *logits = nullptr; // one vocabulary row, for the greedy loop
    uint32_t *sequence = nullptr;
    int *position = nullptr; // device copy of the position
    int hostPosition = 0;
    uint32_t *pinnedToken = nullptr;

    bool debug = false;
    float *debugValues = nullptr; // (layers + 1) x 4 x maxInner
    uint8_t *debugQ8 = nullptr;   // (layers + 1) x 4 x q8_bytes(1, maxInner)
    float *debugAttended = nullptr, *debugActivated = nullptr, *debugNormalised = nullptr;

    // the fused one-token path
    bool useFused = true;
    bool fusedSupported = false;
    bool splitAttention = false; // its attention is the split kernel (else partial/merge)
    // the decode attention's tagged split partials, their tag epoch and the
    // error word its bounded waits set
    uint64_t *attnPart = nullptr, *attnMl = nullptr;
    uint32_t *attnEpoch = nullptr;
    int *attnError = nullptr;
    unsigned long long *headBest = nullptr; // the lm_head argmax slots

    // sampling (Gemma::setSampling, Gemma.cpp:198-202): the options, and the
    // seed's Sampler::uniform draws, one a sampled token of a sequence
    gq8_sampling sampling{0.f, 0, 1.f, 0};
    double *draws = nullptr; // max_positions draws
    int *drawIndex = nullptr;
    void *sampleWorkspace = nullptr;
    size_t sampleWorkspaceBytes = 0;

    // the captured one-token step, one a key-count range (the attention
    // launch is sized to its range: gq8::attention_grid_splits)
    static constexpr int kGraphRanges = gq8::kAttentionRanges;
    hipGraphExec_t graphs[kGraphRanges] = {};
    bool capturing = false;
    int captureKeys = 0; // while capturing: the largest key count of the range

    unsigned timing = 0; // bit s: bracket stage s with events
    struct Mark {
        int stage;
        hipEvent_t start, stop;
    };
    std::vector<Mark> marks;
    std::vector<hipEvent_t> spareEvents;

    std::vector<void *> allocations;
};

namespace {

// Destroys the captured steps once the decoder's stream has finished every
// replay it holds (a replay still in flight keeps using its executable graph).
void drop_graphs(gq8_decoder *d)
{
    bool any = false;
    for (hipGraphExec_t g : d->graphs)
        any = any || g != nullptr;
    if (!any)
        return;
    if (d->stream)
        (void) hipStreamSynchronize(d->stream);
    for (hipGraphExec_t &g : d->graphs)
        if (g) {
            (void) hipGraphExecDestroy(g);
            g = nullptr;
        }
}

bool sampled(const gq8_decoder *d)
{
    return d->sampling.temperature > 0.f;
}

int64_t fused_rows_offset(const gq8_decoder *d, int role)
{
    switch (role) {
    case kK: return d->qWidth;
    case kV: return d->qWidth + d->kvWidth;
    case kUp: return d->shape.intermediate;
    default: return 0;
    }
}

int device_alloc(gq8_decoder *d, void **out, size_t bytes)
{
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void) hipGetLastError();
        return fail(GQ8_ERR_MEMORY, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    d->allocations.push_back(p);
    *out = p;
    return GQ8_OK;
}

template <typename T>
int alloc_as(gq8_decoder *d, T **out, size_t bytes)
{
    void *p = nullptr;
    int s = device_alloc(d, &p, bytes);
    *out = reinterpret_cast<T *>(p);
    return s;
}

bool is_final_norm(const gq8_shape *s, int index)
{
    return index == 1 + kPerLayer * s->layers;
}

} // namespace

extern "C" int gq8_tensor_count(const gq8_shape *shape)
{
    return shape ? 2 + kPerLayer * shape->layers : 0;
}

extern "C" int gq8_tensor_is_norm(const gq8_shape *s, int index)
{
    if (!s || index <= 0)
        return 0;
    if (is_final_norm(s, index))
        return 1;
    const int role = (index - 1) % kPerLayer;
    return role == kInputNorm || role == kPostNorm;
}

extern "C" int64_t gq8_tensor_elements(const gq8_shape *s, int index)
{
    if (!s || index < 0 || index >= gq8_tensor_count(s))
        return -1;
    const int64_t w = s->width, q = (int64_t) s->heads * s->head_dim,
                  kv = (int64_t) s->kv_heads * s->head_dim, f = s->intermediate;
    if (index == 0)
        return (int64_t) s->vocab * w;
    if (is_final_norm(s, index))
        return w;
    switch ((index - 1) % kPerLayer) {
    case kQ: return q * w;
    case kK: case kV: return kv * w;
    case kO: return w * q;
    case kGate: case kUp: return f * w;
    case kDown: return w * f;
    default: return w;
    }
}

static int64_t tensor_inner(const gq8_shape *s, int index)
{
    if (index == 0)
        return s->width;
    switch ((index - 1) % kPerLayer) {
    case kO: return (int64_t) s->heads * s->head_dim;
    case kDown: return s->intermediate;
    default: return s->width;
    }
}

extern "C" int gq8_shape_validate(const gq8_shape *s)
{
    if (!s)
        return fail(GQ8_ERR_ARGUMENT, "null shape");
    const int fields[] = {s->width, s->heads, s->kv_heads, s->head_dim, s->layers,
                          s->intermediate, s->vocab, s->max_positions};
    const char *names[] = {"width", "heads", "kvHeads", "headWidth", "layers",
                           "intermediate", "vocabularySize", "maxPositions"};
    for (int i = 0; i < 8; ++i)
        if (fields[i] <= 0)
            return fail(GQ8_ERR_SHAPE, std::string("a decoder shape's '") + names[i]
                                           + "' must be positive");
    if (s->max_step_rows < 0 || s->max_step_rows > s->max_positions)
        return fail(GQ8_ERR_SHAPE, "step capacity must be 0..maxPositions");
    if (s->head_dim % 4 != 0 || s->head_dim > gq8::kMaxHeadDim)
        return fail(GQ8_ERR_SHAPE, "head width must be a multiple of four and at most 256");
    if (s->heads % s->kv_heads != 0)
        return fail(GQ8_ERR_SHAPE, "kv heads must divide the query heads");
    if (int st = check_attention_shape(s->heads, s->kv_heads, s->head_dim))
        return st;
    for (int i = 0; i < gq8_tensor_count(s); ++i)
        if (!gq8_tensor_is_norm(s, i)
            && !gq8_quantizes_as_int8_blocks(tensor_inner(s, i), gq8_tensor_elements(s, i)))
            return fail(GQ8_ERR_UNQUANTIZABLE, "tensor " + std::to_string(i)
                                                   + " cannot be stored as Int8Blocks");
    if (s->width > 16384 || s->intermediate > 16384 || s->heads * s->head_dim > 16384)
        return fail(GQ8_ERR_SHAPE, "product inner extents are limited to 16384");
    return GQ8_OK;
}

extern "C" gq8_shape gq8_gemma_2b_shape(int layers, int max_positions, int max_step_rows)
{
    gq8_shape s{};
    s.width = 2048;
    s.heads = 8;
    s.kv_heads = 1;
    s.head_dim = 256;
    s.layers = layers;
    s.intermediate = 16384;
    s.vocab = 256000;
    s.max_positions = max_positions;
    s.max_step_rows = max_step_rows;
    s.rms_epsilon = 1e-6f;
    s.rope_theta = 10000.0;
    s.embedding_scale = std::sqrt((float) s.width); // GemmaConfig.cpp:123-126
    return s;
}

extern "C" void gq8_decoder_destroy(gq8_decoder *d)
{
    if (!d)
        return;
    drop_graphs(d);
    if (d->stream)
        (void) hipStreamSynchronize(d->stream);
    for (auto &m : d->marks) {
        (void) hipEventDestroy(m.start);
        (void) hipEventDestroy(m.stop);
    }
    for (auto e : d->spareEvents)
        (void) hipEventDestroy(e);
    for (void *p : d->allocations)
        (void) hipFree(p);
    if (d->pinnedToken)
        (void) hipHostFree(d->pinnedToken);
    if (d->stream)
        (void) hipStreamDestroy(d->stream);
    delete d;
}

extern "C" int gq8_decoder_create(const gq8_shape *shape, gq8_decoder **out)
{
    if (!out)
        return fail(GQ8_ERR_ARGUMENT, "null output");
    *out = nullptr;
    if (int s = gq8_shape_validate(shape))
        return s;

    gq8_decoder *d = new gq8_decoder();
    d->shape = *shape;
    const gq8_shape &s = d->shape;
    d->capacity = s.max_step_rows > 0 ? s.max_step_rows : s.max_positions;
    d->qWidth = s.heads * s.head_dim;
    d->kvWidth = s.kv_heads * s.head_dim;
    d->qkvWidth = d->qWidth + 2 * d->kvWidth;
    d->maxInner = std::max({s.width, d->qWidth, s.intermediate});

    auto cleanup = [&](int status) {
        gq8_decoder_destroy(d);
        return status;
    };
    if (hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking) != hipSuccess)
        return cleanup(fail(GQ8_ERR_DEVICE, "hipStreamCreate failed"));

    const int64_t W = s.width, R = d->capacity, L = s.layers;
    int st = GQ8_OK;
#define GQ8_ALLOC(ptr, bytes)                                \
    if ((st = alloc_as(d, &(ptr), (size_t) (bytes))) != 0) \
        return cleanup(st)

    GQ8_ALLOC(d->embedding, gq8_int8_blocks_byte_count((int64_t) s.vocab * W));
    d->qkv.resize(L);
    d->out.resize(L);
    d->gateUp.resize(L);
    d->down.resize(L);
    d->inputNorm.resize(L);
    d->postNorm.resize(L);
    // one allocation a tensor kind, the layers at a fixed 256-byte-aligned
    // stride (the step kernel addresses a layer as base + l * stride)
    auto stride_of = [](int64_t bytes) { return (bytes + 255) / 256 * 256; };
    d->qkvStride = stride_of(gq8_int8_blocks_byte_count((int64_t) d->qkvWidth * W));
    d->outStride = stride_of(gq8_int8_blocks_byte_count((int64_t) W * d->qWidth));
    d->gateUpStride = stride_of(gq8_int8_blocks_byte_count(2 * (int64_t) s.intermediate * W));
    d->downStride = stride_of(gq8_int8_blocks_byte_count((int64_t) W * s.intermediate));
    d->normStride = stride_of((int64_t) W * sizeof(float)) / (int64_t) sizeof(float);
    uint8_t *qkvBase = nullptr, *outBase = nullptr, *gateUpBase = nullptr, *downBase = nullptr;
    float *inputNormBase = nullptr, *postNormBase = nullptr;
    GQ8_ALLOC(qkvBase, d->qkvStride * L);
    GQ8_ALLOC(outBase, d->outStride * L);
    GQ8_ALLOC(gateUpBase, d->gateUpStride * L);
    GQ8_ALLOC(downBase, d->downStride * L);
    GQ8_ALLOC(inputNormBase, d->normStride * L * sizeof(float));
    GQ8_ALLOC(postNormBase, d->normStride * L * sizeof(float));
    for (int l = 0; l < L; ++l) {
        d->qkv[l] = qkvBase + d->qkvStride * l;
        d->out[l] = outBase + d->outStride * l;
        d->gateUp[l] = gateUpBase + d->gateUpStride * l;
        d->down[l] = downBase + d->downStride * l;
        d->inputNorm[l] = inputNormBase + d->normStride * l;
        d->postNorm[l] = postNormBase + d->normStride * l;
    }
    GQ8_ALLOC(d->finalNorm, W * sizeof(float));
    d->present.assign(gq8_tensor_count(&s), 0);

    const int64_t cacheElements = L * (int64_t) s.max_positions * d->kvWidth;
    GQ8_ALLOC(d->keyCache, cacheElements * sizeof(uint16_t));
    GQ8_ALLOC(d->valueCache, cacheElements * sizeof(uint16_t));

    const int64_t tableElements = (int64_t) s.max_positions * (s.head_dim / 2);
    GQ8_ALLOC(d->cosines, tableElements * sizeof(float));
    GQ8_ALLOC(d->sines, tableElements * sizeof(float));
    {
        std::vector<float> c(tableElements), sn(tableElements);
        gq8_rotary_table_host(s.max_positions, s.head_dim, s.rope_theta, c.data(), sn.data());
        if (hipMemcpy(d->cosines, c.data(), tableElements * sizeof(float), hipMemcpyHostToDevice)
                != hipSuccess
            || hipMemcpy(d->sines, sn.data(), tableElements * sizeof(float), hipMemcpyHostToDevice)
                   != hipSuccess)
            return cleanup(fail(GQ8_ERR_DEVICE, "rotary table upload failed"));
    }

    GQ8_ALLOC(d->hidden, R * W * sizeof(float));
    GQ8_ALLOC(d->normalisedRows, R * W * sizeof(float));
    GQ8_ALLOC(d->qkvRows, R * d->qkvWidth * sizeof(float));
    GQ8_ALLOC(d->fused, R * 2 * (int64_t) s.intermediate * sizeof(float));
    GQ8_ALLOC(d->x8, gq8::q8_bytes(R, d->maxInner));
    d->attentionWorkspaceBytes = gq8::mqa_workspace_bytes((int) R, s.heads, s.head_dim,
                                                          s.max_positions);
    GQ8_ALLOC(d->attentionWorkspace, d->attentionWorkspaceBytes);
    d->argmaxWorkspaceBytes = gq8::argmax_workspace_bytes(1, s.vocab);
    GQ8_ALLOC(d->argmaxWorkspace, d->argmaxWorkspaceBytes);
    GQ8_ALLOC(d->logits, (size_t) s.vocab * sizeof(float));
    GQ8_ALLOC(d->sequence, ((size_t) s.max_positions + 1) * sizeof(uint32_t));
    GQ8_ALLOC(d->position, sizeof(int));
    GQ8_ALLOC(d->debugValues, (size_t) (L + 1) * 4 * d->maxInner * sizeof(float));
    GQ8_ALLOC(d->debugQ8, (size_t) (L + 1) * 4 * gq8::q8_bytes(1, d->maxInner));
    GQ8_ALLOC(d->debugNormalised, R * W * sizeof(float));
    GQ8_ALLOC(d->debugAttended, R * d->qWidth * sizeof(float));
    GQ8_ALLOC(d->debugActivated, R * (int64_t) s.intermediate * sizeof(float));
    d->fusedSupported = gq8::fused_decode_supported(s.width, s.heads, s.kv_heads, s.head_dim,
                                                    s.intermediate);
    {
        // the split attention's workgroups wait on each other: it is taken
        // only where every launch the window reaches fits on the device at once
        int device = 0, resident[gq8::kAttentionRanges] = {};
        d->splitAttention = d->fusedSupported && hipGetDevice(&device) == hipSuccess
                            && gq8::split_attention_resident(device, s.heads, s.kv_heads, s.head_dim,
                                                             s.max_positions, resident)
                            && gq8::split_attention_fits(s.heads, s.kv_heads, s.head_dim,
                                                         s.max_positions, resident);
    }
    {
        const size_t partBytes = (size_t) gq8::kDecodeSplits * d->qWidth * 2 * sizeof(uint64_t);
        const size_t mlBytes = (size_t) gq8::kDecodeSplits * s.heads * 4 * sizeof(uint64_t);
        GQ8_ALLOC(d->attnPart, partBytes);
        GQ8_ALLOC(d->attnMl, mlBytes);
        GQ8_ALLOC(d->attnEpoch, 64 * sizeof(uint32_t));
        GQ8_ALLOC(d->attnError, 64 * sizeof(int));
        if (hipMemset(d->attnPart, 0, partBytes) != hipSuccess
            || hipMemset(d->attnMl, 0, mlBytes) != hipSuccess
            || hipMemset(d->attnEpoch, 0, 64 * sizeof(uint32_t)) != hipSuccess
            || hipMemset(d->attnError, 0, 64 * sizeof(int)) != hipSuccess)
            return cleanup(fail(GQ8_ERR_DEVICE, "attention state: initialisation failed"));
        GQ8_ALLOC(d->headBest, gq8::kHeadSlots * gq8::kHeadSlotStride * sizeof(unsigned long long));
    }
#undef GQ8_ALLOC
    if (hipHostMalloc((void **) &d->pinnedToken, sizeof(uint32_t) * 4) != hipSuccess)
        return cleanup(fail(GQ8_ERR_MEMORY, "pinned allocation failed"));
    if (hipMemset(d->sequence, 0, ((size_t) s.max_positions + 1) * sizeof(uint32_t)) != hipSuccess
        || hipMemset(d->position, 0, sizeof(int)) != hipSuccess
        || hipMemset(d->headBest, 0, gq8::kHeadSlots * gq8::kHeadSlotStride * sizeof(unsigned long long))
               != hipSuccess
        || hipMemset(d->keyCache, 0, cacheElements * sizeof(uint16_t)) != hipSuccess
        || hipMemset(d->valueCache, 0, cacheElements * sizeof(uint16_t)) != hipSuccess
        || hipDeviceSynchronize() != hipSuccess)
        return cleanup(fail(GQ8_ERR_DEVICE, "initialisation failed"));
    *out = d;
    return GQ8_OK;
}

// Where tensor `index` lives: the device bytes of its own region inside the
// fused q|k|v or gate|up tensor (quantized) or its fp32 norm buffer.
namespace {
struct Placement {
    uint8_t *q = nullptr;        // first quantized byte
    uint16_t *scales = nullptr;  // first scale
    float *values = nullptr;     // norms
    int64_t elements = 0;
};

Placement placement(gq8_decoder *d, int index)
{
    const gq8_shape &s = d->shape;
    Placement p;
    p.elements = gq8_tensor_elements(&s, index);
    if (index == 0) {
        p.q = d->embedding;
        p.scales = reinterpret_cast<uint16_t *>(d->embedding + p.elements);
        return p;
    }
    if (is_final_norm(&s, index)) {
        p.values = d->finalNorm;
        return p;
    }
    const int layer = (index - 1) / kPerLayer, role = (index - 1) % kPerLayer;
    const int64_t W = s.width;
    uint8_t *base = nullptr;
    int64_t total = 0, rowOffset = fused_rows_offset(d, role), inner = W;
    switch (role) {
    case kQ: case kK: case kV:
        base = d->qkv[layer];
        total = (int64_t) d->qkvWidth * W;
        break;
    case kGate: case kUp:
        base = d->gateUp[layer];
        total = 2 * (int64_t) s.intermediate * W;
        break;
    case kO:
        base = d->out[layer];
        total = W * d->qWidth;
        inner = d->qWidth;
        break;
    case kDown:
        base = d->down[layer];
        total = W * s.intermediate;
        inner = s.intermediate;
        break;
    case kInputNorm: p.values = d->inputNorm[layer]; return p;
    default: p.values = d->postNorm[layer]; return p;
    }
    p.q = base + rowOffset * inner;
    p.scales = reinterpret_cast<uint16_t *>(base + total) + rowOffset * inner / gq8::kBlock;
    return p;
}

int mark_present(gq8_decoder *d, int index)
{
    d->present[index] = 1;
    ++d->weightVersion;
    return GQ8_OK;
}
} // namespace

// fp32 values (host) -> device, quantized on the device in pieces.
static int upload_values(gq8_decoder *d, int index, const float *host, int64_t first,
                         int64_t count, float *staging)
{
    Placement p = placement(d, index);
    if (p.values) {
        GQ8_HIP(hipMemcpyAsync(p.values + first, host, count * sizeof(float), hipMemcpyHostToDevice,
                               d->stream));
        return GQ8_OK;
    }
    GQ8_HIP(hipMemcpyAsync(staging, host, count * sizeof(float), hipMemcpyHostToDevice, d->stream));
    GQ8_LAUNCH(gq8::launch_quantize(staging, count, p.q + first, p.scales + first / gq8::kBlock,
                                    d->stream));
    return GQ8_OK;
}

extern "C" int gq8_decoder_load_tensor(gq8_decoder *d, int index, const float *host_values)
{
    if (!d || !host_values || index < 0 || index >= gq8_tensor_count(&d->shape))
        return fail(GQ8_ERR_ARGUMENT, "load_tensor: bad arguments");
    const int64_t elements = gq8_tensor_elements(&d->shape, index);
    const int64_t piece = int64_t(64) << 20;
    float *staging = nullptr;
    if (!gq8_tensor_is_norm(&d->shape, index))
        GQ8_HIP(hipMalloc(&staging, std::min(piece, elements) * sizeof(float)));
    int status = GQ8_OK;
    for (int64_t first = 0; first < elements && status == GQ8_OK; first += piece) {
        const int64_t count = std::min(piece, elements - first);
        status = upload_values(d, index, host_values + first, first, count, staging);
        if (status == GQ8_OK && hipStreamSynchronize(d->stream) != hipSuccess)
            status = fail(GQ8_ERR_DEVICE, "load_tensor: synchronize failed");
    }
    if (staging)
        (void) hipFree(staging);
    return status == GQ8_OK ? mark_present(d, index) : status;
}

extern "C" int gq8_decoder_load_tensor_q8(gq8_decoder *d, int index, const uint8_t *host_bytes)
{
    if (!d || !host_bytes || index < 0 || index >= gq8_tensor_count(&d->shape))
        return fail(GQ8_ERR_ARGUMENT, "load_tensor_q8: bad arguments");
    if (gq8_tensor_is_norm(&d->shape, index))
        return fail(GQ8_ERR_ARGUMENT, "load_tensor_q8: norms are fp32 tensors");
    Placement p = placement(d, index);
    GQ8_HIP(hipMemcpy(p.q, host_bytes, p.elements, hipMemcpyHostToDevice));
    GQ8_HIP(hipMemcpy(p.scales, host_bytes + p.elements, p.elements / 16, hipMemcpyHostToDevice));
    return mark_present(d, index);
}

namespace {
// The checkpoint's name for catalogue entry `index` (GemmaTensors.h:29-44).
std::string checkpoint_name(const gq8_shape &s, int index)
{
    if (index == 0)
        return "model.embed_tokens.weight";
    if (is_final_norm(&s, index))
        return "model.norm.weight";
    static const char *const suffix[kPerLayer] = {
        "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
        "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
        "mlp.down_proj.weight", "input_layernorm.weight", "post_attention_layernorm.weight"};
    return "model.layers." + std::to_string((index - 1) / kPerLayer) + "." + suffix[(index - 1) % kPerLayer];
}

// HuggingFace stores a linear weight as [outputs, inputs] (GemmaTensors.h:13-16).
std::vector<int64_t> checkpoint_dims(const gq8_shape &s, int index)
{
    const int64_t w = s.width, q = (int64_t) s.heads * s.head_dim,
                  kv = (int64_t) s.kv_heads * s.head_dim, f = s.intermediate;
    if (index == 0)
        return {s.vocab, w};
    if (is_final_norm(&s, index))
        return {w};
    switch ((index - 1) % kPerLayer) {
    case kQ: return {q, w};
    case kK: case kV: return {kv, w};
    case kO: return {w, q};
    case kGate: case kUp: return {f, w};
    case kDown: return {w, f};
    default: return {w};
    }
}

std::string dims_text(const std::vector<int64_t> &dims)
{
    std::string t = "[";
    for (size_t i = 0; i < dims.size(); ++i)
        t += (i ? ", " : "") + std::to_string(dims[i]);
    return t + "]";
}
} // namespace

extern "C" int gq8_decoder_load_safetensors(gq8_decoder *d, gq8_safetensors *const *shards,
                                            int shard_count)
{
    if (!d || !shards || shard_count <= 0)
        return fail(GQ8_ERR_ARGUMENT, "load_safetensors: bad arguments");
    const gq8_shape &s = d->shape;
    const int count = gq8_tensor_count(&s);
    // every tensor found and checked before a byte is uploaded
    std::vector<std::pair<const gq8::SafeTensorsFile *, const gq8::TensorInfo *>> found(count);
    for (int i = 0; i < count; ++i) {
        const std::string name = checkpoint_name(s, i);
        for (int k = 0; k < shard_count && !found[i].first; ++k) {
            const gq8::SafeTensorsFile *f = gq8::file_of(shards[k]);
            if (!f)
                return fail(GQ8_ERR_ARGUMENT, "load_safetensors: null shard");
            const int at = f->find(name);
            if (at >= 0)
                found[i] = {f, &f->tensors()[at]};
        }
        if (!found[i].first)
            return fail(GQ8_ERR_FORMAT, "the checkpoint has no tensor '" + name + "'");
        const gq8::TensorInfo &t = *found[i].second;
        const std::vector<int64_t> want = checkpoint_dims(s, i);
        if (t.shape != want)
            return fail(GQ8_ERR_FORMAT, "tensor '" + name + "' is " + dims_text(t.shape)
                                            + ", the config implies " + dims_text(want));
        if (t.dtype != gq8::kF32 && t.dtype != gq8::kF16 && t.dtype != gq8::kBF16
            && t.dtype != gq8::kF64)
            return fail(GQ8_ERR_FORMAT, "tensor '" + name + "' is " + gq8::dtype_name(t.dtype)
                                            + ", not a floating-point tensor");
    }
    const int64_t piece = int64_t(16) << 20; // elements a piece (a multiple of the block)
    float *host = nullptr, *staging = nullptr;
    if (hipHostMalloc(reinterpret_cast<void **>(&host), piece * sizeof(float)) != hipSuccess) {
        (void) hipGetLastError();
        return fail(GQ8_ERR_MEMORY, "load_safetensors: pinned staging allocation failed");
    }
    int status = GQ8_OK;
    if (hipMalloc(&staging, piece * sizeof(float)) != hipSuccess) {
        (void) hipGetLastError();
        status = fail(GQ8_ERR_MEMORY, "load_safetensors: device staging allocation failed");
    }
    for (int i = 0; i < count && status == GQ8_OK; ++i) {
        const gq8::TensorInfo &t = *found[i].second;
        const int64_t elements = t.elements();
        for (int64_t first = 0; first < elements && status == GQ8_OK; first += piece) {
            const int64_t n = std::min(piece, elements - first);
            status = found[i].first->read_floats(t, first, n, host);
            if (status == GQ8_OK)
                status = upload_values(d, i, host, first, n, staging);
            if (status == GQ8_OK && hipStreamSynchronize(d->stream) != hipSuccess)
                status = fail(GQ8_ERR_DEVICE, "load_safetensors: synchronize failed");
        }
        if (status == GQ8_OK)
            mark_present(d, i);
    }
    if (staging)
        (void) hipFree(staging);
    (void) hipHostFree(host);
    return status;
}

extern "C" int gq8_decoder_fill_synthetic(gq8_decoder *d, int threads)
{
    if (!d)
        return fail(GQ8_ERR_ARGUMENT, "fill_synthetic: null decoder");
    threads = hardware_threads(threads);
    const int64_t piece = int64_t(64) << 20; // a whole number of 2^20 chunks
    float *host = nullptr;
    float *staging = nullptr;
    GQ8_HIP(hipHostMalloc((void **) &host, piece * sizeof(float)));
    if (hipMalloc(&staging, piece * sizeof(float)) != hipSuccess) {
        (void) hipHostFree(host);
        return fail(GQ8_ERR_MEMORY, "fill_synthetic: staging allocation failed");
    }
    int status = GQ8_OK;
    for (int index = 0; index < gq8_tensor_count(&d->shape) && status == GQ8_OK; ++index) {
        const int64_t elements = gq8_tensor_elements(&d->shape, index);
        const uint64_t seed = 0x5EED0000ULL + (uint64_t) index;
        const double sigma = gq8_tensor_is_norm(&d->shape, index) ? 0.1 : 0.02;
        for (int64_t first = 0; first < elements && status == GQ8_OK; first += piece) {
            const int64_t count = std::min(piece, elements - first);
            const int64_t chunk0 = first / kChunk;
            const int64_t chunks = (count + kChunk - 1) / kChunk;
            // the previous piece's copy reads `host`: finish it before refilling
            if (hipStreamSynchronize(d->stream) != hipSuccess) {
                status = fail(GQ8_ERR_DEVICE, "fill_synthetic: synchronize failed");
                break;
            }
            parallel_for(chunks, threads, [&](int64_t c) {
                normal_chunk(seed, sigma, chunk0 + c, elements, host + c * kChunk);
            });
            status = upload_values(d, index, host, first, count, staging);
        }
        if (status == GQ8_OK)
            mark_present(d, index);
    }
    if (hipStreamSynchronize(d->stream) != hipSuccess && status == GQ8_OK)
        status = fail(GQ8_ERR_DEVICE, "fill_synthetic: synchronize failed");
    (void) hipFree(staging);
    (void) hipHostFree(host);
    return status;
}

extern "C" int gq8_normal_fill_host(uint64_t tensor_seed, double sigma, float *out, int64_t count)
{
    if (count < 0 || (count > 0 && !out))
        return fail(GQ8_ERR_ARGUMENT, "normal_fill_host: bad arguments");
    const int64_t chunks = (count + kChunk - 1) / kChunk;
    parallel_for(chunks, hardware_threads(0), [&](int64_t c) {
        normal_chunk(tensor_seed, sigma, c, count, out + c * kChunk);
    });
    return GQ8_OK;
}

extern "C" int gq8_prompt_ids(uint64_t seed, int vocab, int count, int32_t *out)
{
    if (vocab <= 0 || count < 0 || (count > 0 && !out))
        return fail(GQ8_ERR_ARGUMENT, "prompt_ids: bad arguments");
    std::mt19937_64 engine(seed);
    for (int i = 0; i < count; ++i)
        out[i] = (int32_t) (engine() % (uint64_t) vocab);
    return GQ8_OK;
}

extern "C" int gq8_decoder_read_tensor(gq8_decoder *d, int index, void *host_out, size_t bytes)
{
    if (!d || !host_out || index < 0 || index >= gq8_tensor_count(&d->shape))
        return fail(GQ8_ERR_ARGUMENT, "read_tensor: bad arguments");
    Placement p = placement(d, index);
    if (p.values) {
        if (bytes < (size_t) p.elements * sizeof(float))
            return fail(GQ8_ERR_ARGUMENT, "read_tensor: buffer too small");
        GQ8_HIP(hipMemcpy(host_out, p.values, p.elements * sizeof(float), hipMemcpyDeviceToHost));
        return GQ8_OK;
    }
    if (bytes < (size_t) gq8_int8_blocks_byte_count(p.elements))
        return fail(GQ8_ERR_ARGUMENT, "read_tensor: buffer too small");
    uint8_t *h = reinterpret_cast<uint8_t *>(host_out);
    GQ8_HIP(hipMemcpy(h, p.q, p.elements, hipMemcpyDeviceToHost));
    GQ8_HIP(hipMemcpy(h + p.elements, p.scales, p.elements / 16, hipMemcpyDeviceToHost));
    return GQ8_OK;
}

extern "C" int gq8_decoder_begin_sequence(gq8_decoder *d)
{
    if (!d)
        return fail(GQ8_ERR_ARGUMENT, "null decoder");
    GQ8_HIP(hipStreamSynchronize(d->stream));
    d->hostPosition = 0;
    const int zero = 0;
    GQ8_HIP(hipMemcpy(d->position, &zero, sizeof(int), hipMemcpyHostToDevice));
    // every run draws from a freshly seeded generator (Gemma.cpp:549)
    if (d->drawIndex)
        GQ8_HIP(hipMemcpy(d->drawIndex, &zero, sizeof(int), hipMemcpyHostToDevice));
    return GQ8_OK;
}


extern "C" int gq8_decoder_set_sampling(gq8_decoder *d, const gq8_sampling *options)
{
    if (!d || !options)
        return fail(GQ8_ERR_ARGUMENT, "decoder_set_sampling: null argument");
    if (int st = sampling_error(*options))
        return st;
    const int count = d->shape.max_positions;
    if (options->temperature > 0.f && !d->draws) {
        if (int st = alloc_as(d, &d->draws, (size_t) count * sizeof(double)))
            return st;
        if (int st = alloc_as(d, &d->drawIndex, sizeof(int)))
            return st;
        d->sampleWorkspaceBytes = gq8::sample_workspace_bytes(d->shape.vocab);
        if (int st = device_alloc(d, &d->sampleWorkspace, d->sampleWorkspaceBytes))
            return st;
    }
    GQ8_HIP(hipStreamSynchronize(d->stream));
    if (options->temperature > 0.f) {
        std::vector<double> draws(count);
        uniform_draws(options->seed, count, draws.data());
        GQ8_HIP(hipMemcpy(d->draws, draws.data(), count * sizeof(double), hipMemcpyHostToDevice));
        const int zero = 0;
        GQ8_HIP(hipMemcpy(d->drawIndex, &zero, sizeof(int), hipMemcpyHostToDevice));
    }
    d->sampling = *options;
    drop_graphs(d); // a captured step keeps the chooser it was captured with
    return GQ8_OK;
}

extern "C" int gq8_decoder_position(const gq8_decoder *d)
{
    return d ? d->hostPosition : -1;
}

extern "C" int gq8_decoder_device_position(gq8_decoder *d)
{
    if (!d)
        return fail(GQ8_ERR_ARGUMENT, "decoder_device_position: null decoder");
    int position = 0;
    GQ8_HIP(hipStreamSynchronize(d->stream));
    GQ8_HIP(hipMemcpy(&position, d->position, sizeof(int), hipMemcpyDeviceToHost));
    return position;
}

extern "C" int gq8_decoder_attention_path(const gq8_decoder *d)
{
    if (!d)
        return fail(GQ8_ERR_ARGUMENT, "decoder_attention_path: null decoder");
    return d->fusedSupported ? (d->splitAttention ? 1 : 0) : -1;
}

extern "C" int gq8_decode_attention_fits(const gq8_shape *shape, int resident_workgroups)
{
    if (int s = gq8_shape_validate(shape))
        return s;
    const gq8_shape &s = *shape;
    int resident[gq8::kAttentionRanges];
    for (int &r : resident)
        r = resident_workgroups;
    return gq8::fused_decode_supported(s.width, s.heads, s.kv_heads, s.head_dim, s.intermediate)
                   && gq8::split_attention_fits(s.heads, s.kv_heads, s.head_dim, s.max_positions,
                                                resident)
               ? 1
               : 0;
}

extern "C" int gq8_decoder_inject_wait_failure(gq8_decoder *d)
{
    if (!d)
        return fail(GQ8_ERR_ARGUMENT, "decoder_inject_wait_failure: null decoder");
    if (!d->splitAttention)
        return fail(GQ8_ERR_SHAPE, "decoder_inject_wait_failure: the attention is not the split kernel");
    const int one = 1;
    GQ8_HIP(hipStreamSynchronize(d->stream));
    GQ8_HIP(hipMemcpy(d->attnError, &one, sizeof(int), hipMemcpyHostToDevice));
    return GQ8_OK;
}

extern "C" int gq8_decoder_set_fused(gq8_decoder *d, int enabled)
{
    if (!d)
        return fail(GQ8_ERR_ARGUMENT, "null decoder");
    d->useFused = enabled != 0;
    drop_graphs(d); // a captured step follows the path it was captured with
    return GQ8_OK;
}

extern "C" int gq8_decoder_set_debug(gq8_decoder *d, int enabled)
{
    if (!d)
        return fail(GQ8_ERR_ARGUMENT, "null decoder");
    d->debug = enabled != 0;
    return GQ8_OK;
}

namespace {

// The last row of a Q8 row buffer of `rows` x `inner` into a one-row buffer.
int copy_last_q8_row(gq8_decoder *d, const uint8_t *x8, int rows, int inner, uint8_t *dst)
{
    const int64_t elements = (int64_t) rows * inner;
    GQ8_HIP(hipMemcpyAsync(dst, x8 + (int64_t) (rows - 1) * inner, inner, hipMemcpyDeviceToDevice,
                           d->stream));
    GQ8_HIP(hipMemcpyAsync(dst + inner, x8 + elements + 2 * (int64_t) (rows - 1) * (inner / 32),
                           inner / 16, hipMemcpyDeviceToDevice, d->stream));
    return GQ8_OK;
}

int capture_debug(gq8_decoder *d, int which, int layer, const float *rowsValues, int rows,
                  int inner, const uint8_t *x8)
{
    const int64_t slot = (int64_t) layer * 4 + which;
    float *dst = d->debugValues + slot * d->maxInner;
    GQ8_HIP(hipMemcpyAsync(dst, rowsValues + (int64_t) (rows - 1) * inner, inner * sizeof(float),
                           hipMemcpyDeviceToDevice, d->stream));
    if (x8)
        return copy_last_q8_row(d, x8, rows, inner,
                                d->debugQ8 + slot * gq8::q8_bytes(1, d->maxInner));
    return GQ8_OK;
}

enum Stage {
    kStageEmbed = 0, kStageNorm, kStageQkv, kStageRope, kStageAttention, kStageO, kStageGateUp,
    kStageGeglu, kStageDown, kStageLogits, kStageArgmax
};

hipEvent_t take_event(gq8_decoder *d)
{
    if (!d->spareEvents.empty()) {
        hipEvent_t e = d->spareEvents.back();
        d->spareEvents.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess)
        return nullptr;
    return e;
}

// Brackets one launch group with events on the decoder's stream while
// stage timing is on and the step is not being captured.
struct StageTimer {
    gq8_decoder *d;
    int stage;
    hipEvent_t start = nullptr;
    StageTimer(gq8_decoder *decoder, int s) : d(decoder), stage(s)
    {
        if (s >= 0 && s < GQ8_STAGE_COUNT && ((d->timing >> s) & 1u) && !d->capturing) {
            start = take_event(d);
            if (start)
                (void) hipEventRecord(start, d->stream);
        }
    }
    ~StageTimer()
    {
        if (!start)
            return;
        hipEvent_t stop = take_event(d);
        if (!stop) {
            d->spareEvents.push_back(start);
            return;
        }
        (void) hipEventRecord(stop, d->stream);
        d->marks.push_back({stage, start, stop});
    }
};

#define GQ8_STAGE(stage, expr)                    \
    do {                                          \
        StageTimer timer_(d, stage);              \
        GQ8_LAUNCH(expr);                         \
    } while (0)

// The sample of one logits row; the id goes to slot *position + offset.
int encode_sample(gq8_decoder *d, const float *row, int offset)
{
    gq8::SampleArgs a{};
    a.logits = row;
    a.vocab = d->shape.vocab;
    a.temperature = d->sampling.temperature;
    a.top_k = d->sampling.top_k;
    a.top_p = d->sampling.top_p;
    a.draws = d->draws;
    a.draw_count = d->shape.max_positions;
    a.draw_index = d->drawIndex;
    a.sequence = d->sequence;
    a.position = d->position;
    a.offset = offset;
    GQ8_STAGE(kStageArgmax, gq8::launch_sample(a, d->sampleWorkspace, d->sampleWorkspaceBytes,
                                               d->stream));
    return GQ8_OK;
}


// Reads and clears the split attention's error word.  A set word means a
// bounded wait of a split merge gave up (or a launch was too small for its
// keys), so the steps enqueued since the last check are invalid: the device
// and host positions go back to `rollback`, the position before those steps,
// and the caller can run them again (their cache rows are rewritten).
int check_step_error(gq8_decoder *d, int rollback)
{
    if (!d->splitAttention)
        return GQ8_OK;
    int error = 0;
    GQ8_HIP(hipStreamSynchronize(d->stream));
    GQ8_HIP(hipMemcpy(&error, d->attnError, sizeof(int), hipMemcpyDeviceToHost));
    if (error == 0)
        return GQ8_OK;
    GQ8_HIP(hipMemset(d->attnError, 0, sizeof(int)));
    GQ8_HIP(hipMemcpy(d->position, &rollback, sizeof(int), hipMemcpyHostToDevice));
    d->hostPosition = rollback;
    return fail(GQ8_ERR_DEVICE, "decode attention: a split merge's wait gave up (the steps since "
                                "position " + std::to_string(rollback) + " are undone)");
}

// The one-token step through the fused kernels (gq8_decode.hip): five
// launches a layer and one for the head, which also chooses the next id and
// advances the device position.
int encode_fused_token(gq8_decoder *d, float *logits, bool sample)
{
    const gq8_shape &s = d->shape;
    const int W = s.width, F = s.intermediate;
    hipStream_t st = d->stream;
    const bool dbg = d->debug && !d->capturing;
    auto debugValues = [&](int which, int layer) {
        return dbg ? d->debugValues + ((int64_t) layer * 4 + which) * d->maxInner : nullptr;
    };
    auto debugQ8 = [&](int which, int layer) {
        return dbg ? d->debugQ8 + ((int64_t) layer * 4 + which) * gq8::q8_bytes(1, d->maxInner)
                   : nullptr;
    };

    for (int l = 0; l < s.layers; ++l) {
        const size_t layerCache = (size_t) l * s.max_positions * d->kvWidth;
        gq8::QkvArgs q{};
        q.hidden = d->hidden;
        q.sequence = d->sequence;
        q.embedding = l == 0 ? d->embedding : nullptr;
        q.vocab = s.vocab;
        q.embed_scale = s.embedding_scale;
        q.hidden_out = l == 0 ? d->hidden : nullptr;
        q.norm_weight = d->inputNorm[l];
        q.width = W;
        q.epsilon = s.rms_epsilon;
        q.weights = d->qkv[l];
        q.heads = s.heads;
        q.kv_heads = s.kv_heads;
        q.head_dim = s.head_dim;
        q.position = d->position;
        q.cosines = d->cosines;
        q.sines = d->sines;
        q.query = d->qkvRows;
        q.key_cache = d->keyCache + layerCache;
        q.value_cache = d->valueCache + layerCache;
        q.debug_normalised = debugValues(0, l);
        q.debug_q8 = debugQ8(0, l);
        q.tag_epoch = d->attnEpoch;
        GQ8_STAGE(kStageQkv, gq8::launch_qkv_rope(q, st));

        gq8::AttentionArgs at{};
        at.query = d->qkvRows;
        at.key_cache = q.key_cache;
        at.value_cache = q.value_cache;
        at.heads = s.heads;
        at.kv_heads = s.kv_heads;
        at.head_dim = s.head_dim;
        at.max_positions = s.max_positions;
        at.position = d->position;
        at.scale = 1.f / std::sqrt((float) s.head_dim);
        at.part_ll = d->attnPart;
        at.ml_ll = d->attnMl;
        at.tag_epoch = d->attnEpoch;
        at.error = d->attnError;
        at.out = debugValues(1, l);
        at.q8 = d->x8;
        const int rangeKeys = d->capturing ? d->captureKeys : d->hostPosition + 1;
        at.grid_splits = gq8::attention_grid_splits(rangeKeys);
        at.rounds = gq8::attention_rounds(rangeKeys);
        at.spec_keys = at.rounds * 32;
        if (d->splitAttention) {
            GQ8_STAGE(kStageAttention, gq8::launch_attention(at, st));
        } else {
            GQ8_STAGE(kStageAttention, gq8::launch_mqa(d->qkvRows, d->qWidth, q.key_cache, q.value_cache,
                                                       s.heads, s.kv_heads, s.head_dim, 1, d->position, 0,
                                                       s.max_positions, at.scale, at.out, d->x8,
                                                       d->attentionWorkspace,
                                                       d->attentionWorkspaceBytes, st));
        }
        if (dbg && copy_last_q8_row(d, d->x8, 1, d->qWidth, debugQ8(1, l)))
            return GQ8_ERR_DEVICE;

        GQ8_STAGE(kStageO, gq8::launch_q8_product(d->x8, 1, 0, 1, d->out[l], d->qWidth, W,
                                                  d->hidden, W, 1, st));

        gq8::GateUpArgs g{};
        g.hidden = d->hidden;
        g.norm_weight = d->postNorm[l];
        g.width = W;
        g.epsilon = s.rms_epsilon;
        g.weights = d->gateUp[l];
        g.intermediate = F;
        g.q8 = d->x8;
        g.debug_activated = debugValues(2, l);
        GQ8_STAGE(kStageGateUp, gq8::launch_gateup_geglu(g, st));
        if (dbg && copy_last_q8_row(d, d->x8, 1, F, debugQ8(2, l)))
            return GQ8_ERR_DEVICE;

        GQ8_STAGE(kStageDown, gq8::launch_q8_product(d->x8, 1, 0, 1, d->down[l], F, W, d->hidden,
                                                     W, 1, st));
        if (dbg && capture_debug(d, 3, l, d->hidden, 1, W, nullptr))
            return GQ8_ERR_DEVICE;
    }

    gq8::HeadArgs h{};
    h.hidden = d->hidden;
    h.norm_weight = d->finalNorm;
    h.width = W;
    h.epsilon = s.rms_epsilon;
    h.weights = d->embedding;
    h.vocab = s.vocab;
    h.logits = logits;
    h.normalised_out = d->normalisedRows;
    h.q8 = d->x8;
    h.best = d->headBest;
    h.sequence = sample && !sampled(d) ? d->sequence : nullptr;
    h.position = d->position;
    h.advance = 1;
    GQ8_STAGE(kStageLogits, gq8::launch_lmhead_argmax(h, st)); // the final norm included
    GQ8_STAGE(kStageArgmax, gq8::launch_head_finalize(h, st));
    // the position has advanced: the sample fills slot *position
    if (sample && sampled(d))
        if (int status = encode_sample(d, logits, 0))
            return status;
    if (dbg && copy_last_q8_row(d, d->x8, 1, W, debugQ8(0, s.layers)))
        return GQ8_ERR_DEVICE;
    if (dbg) {
        float *slot = d->debugValues + (int64_t) s.layers * 4 * d->maxInner;
        GQ8_HIP(hipMemcpyAsync(slot, d->normalisedRows, W * sizeof(float), hipMemcpyDeviceToDevice,
                               st));
    }
    return GQ8_OK;
}

// Decoder::step's recording (Decoder.cpp:579-706) for `rows` tokens read
// from the sequence slots at the device position; logits of the last
// logitsRows rows; with sample, the argmax of the last row is written to the
// slot after the step; the device position advances by rows.
int encode_step(gq8_decoder *d, int rows, float *logits, int logitsRows, bool sample)
{
    const gq8_shape &s = d->shape;
    const int W = s.width, F = s.intermediate;
    hipStream_t st = d->stream;
    const float attentionScale = 1.f / std::sqrt((float) s.head_dim);
    const bool dbg = d->debug;
    if (rows == 1 && logits && logitsRows == 1 && d->useFused && d->fusedSupported)
        return encode_fused_token(d, logits, sample);

    GQ8_STAGE(kStageEmbed, gq8::launch_embed(d->sequence, d->position, rows, d->embedding, s.vocab, W,
                                 s.embedding_scale, d->hidden, st));

    for (int l = 0; l < s.layers; ++l) {
        const size_t layerCache = (size_t) l * s.max_positions * d->kvWidth;
        uint16_t *keys = d->keyCache + layerCache;
        uint16_t *values = d->valueCache + layerCache;

        GQ8_STAGE(kStageNorm, gq8::launch_rmsnorm(d->hidden, d->inputNorm[l], rows, W, s.rms_epsilon,
                                       dbg ? d->debugNormalised : nullptr, d->x8, st));
        if (dbg && capture_debug(d, 0, l, d->debugNormalised, rows, W, d->x8))
            return GQ8_ERR_DEVICE;
        GQ8_STAGE(kStageQkv, gq8::launch_q8_product(d->x8, rows, 0, rows, d->qkv[l], W, d->qkvWidth,
                                          d->qkvRows, d->qkvWidth, 0, st));
        GQ8_STAGE(kStageRope, gq8::launch_rope_kv(d->qkvRows, d->qkvWidth, s.heads, s.kv_heads, s.head_dim,
                                       d->position, 0, rows, d->cosines, d->sines, keys, values,
                                       st));
        GQ8_STAGE(kStageAttention, gq8::launch_mqa(d->qkvRows, d->qkvWidth, keys, values, s.heads, s.kv_heads,
                                   s.head_dim, rows, d->position, 0, s.max_positions,
                                   attentionScale, dbg ? d->debugAttended : nullptr, d->x8,
                                   d->attentionWorkspace, d->attentionWorkspaceBytes, st));
        if (dbg && capture_debug(d, 1, l, d->debugAttended, rows, d->qWidth, d->x8))
            return GQ8_ERR_DEVICE;
        GQ8_STAGE(kStageO, gq8::launch_q8_product(d->x8, rows, 0, rows, d->out[l], d->qWidth, W,
                                          d->hidden, W, 1, st));
        GQ8_STAGE(kStageNorm, gq8::launch_rmsnorm(d->hidden, d->postNorm[l], rows, W, s.rms_epsilon,
                                       nullptr, d->x8, st));
        if (gq8::q8_gemm_geglu_supported(rows, W, F)) {
            // gate|up, GeGLU and its Q8 in one GEMM; the activation rows go
            // to the fused buffer (the GEMM still reads x8)
            uint8_t *act8 = reinterpret_cast<uint8_t *>(d->fused);
            GQ8_STAGE(kStageGateUp, gq8::launch_q8_gemm_geglu(d->x8, (int64_t) rows * W, 0, rows,
                                                              d->gateUp[l], W, F, act8,
                                                              dbg ? d->debugActivated : nullptr, st));
            if (dbg && capture_debug(d, 2, l, d->debugActivated, rows, F, act8))
                return GQ8_ERR_DEVICE;
            GQ8_STAGE(kStageDown, gq8::launch_q8_product(act8, rows, 0, rows, d->down[l], F, W,
                                                         d->hidden, W, 1, st));
        } else {
            GQ8_STAGE(kStageGateUp, gq8::launch_q8_product(d->x8, rows, 0, rows, d->gateUp[l], W,
                                                           2 * F, d->fused, 2 * F, 0, st));
            GQ8_STAGE(kStageGeglu, gq8::launch_geglu(d->fused, rows, F,
                                                     dbg ? d->debugActivated : nullptr, d->x8, st));
            if (dbg && capture_debug(d, 2, l, d->debugActivated, rows, F, d->x8))
                return GQ8_ERR_DEVICE;
            GQ8_STAGE(kStageDown, gq8::launch_q8_product(d->x8, rows, 0, rows, d->down[l], F, W,
                                                         d->hidden, W, 1, st));
        }
        if (dbg && capture_debug(d, 3, l, d->hidden, rows, W, nullptr))
            return GQ8_ERR_DEVICE;
    }

    GQ8_STAGE(kStageNorm, gq8::launch_rmsnorm(d->hidden, d->finalNorm, rows, W, s.rms_epsilon,
                                   d->normalisedRows, d->x8, st));
    if (dbg && capture_debug(d, 0, s.layers, d->normalisedRows, rows, W, d->x8))
        return GQ8_ERR_DEVICE;
    if (logits && logitsRows > 0)
        GQ8_STAGE(kStageLogits, gq8::launch_q8_product(d->x8, rows, rows - logitsRows, logitsRows,
                                          d->embedding, W, s.vocab, logits, s.vocab, 0, st));
    if (sample && sampled(d)) {
        if (int status = encode_sample(d, logits + (int64_t) (logitsRows - 1) * s.vocab, rows))
            return status;
    } else if (sample) {
        GQ8_STAGE(kStageArgmax, gq8::launch_argmax(logits + (int64_t) (logitsRows - 1) * s.vocab, nullptr, 1,
                                      s.vocab, d->sequence, d->position, rows,
                                      d->argmaxWorkspace, d->argmaxWorkspaceBytes, st));
    }
    GQ8_LAUNCH(gq8::launch_advance(d->position, rows, st));
    return GQ8_OK;
}

int check_step(gq8_decoder *d, int rows)
{
    for (size_t i = 0; i < d->present.size(); ++i)
        if (!d->present[i])
            return fail(GQ8_ERR_NOT_PREPARED, "tensor " + std::to_string(i) + " was never loaded");
    if (rows <= 0)
        return fail(GQ8_ERR_EMPTY, "a decoder step needs at least one token");
    if (rows > d->capacity)
        return fail(GQ8_ERR_CAPACITY, "this step carries " + std::to_string(rows)
                                          + " rows and the step capacity is "
                                          + std::to_string(d->capacity));
    if (d->hostPosition + rows > d->shape.max_positions)
        return fail(GQ8_ERR_WINDOW, "this step would carry the sequence to "
                                        + std::to_string(d->hostPosition + rows)
                                        + " tokens, past the window of "
                                        + std::to_string(d->shape.max_positions));
    return GQ8_OK;
}

} // namespace

extern "C" int gq8_decoder_step(gq8_decoder *d, const uint32_t *tokens, int n, float *logits,
                                int logits_rows)
{
    if (!d || !tokens)
        return fail(GQ8_ERR_ARGUMENT, "decoder_step: null argument");
    if (int s = check_step(d, n))
        return s;
    if (logits && logits_rows != 1 && logits_rows != n)
        return fail(GQ8_ERR_ARGUMENT, "decoder_step: logits_rows is 1 or n");
    // token ids are validated here: the reference validates the prompt
    // (Gemma.cpp:418-424); a step's ids are checked the same way.
    std::vector<uint32_t> ids(n);
    GQ8_HIP(hipMemcpy(ids.data(), tokens, n * sizeof(uint32_t), hipMemcpyDeviceToHost));
    for (uint32_t id : ids)
        if (id >= (uint32_t) d->shape.vocab)
            return fail(GQ8_ERR_TOKEN, "token " + std::to_string(id) + " is outside a vocabulary of "
                                           + std::to_string(d->shape.vocab));
    GQ8_HIP(hipMemcpyAsync(d->sequence + d->hostPosition, ids.data(), n * sizeof(uint32_t),
                           hipMemcpyHostToDevice, d->stream));
    if (int s = encode_step(d, n, logits, logits ? logits_rows : 0, false))
        return s;
    GQ8_HIP(hipStreamSynchronize(d->stream));
    if (int s = check_step_error(d, d->hostPosition))
        return s;
    d->hostPosition += n;
    return GQ8_OK;
}

extern "C" int gq8_decoder_hidden(gq8_decoder *d, float *host_out, int rows)
{
    if (!d || !host_out || rows <= 0 || rows > d->capacity)
        return fail(GQ8_ERR_ARGUMENT, "decoder_hidden: bad arguments");
    GQ8_HIP(hipMemcpy(host_out, d->normalisedRows, (size_t) rows * d->shape.width * sizeof(float),
                      hipMemcpyDeviceToHost));
    return GQ8_OK;
}

extern "C" int gq8_decoder_debug(gq8_decoder *d, int which, int layer, float *host_values,
                                 uint8_t *host_q8)
{
    if (!d || which < 0 || which > 3 || layer < 0 || layer > d->shape.layers)
        return fail(GQ8_ERR_ARGUMENT, "decoder_debug: bad arguments");
    const int inner = which == 1 ? d->qWidth : (which == 2 ? d->shape.intermediate : d->shape.width);
    const int64_t slot = (int64_t) layer * 4 + which;
    if (host_values)
        GQ8_HIP(hipMemcpy(host_values, d->debugValues + slot * d->maxInner, inner * sizeof(float),
                          hipMemcpyDeviceToHost));
    if (host_q8)
        GQ8_HIP(hipMemcpy(host_q8, d->debugQ8 + slot * gq8::q8_bytes(1, d->maxInner),
                          gq8::q8_bytes(1, inner), hipMemcpyDeviceToHost));
    return GQ8_OK;
}

// ============================================================================
// Greedy loop (Gemma::generate at temperature 0, Gemma.cpp:395-543)
// ============================================================================
namespace {

// The captured step for steps of `keyCount` keys: one graph a key-count
// range, captured on first use.
int graph_range(const gq8_decoder *d, int keyCount)
{
    (void) d;
    return gq8::attention_graph_range(keyCount);
}

int ensure_graph(gq8_decoder *d, int keyCount)
{
    const int range = graph_range(d, keyCount);
    if (d->graphs[range])
        return GQ8_OK;
    // One decode step reads its token and position from device memory and
    // advances the position itself, so the same graph replays at every step
    // of its key-count range.
    hipGraph_t graph = nullptr;
    GQ8_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
    const bool debug = d->debug;
    d->debug = false;
    d->capturing = true;
    d->captureKeys = gq8::attention_key_range(keyCount, d->shape.max_positions);
    const int status = encode_step(d, 1, d->logits, 1, true);
    d->capturing = false;
    d->debug = debug;
    hipError_t end = hipStreamEndCapture(d->stream, &graph);
    if (status != GQ8_OK) {
        if (graph)
            (void) hipGraphDestroy(graph);
        return status;
    }
    if (end != hipSuccess)
        return fail(GQ8_ERR_DEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(end));
    hipError_t inst = hipGraphInstantiate(&d->graphs[range], graph, nullptr, nullptr, 0);
    (void) hipGraphDestroy(graph);
    if (inst != hipSuccess) {
        d->graphs[range] = nullptr;
        return fail(GQ8_ERR_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(inst));
    }
    return GQ8_OK;
}

// Captures, before a run, the graphs of every key-count range its decode
// steps [firstKeys, lastKeys] touch, so no capture falls inside the run.
int ensure_graphs(gq8_decoder *d, int firstKeys, int lastKeys)
{
    lastKeys = std::min(lastKeys, d->shape.max_positions);
    for (int keys = std::max(firstKeys, 1); keys <= lastKeys;) {
        if (int st = ensure_graph(d, keys))
            return st;
        keys = gq8::attention_key_range(keys, d->shape.max_positions) + 1;
    }
    return GQ8_OK;
}

int decode_one(gq8_decoder *d, bool useGraph)
{
    if (int s = check_step(d, 1))
        return s;
    if (useGraph) {
        if (int s = ensure_graph(d, d->hostPosition + 1))
            return s;
        GQ8_HIP(hipGraphLaunch(d->graphs[graph_range(d, d->hostPosition + 1)], d->stream));
    } else if (int s = encode_step(d, 1, d->logits, 1, true)) {
        return s;
    }
    d->hostPosition += 1;
    return GQ8_OK;
}

int read_slot(gq8_decoder *d, int slot, uint32_t *value)
{
    GQ8_HIP(hipMemcpyAsync(d->pinnedToken, d->sequence + slot, sizeof(uint32_t),
                           hipMemcpyDeviceToHost, d->stream));
    GQ8_HIP(hipStreamSynchronize(d->stream));
    *value = d->pinnedToken[0];
    return GQ8_OK;
}

} // namespace

extern "C" int gq8_generate(gq8_decoder *d, const int32_t *prompt, int prompt_length,
                            int max_tokens, int eos, int use_graph, int32_t *out,
                            gq8_run_stats *stats)
{
    return gq8_generate_streaming(d, prompt, prompt_length, max_tokens, eos, use_graph, out,
                                  stats, nullptr, nullptr);
}

extern "C" int gq8_generate_streaming(gq8_decoder *d, const int32_t *prompt, int prompt_length,
                                      int max_tokens, int eos, int use_graph, int32_t *out,
                                      gq8_run_stats *stats, gq8_token_callback on_token,
                                      void *user)
{
    using Clock = std::chrono::steady_clock;
    if (!d || !prompt || !out)
        return fail(GQ8_ERR_ARGUMENT, "generate: null argument");
    const gq8_shape &s = d->shape;
    if (prompt_length <= 0)
        return fail(GQ8_ERR_EMPTY, "a run needs at least one prompt token");
    if (prompt_length > s.max_positions)
        return fail(GQ8_ERR_WINDOW, "the prompt is longer than the window");
    for (int i = 0; i < prompt_length; ++i)
        if (prompt[i] < 0 || prompt[i] >= s.vocab)
            return fail(GQ8_ERR_TOKEN, "prompt token " + std::to_string(prompt[i])
                                           + " is outside a vocabulary of "
                                           + std::to_string(s.vocab));
    for (size_t i = 0; i < d->present.size(); ++i)
        if (!d->present[i])
            return fail(GQ8_ERR_NOT_PREPARED, "tensor " + std::to_string(i) + " was never loaded");

    if (int st = gq8_decoder_begin_sequence(d))
        return st;
    GQ8_HIP(hipMemcpy(d->sequence, prompt, prompt_length * sizeof(uint32_t), hipMemcpyHostToDevice));
    const int window = s.max_positions - prompt_length;
    const int limit = max_tokens > 0 ? std::min(max_tokens, window) : window;
    if (use_graph) // the decode steps attend prompt_length + 1 .. prompt_length + limit keys
        if (int st = ensure_graphs(d, prompt_length + 1, prompt_length + limit))
            return st;
    gq8_run_stats local{};
    int steps = 0;

    // the prefill, in blocks of the step capacity (Gemma.cpp:350-380)
    const auto prefillStart = Clock::now();
    for (int first = 0; first < prompt_length; first += d->capacity) {
        const int rows = std::min(d->capacity, prompt_length - first);
        const bool last = first + rows >= prompt_length;
        if (int st = check_step(d, rows))
            return st;
        if (int st = encode_step(d, rows, last ? d->logits : nullptr, last ? 1 : 0,
                                 last && limit > 0))
            return st;
        d->hostPosition += rows;
        ++steps;
    }
    GQ8_HIP(hipStreamSynchronize(d->stream));
    local.prefill_seconds = std::chrono::duration<double>(Clock::now() - prefillStart).count();

    int count = 0;
    const auto decodeStart = Clock::now();
    if (limit > 0 && eos < 0) {
        // nothing can stop the run early: every step is enqueued back to back
        for (int step = 1; step < limit; ++step) {
            if (int st = decode_one(d, use_graph != 0))
                return st;
            ++steps;
        }
        GQ8_HIP(hipStreamSynchronize(d->stream));
        if (int st = check_step_error(d, 0)) // the run is void
            return st;
        std::vector<uint32_t> ids(limit);
        GQ8_HIP(hipMemcpy(ids.data(), d->sequence + prompt_length, limit * sizeof(uint32_t),
                          hipMemcpyDeviceToHost));
        for (int i = 0; i < limit; ++i) {
            out[i] = (int32_t) ids[i];
            if (on_token)
                on_token(out[i], user);
        }
        count = limit;
    } else if (limit > 0) {
        // Gemma::generateGreedily (Gemma.cpp:459-543): two steps in flight;
        // step k's token is copied to a pinned slot behind an event of its
        // own, so reading it waits for step k alone while step k + 1 runs.
        hipEvent_t ready[2] = {nullptr, nullptr};
        for (auto &e : ready)
            GQ8_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        auto finish = [&](int status) {
            (void) hipStreamSynchronize(d->stream);
            for (auto &e : ready)
                (void) hipEventDestroy(e);
            return status;
        };
        auto startStep = [&](int step) -> int {
            if (int st = decode_one(d, use_graph != 0))
                return st;
            GQ8_HIP(hipMemcpyAsync(d->pinnedToken + (step & 1), d->sequence + prompt_length + step,
                                   sizeof(uint32_t), hipMemcpyDeviceToHost, d->stream));
            GQ8_HIP(hipEventRecord(ready[step & 1], d->stream));
            ++steps;
            return GQ8_OK;
        };
        int nextStep = 1;
        if (nextStep < limit) {
            if (int st = startStep(nextStep))
                return finish(st);
            ++nextStep;
        }
        for (int step = 0; step < nextStep; ++step) {
            uint32_t token = 0;
            if (step == 0) {
                // the prefill's argmax, already complete
                GQ8_HIP(hipMemcpy(&token, d->sequence + prompt_length, sizeof(uint32_t),
                                  hipMemcpyDeviceToHost));
            } else {
                if (hipEventSynchronize(ready[step & 1]) != hipSuccess)
                    return finish(fail(GQ8_ERR_DEVICE, "generate: event wait failed"));
                token = d->pinnedToken[step & 1];
            }
            if ((int) token == eos)
                break;
            out[count++] = (int32_t) token;
            if (on_token)
                on_token((int32_t) token, user);
            if (nextStep < limit) {
                if (int st = startStep(nextStep))
                    return finish(st);
                ++nextStep;
            }
        }
        finish(GQ8_OK);
        if (int st = check_step_error(d, 0)) // the run is void
            return st;
    }
    local.decode_seconds = std::chrono::duration<double>(Clock::now() - decodeStart).count();
    local.step_count = steps;
    local.generated = count;
    if (stats)
        *stats = local;
    return count;
}

extern "C" int gq8_decoder_decode(gq8_decoder *d, int steps, int use_graph)
{
    if (!d || steps < 0)
        return fail(GQ8_ERR_ARGUMENT, "decoder_decode: bad arguments");
    if (d->hostPosition + steps > d->shape.max_positions)
        return fail(GQ8_ERR_WINDOW, "decoder_decode: the steps would pass the window");
    const int start = d->hostPosition;
    if (use_graph)
        if (int st = ensure_graphs(d, d->hostPosition + 1, d->hostPosition + steps))
            return st;
    for (int i = 0; i < steps; ++i)
        if (int st = decode_one(d, use_graph != 0))
            return st;
    GQ8_HIP(hipStreamSynchronize(d->stream));
    return check_step_error(d, start);
}

extern "C" int gq8_decoder_tokens(gq8_decoder *d, int first, int count, int32_t *host_out)
{
    if (!d || !host_out || first < 0 || count < 0 || first + count > d->shape.max_positions + 1)
        return fail(GQ8_ERR_ARGUMENT, "decoder_tokens: bad range");
    GQ8_HIP(hipStreamSynchronize(d->stream));
    GQ8_HIP(hipMemcpy(host_out, d->sequence + first, count * sizeof(uint32_t),
                      hipMemcpyDeviceToHost));
    return GQ8_OK;
}

extern "C" int gq8_decoder_set_timing(gq8_decoder *d, int stage_mask)
{
    if (!d)
        return fail(GQ8_ERR_ARGUMENT, "null decoder");
    d->timing = (unsigned) stage_mask & ((1u << GQ8_STAGE_COUNT) - 1u);
    return GQ8_OK;
}

// Times one fused one-token kernel alone: `repeats` rounds over every layer's
// weights (gate|up, down) or of the lm_head, back to back on the decoder's
// stream between two HIP events.  The layers' weights rotate as in a step,
// so the kernel streams them from HBM as it does there.  Only scratch is
// written (the Q8 row, a scratch residual row, the logits row); the lm_head
// rounds are followed, outside the events, by a finalize that clears the
// argmax slots without touching the sequence or the position.
extern "C" int gq8_decoder_time_kernel(gq8_decoder *d, int stage, int repeats, double *milliseconds,
                                       int *launches)
{
    if (!d || !milliseconds || !launches || repeats <= 0)
        return fail(GQ8_ERR_ARGUMENT, "decoder_time_kernel: bad arguments");
    if (!d->fusedSupported)
        return fail(GQ8_ERR_SHAPE, "decoder_time_kernel: the shape has no fused kernels");
    if (stage != kStageGateUp && stage != kStageDown && stage != kStageLogits)
        return fail(GQ8_ERR_ARGUMENT, "decoder_time_kernel: stage must be gate|up, down or lm_head");
    const gq8_shape &s = d->shape;
    const int W = s.width, F = s.intermediate;
    hipStream_t st = d->stream;
    hipEvent_t start = take_event(d), stop = take_event(d);
    if (!start || !stop)
        return fail(GQ8_ERR_DEVICE, "decoder_time_kernel: no events");
    gq8::HeadArgs h{};
    h.hidden = d->hidden;
    h.norm_weight = d->finalNorm;
    h.width = W;
    h.epsilon = s.rms_epsilon;
    h.weights = d->embedding;
    h.vocab = s.vocab;
    h.logits = d->logits;
    h.normalised_out = nullptr;
    h.q8 = d->x8;
    h.best = d->headBest;
    h.sequence = nullptr;
    h.position = d->position;
    h.advance = 0;
    int count = 0;
    GQ8_HIP(hipEventRecord(start, st));
    for (int r = 0; r < repeats; ++r) {
        if (stage == kStageLogits) {
            GQ8_LAUNCH(gq8::launch_lmhead_argmax(h, st));
            ++count;
            continue;
        }
        for (int l = 0; l < s.layers; ++l, ++count) {
            if (stage == kStageGateUp) {
                gq8::GateUpArgs g{};
                g.hidden = d->hidden;
                g.norm_weight = d->postNorm[l];
                g.width = W;
                g.epsilon = s.rms_epsilon;
                g.weights = d->gateUp[l];
                g.intermediate = F;
                g.q8 = d->x8;
                GQ8_LAUNCH(gq8::launch_gateup_geglu(g, st));
            } else {
                GQ8_LAUNCH(gq8::launch_q8_product(d->x8, 1, 0, 1, d->down[l], F, W,
                                                  d->normalisedRows, W, 1, st));
            }
        }
    }
    GQ8_HIP(hipEventRecord(stop, st));
    if (stage == kStageLogits)
        GQ8_LAUNCH(gq8::launch_head_finalize(h, st));
    GQ8_HIP(hipStreamSynchronize(st));
    float ms = 0.f;
    GQ8_HIP(hipEventElapsedTime(&ms, start, stop));
    d->spareEvents.push_back(start);
    d->spareEvents.push_back(stop);
    *milliseconds = ms;
    *launches = count;
    return GQ8_OK;
}

extern "C" int gq8_decoder_timing(gq8_decoder *d, double *milliseconds, int *launches)
{
    if (!d || !milliseconds || !launches)
        return fail(GQ8_ERR_ARGUMENT, "decoder_timing: null argument");
    GQ8_HIP(hipStreamSynchronize(d->stream));
    for (int i = 0; i < GQ8_STAGE_COUNT; ++i) {
        milliseconds[i] = 0.0;
        launches[i] = 0;
    }
    for (auto &m : d->marks) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, m.start, m.stop) == hipSuccess && m.stage >= 0
            && m.stage < GQ8_STAGE_COUNT) {
            milliseconds[m.stage] += ms;
            launches[m.stage] += 1;
        }
        d->spareEvents.push_back(m.start);
        d->spareEvents.push_back(m.stop);
    }
    d->marks.clear();
    return GQ8_OK;
}

// ==== lockstep sequences ======================================================
// S sequences (S <= 16) decoded in lockstep over one decoder's weights: the
// reference's S separate greedy loops (Gemma.cpp:459-543), each with its own
// cache and token slots.  A prompt is prefilled through the decoder's own step
// path with the decoder pointed at the sequence's cache, slots and position
// (the prefill arithmetic is the one-sequence path's); a lockstep step then
// carries one row per sequence: the products run all rows against one read of
// the weights (q8_rows_kernel), RoPE, the cache append and attention take
// each row's own position and cache.

struct gq8_batch {
    gq8_decoder *d = nullptr;
    int sequences = 0;
    int64_t cacheStride = 0; // elements between two sequences' caches
    int64_t slotStride = 0;  // slots a sequence (max_positions + 1)
    uint16_t *keyCache = nullptr, *valueCache = nullptr;
    uint32_t *slots = nullptr;
    int *positions = nullptr; // device: the position each sequence's next step takes
    std::vector<int> hostPositions;
    float *hidden = nullptr, *qkvRows = nullptr, *fused = nullptr, *logits = nullptr;
    uint8_t *x8 = nullptr;  // Q8 rows of the norms and of attention
    uint8_t *x8b = nullptr; // Q8 rows of GeGLU (gate | up reads x8 while they are written)
    uint32_t *chosen = nullptr;
    double *attnO = nullptr, *attnMl = nullptr;
    float *rowAngles = nullptr; // each row's RoPE cosines and sines for the step
    unsigned long long *pick = nullptr; // the lm_head's greedy-pick slots, zero between steps
    double *partials = nullptr;
    size_t partialBytes = 0;
    int *tickets = nullptr;
    // the products' weights in fragment order (rows_tiled_bytes), per layer
    // q|k|v, o, gate|up, down and the tied lm_head, made from the decoder's
    // weights of version tiledVersion
    std::vector<uint8_t *> tiledQkv, tiledO, tiledGateUp, tiledDown;
    uint8_t *tiledHead = nullptr;
    uint64_t tiledVersion = 0;
    bool tiled = false;
    void *argmaxWorkspace = nullptr;
    size_t argmaxWorkspaceBytes = 0;
    hipGraphExec_t graph = nullptr;
    std::vector<void *> allocations;
};

namespace {

int batch_alloc(gq8_batch *b, void **out, size_t bytes)
{
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void) hipGetLastError();
        return fail(GQ8_ERR_MEMORY, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    b->allocations.push_back(p);
    *out = p;
    return GQ8_OK;
}

template <typename T>
int batch_alloc_as(gq8_batch *b, T **out, size_t bytes)
{
    void *p = nullptr;
    const int s = batch_alloc(b, &p, bytes);
    *out = reinterpret_cast<T *>(p);
    return s;
}

// The decoder pointed at one sequence of a batch for the length of a prefill.
struct SequenceLoan {
    gq8_decoder *d;
    uint16_t *keyCache, *valueCache;
    uint32_t *sequence;
    int *position;
    int hostPosition;
    SequenceLoan(gq8_decoder *decoder, gq8_batch *b, int s)
        : d(decoder), keyCache(d->keyCache), valueCache(d->valueCache), sequence(d->sequence),
          position(d->position), hostPosition(d->hostPosition)
    {
        d->keyCache = b->keyCache + s * b->cacheStride;
        d->valueCache = b->valueCache + s * b->cacheStride;
        d->sequence = b->slots + s * b->slotStride;
        d->position = b->positions + s;
        d->hostPosition = 0;
    }
    ~SequenceLoan()
    {
        d->keyCache = keyCache;
        d->valueCache = valueCache;
        d->sequence = sequence;
        d->position = position;
        d->hostPosition = hostPosition;
    }
};

int batch_product(gq8_batch *b, int inner, int outputs, const uint8_t *w, const uint8_t *wTiled,
                  float *y, int yStride, int residual, unsigned long long *pick = nullptr)
{
    GQ8_LAUNCH(gq8::launch_q8_rows(b->x8, b->sequences, b->sequences, w, inner, outputs, y, yStride,
                                   residual, b->partials, b->partialBytes, b->tickets, b->d->stream,
                                   wTiled, pick));
    return GQ8_OK;
}

// The fragment-ordered copies, remade when the decoder's weights changed
// since they were made (the copies sit at fixed addresses, so a captured step
// stays valid).
int refresh_tiled(gq8_batch *b)
{
    gq8_decoder *d = b->d;
    if (!b->tiled || b->tiledVersion == d->weightVersion)
        return GQ8_OK;
    const gq8_shape &s = d->shape;
    const int W = s.width, F = s.intermediate;
    hipStream_t st = d->stream;
    for (int l = 0; l < s.layers; ++l) {
        GQ8_LAUNCH(gq8::launch_tile_weights(d->qkv[l], W, d->qkvWidth, b->tiledQkv[l], st));
        GQ8_LAUNCH(gq8::launch_tile_weights(d->out[l], d->qWidth, W, b->tiledO[l], st));
        GQ8_LAUNCH(gq8::launch_tile_weights(d->gateUp[l], W, 2 * F, b->tiledGateUp[l], st));
        GQ8_LAUNCH(gq8::launch_tile_weights(d->down[l], F, W, b->tiledDown[l], st));
    }
    GQ8_LAUNCH(gq8::launch_tile_weights(d->embedding, W, s.vocab, b->tiledHead, st));
    GQ8_HIP(hipStreamSynchronize(st));
    b->tiledVersion = d->weightVersion;
    return GQ8_OK;
}

#define GQ8_BATCH_STAGE(stage, expr)         \
    do {                                     \
        StageTimer timer_(d, stage);         \
        if (int status_ = (expr))            \
            return status_;                  \
    } while (0)

// One lockstep step: every sequence's token at its position, its argmax into
// the next slot, every position advanced by one.
int encode_batch_step(gq8_batch *b)
{
    gq8_decoder *d = b->d;
    const gq8_shape &s = d->shape;
    const int S = b->sequences, W = s.width, F = s.intermediate;
    hipStream_t st = d->stream;

    GQ8_STAGE(kStageEmbed, gq8::launch_embed_slots(b->slots, b->slotStride, b->positions, S,
                                                   d->embedding, s.vocab, W, s.embedding_scale,
                                                   b->hidden, d->cosines, d->sines, s.head_dim / 2,
                                                   b->rowAngles, st));
    for (int l = 0; l < s.layers; ++l) {
        const int64_t layerCache = (int64_t) l * s.max_positions * d->kvWidth;
        GQ8_STAGE(kStageNorm, gq8::launch_rmsnorm(b->hidden, d->inputNorm[l], S, W, s.rms_epsilon,
                                                  nullptr, b->x8, st));
        GQ8_BATCH_STAGE(kStageQkv, batch_product(b, W, d->qkvWidth, d->qkv[l],
                                                 b->tiled ? b->tiledQkv[l] : nullptr, b->qkvRows,
                                                 d->qkvWidth, 0));
        gq8::RowsAttentionArgs at{};
        at.qkv = b->qkvRows;
        at.qkv_stride = d->qkvWidth;
        at.positions = b->positions;
        at.row_angles = b->rowAngles;
        at.key_cache = b->keyCache + layerCache;
        at.value_cache = b->valueCache + layerCache;
        at.cache_stride = b->cacheStride;
        at.max_positions = s.max_positions;
        at.heads = s.heads;
        at.head_dim = s.head_dim;
        at.scale = 1.f / std::sqrt((float) s.head_dim);
        at.per_split = gq8::rows_attention_split_keys(s.max_positions);
        at.ws_o = b->attnO;
        at.ws_ml = b->attnMl;
        at.q8 = b->x8;
        at.q8_rows = S;
        GQ8_STAGE(kStageAttention, gq8::launch_rows_attention(at, S, s.max_positions, st));
        GQ8_BATCH_STAGE(kStageO, batch_product(b, d->qWidth, W, d->out[l],
                                               b->tiled ? b->tiledO[l] : nullptr, b->hidden, W, 1));
        GQ8_STAGE(kStageNorm, gq8::launch_rmsnorm(b->hidden, d->postNorm[l], S, W, s.rms_epsilon,
                                                  nullptr, b->x8, st));
        if (gq8::rows_geglu_supported(W, F)) { // GeGLU in the gate | up product's epilogue
            GQ8_STAGE(kStageGateUp, gq8::launch_q8_rows_geglu(b->x8, S, S, d->gateUp[l], W, F,
                                                               b->x8b, st,
                                                               b->tiled ? b->tiledGateUp[l]
                                                                        : nullptr));
        } else {
            GQ8_BATCH_STAGE(kStageGateUp, batch_product(b, W, 2 * F, d->gateUp[l],
                                                        b->tiled ? b->tiledGateUp[l] : nullptr,
                                                        b->fused, 2 * F, 0));
            GQ8_STAGE(kStageGeglu, gq8::launch_geglu(b->fused, S, F, nullptr, b->x8b, st));
        }
        GQ8_STAGE(kStageDown, gq8::launch_q8_rows(b->x8b, S, S, d->down[l], F, W, b->hidden, W, 1,
                                                  b->partials, b->partialBytes, b->tickets, st,
                                                  b->tiled ? b->tiledDown[l] : nullptr));
    }
    GQ8_STAGE(kStageNorm, gq8::launch_rmsnorm(b->hidden, d->finalNorm, S, W, s.rms_epsilon, nullptr,
                                              b->x8, st));
    // the greedy pick rides on the streamed lm_head where it streams
    const uint8_t *headTiled = b->tiled ? b->tiledHead : nullptr;
    const bool pick = gq8::rows_pick_supported(d->embedding, headTiled, W, s.vocab);
    GQ8_BATCH_STAGE(kStageLogits, batch_product(b, W, s.vocab, d->embedding, headTiled, b->logits,
                                                s.vocab, 0, pick ? b->pick : nullptr));
    if (pick) {
        GQ8_STAGE(kStageArgmax, gq8::launch_batch_pick_advance(b->pick, b->chosen, b->slots,
                                                               b->slotStride, b->positions, S, st));
        return GQ8_OK;
    }
    GQ8_STAGE(kStageArgmax, gq8::launch_argmax(b->logits, nullptr, S, s.vocab, b->chosen, nullptr, 0,
                                               b->argmaxWorkspace, b->argmaxWorkspaceBytes, st));
    GQ8_LAUNCH(gq8::launch_batch_advance(b->chosen, b->slots, b->slotStride, b->positions, S, st));
    return GQ8_OK;
}

int ensure_batch_graph(gq8_batch *b)
{
    if (b->graph)
        return GQ8_OK;
    gq8_decoder *d = b->d;
    hipGraph_t graph = nullptr;
    GQ8_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
    d->capturing = true;
    const int status = encode_batch_step(b);
    d->capturing = false;
    hipError_t end = hipStreamEndCapture(d->stream, &graph);
    if (status != GQ8_OK) {
        if (graph)
            (void) hipGraphDestroy(graph);
        return status;
    }
    if (end != hipSuccess)
        return fail(GQ8_ERR_DEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(end));
    hipError_t inst = hipGraphInstantiate(&b->graph, graph, nullptr, nullptr, 0);
    (void) hipGraphDestroy(graph);
    if (inst != hipSuccess) {
        b->graph = nullptr;
        return fail(GQ8_ERR_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(inst));
    }
    return GQ8_OK;
}

int check_sequence(const gq8_batch *b, int sequence)
{
    if (sequence < 0 || sequence >= b->sequences)
        return fail(GQ8_ERR_ARGUMENT, "sequence " + std::to_string(sequence) + " is outside a batch of "
                                          + std::to_string(b->sequences));
    return GQ8_OK;
}

} // namespace

extern "C" void gq8_batch_destroy(gq8_batch *b)
{
    if (!b)
        return;
    if (b->d && b->d->stream)
        (void) hipStreamSynchronize(b->d->stream);
    if (b->graph)
        (void) hipGraphExecDestroy(b->graph);
    for (void *p : b->allocations)
        (void) hipFree(p);
    delete b;
}

extern "C" int gq8_batch_create(gq8_decoder *d, int sequences, gq8_batch **out)
{
    if (!d || !out)
        return fail(GQ8_ERR_ARGUMENT, "batch_create: null argument");
    *out = nullptr;
    if (sequences <= 0 || sequences > gq8::kBatchRows)
        return fail(GQ8_ERR_ARGUMENT, "a lockstep batch holds 1 to " + std::to_string(gq8::kBatchRows)
                                          + " sequences, not " + std::to_string(sequences));
    const gq8_shape &s = d->shape;
    if (!gq8::rows_attention_supported(s.heads, s.kv_heads, s.head_dim, s.max_positions))
        return fail(GQ8_ERR_SHAPE, "lockstep decode takes multi-query attention (one KV head) "
                                   "with 2, 4 or 8 query heads of width 64, 128 or 256");
    auto *b = new gq8_batch();
    b->d = d;
    b->sequences = sequences;
    b->cacheStride = (int64_t) s.layers * s.max_positions * d->kvWidth;
    b->slotStride = (int64_t) s.max_positions + 1;
    b->hostPositions.assign(sequences, 0);
    auto cleanup = [&](int status) {
        gq8_batch_destroy(b);
        return status;
    };
    const int S = sequences, W = s.width, F = s.intermediate;
    int st = GQ8_OK;
#define GQ8_BATCH_ALLOC(ptr, bytes)                                \
    if ((st = batch_alloc_as(b, &(ptr), (size_t) (bytes))) != 0)   \
        return cleanup(st)
    GQ8_BATCH_ALLOC(b->keyCache, b->cacheStride * S * sizeof(uint16_t));
    GQ8_BATCH_ALLOC(b->valueCache, b->cacheStride * S * sizeof(uint16_t));
    GQ8_BATCH_ALLOC(b->slots, b->slotStride * S * sizeof(uint32_t));
    GQ8_BATCH_ALLOC(b->positions, S * sizeof(int));
    GQ8_BATCH_ALLOC(b->hidden, (size_t) S * W * sizeof(float));
    GQ8_BATCH_ALLOC(b->qkvRows, (size_t) S * d->qkvWidth * sizeof(float));
    GQ8_BATCH_ALLOC(b->fused, (size_t) S * 2 * F * sizeof(float));
    GQ8_BATCH_ALLOC(b->logits, (size_t) S * s.vocab * sizeof(float));
    GQ8_BATCH_ALLOC(b->x8, gq8::q8_bytes(S, d->maxInner));
    GQ8_BATCH_ALLOC(b->x8b, gq8::q8_bytes(S, F));
    GQ8_BATCH_ALLOC(b->chosen, S * sizeof(uint32_t));
    GQ8_BATCH_ALLOC(b->rowAngles, (size_t) S * s.head_dim * sizeof(float));
    GQ8_BATCH_ALLOC(b->pick, gq8::rows_pick_bytes());
    if (hipMemset(b->pick, 0, gq8::rows_pick_bytes()) != hipSuccess)
        return cleanup(fail(GQ8_ERR_DEVICE, "batch pick slots: initialisation failed"));
    GQ8_BATCH_ALLOC(b->attnO, gq8::rows_attention_workspace_doubles(S, s.heads, s.head_dim)
                                  * sizeof(double));
    b->attnMl = b->attnO + (size_t) S * gq8::kRowsMaxSplits * d->qWidth;
    {
        const int products[5][2] = {{W, d->qkvWidth}, {d->qWidth, W}, {W, 2 * F}, {F, W},
                                    {W, s.vocab}};
        size_t bytes = 0;
        int tickets = 0;
        for (auto &p : products) {
            bytes = std::max(bytes, gq8::rows_workspace_bytes(p[0], p[1]));
            tickets = std::max(tickets, gq8::rows_ticket_count(p[1]));
        }
        b->partialBytes = bytes;
        if (bytes)
            GQ8_BATCH_ALLOC(b->partials, bytes);
        GQ8_BATCH_ALLOC(b->tickets, (size_t) tickets * sizeof(int));
        if (hipMemset(b->tickets, 0, (size_t) tickets * sizeof(int)) != hipSuccess)
            return cleanup(fail(GQ8_ERR_DEVICE, "batch tickets: initialisation failed"));
    }
    // the fragment-ordered weight copies, when every product's rows are whole
    // chunks (made at the first decode)
    auto aligned = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    b->tiled = gq8::rows_tiled_supported(W, d->qkvWidth) && gq8::rows_tiled_supported(d->qWidth, W)
               && gq8::rows_tiled_supported(W, 2 * F) && gq8::rows_tiled_supported(F, W)
               && gq8::rows_tiled_supported(W, s.vocab) && aligned(d->embedding);
    for (int l = 0; l < s.layers && b->tiled; ++l)
        b->tiled = aligned(d->qkv[l]) && aligned(d->out[l]) && aligned(d->gateUp[l])
                   && aligned(d->down[l]);
    if (b->tiled) {
        for (int l = 0; l < s.layers; ++l) {
            uint8_t *p = nullptr;
            GQ8_BATCH_ALLOC(p, gq8::rows_tiled_bytes(W, d->qkvWidth));
            b->tiledQkv.push_back(p);
            GQ8_BATCH_ALLOC(p, gq8::rows_tiled_bytes(d->qWidth, W));
            b->tiledO.push_back(p);
            GQ8_BATCH_ALLOC(p, gq8::rows_tiled_bytes(W, 2 * F));
            b->tiledGateUp.push_back(p);
            GQ8_BATCH_ALLOC(p, gq8::rows_tiled_bytes(F, W));
            b->tiledDown.push_back(p);
        }
        GQ8_BATCH_ALLOC(b->tiledHead, gq8::rows_tiled_bytes(W, s.vocab));
        b->tiledVersion = d->weightVersion - 1; // made at the first decode
    }
    b->argmaxWorkspaceBytes = gq8::argmax_workspace_bytes(S, s.vocab);
    if (b->argmaxWorkspaceBytes)
        GQ8_BATCH_ALLOC(b->argmaxWorkspace, b->argmaxWorkspaceBytes);
#undef GQ8_BATCH_ALLOC
    if (hipMemset(b->positions, 0, S * sizeof(int)) != hipSuccess
        || hipMemset(b->slots, 0, b->slotStride * S * sizeof(uint32_t)) != hipSuccess)
        return cleanup(fail(GQ8_ERR_DEVICE, "batch state: initialisation failed"));
    *out = b;
    return GQ8_OK;
}

extern "C" int gq8_batch_prefill(gq8_batch *b, int sequence, const int32_t *prompt,
                                 int prompt_length)
{
    if (!b || !prompt)
        return fail(GQ8_ERR_ARGUMENT, "batch_prefill: null argument");
    if (int st = check_sequence(b, sequence))
        return st;
    gq8_decoder *d = b->d;
    const gq8_shape &s = d->shape;
    if (prompt_length <= 0)
        return fail(GQ8_ERR_EMPTY, "a run needs at least one prompt token");
    if (prompt_length > s.max_positions)
        return fail(GQ8_ERR_WINDOW, "the prompt is longer than the window");
    for (int i = 0; i < prompt_length; ++i)
        if (prompt[i] < 0 || prompt[i] >= s.vocab)
            return fail(GQ8_ERR_TOKEN, "prompt token " + std::to_string(prompt[i])
                                           + " is outside a vocabulary of "
                                           + std::to_string(s.vocab));
    for (size_t i = 0; i < d->present.size(); ++i)
        if (!d->present[i])
            return fail(GQ8_ERR_NOT_PREPARED, "tensor " + std::to_string(i) + " was never loaded");
    GQ8_HIP(hipStreamSynchronize(d->stream));
    uint32_t *slots = b->slots + sequence * b->slotStride;
    GQ8_HIP(hipMemsetAsync(b->positions + sequence, 0, sizeof(int), d->stream));
    GQ8_HIP(hipMemcpyAsync(slots, prompt, prompt_length * sizeof(uint32_t), hipMemcpyHostToDevice,
                           d->stream));
    b->hostPositions[sequence] = 0;
    {
        SequenceLoan loan(d, b, sequence);
        // the prefill in blocks of the step capacity (Gemma.cpp:350-380); the
        // last row's argmax goes to slot prompt_length
        for (int first = 0; first < prompt_length; first += d->capacity) {
            const int rows = std::min(d->capacity, prompt_length - first);
            const bool last = first + rows >= prompt_length;
            if (int st = encode_step(d, rows, last ? d->logits : nullptr, last ? 1 : 0, last))
                return st;
            d->hostPosition += rows;
        }
        GQ8_HIP(hipStreamSynchronize(d->stream));
        if (int st = check_step_error(d, 0)) // the run is void
            return st;
    }
    b->hostPositions[sequence] = prompt_length;
    return GQ8_OK;
}

extern "C" int gq8_batch_decode(gq8_batch *b, int steps, int use_graph)
{
    if (!b || steps < 0)
        return fail(GQ8_ERR_ARGUMENT, "batch_decode: bad arguments");
    const gq8_shape &s = b->d->shape;
    for (int i = 0; i < b->sequences; ++i) {
        if (b->hostPositions[i] == 0)
            return fail(GQ8_ERR_NOT_PREPARED, "sequence " + std::to_string(i) + " has no prompt");
        if (b->hostPositions[i] + steps > s.max_positions)
            return fail(GQ8_ERR_WINDOW, "sequence " + std::to_string(i) + " would pass the window of "
                                            + std::to_string(s.max_positions));
    }
    if (steps == 0)
        return GQ8_OK;
    if (int st = refresh_tiled(b))
        return st;
    if (use_graph)
        if (int st = ensure_batch_graph(b))
            return st;
    for (int i = 0; i < steps; ++i) {
        if (use_graph)
            GQ8_HIP(hipGraphLaunch(b->graph, b->d->stream));
        else if (int st = encode_batch_step(b))
            return st;
    }
    for (int &p : b->hostPositions)
        p += steps;
    GQ8_HIP(hipStreamSynchronize(b->d->stream));
    return GQ8_OK;
}

extern "C" int gq8_batch_sequences(const gq8_batch *b)
{
    return b ? b->sequences : fail(GQ8_ERR_ARGUMENT, "batch_sequences: null batch");
}

extern "C" int gq8_batch_position(const gq8_batch *b, int sequence)
{
    if (!b)
        return fail(GQ8_ERR_ARGUMENT, "batch_position: null batch");
    if (int st = check_sequence(b, sequence))
        return st;
    return b->hostPositions[sequence];
}

extern "C" int gq8_batch_tokens(gq8_batch *b, int sequence, int first, int count,
                                int32_t *host_out)
{
    if (!b || !host_out || first < 0 || count < 0 || first + count > b->slotStride)
        return fail(GQ8_ERR_ARGUMENT, "batch_tokens: bad range");
    if (int st = check_sequence(b, sequence))
        return st;
    GQ8_HIP(hipStreamSynchronize(b->d->stream));
    GQ8_HIP(hipMemcpy(host_out, b->slots + sequence * b->slotStride + first,
                      count * sizeof(uint32_t), hipMemcpyDeviceToHost));
    return GQ8_OK;
}

extern "C" int gq8_batch_logits(gq8_batch *b, float *host_out)
{
    if (!b || !host_out)
        return fail(GQ8_ERR_ARGUMENT, "batch_logits: null argument");
    GQ8_HIP(hipStreamSynchronize(b->d->stream));
    GQ8_HIP(hipMemcpy(host_out, b->logits, (size_t) b->sequences * b->d->shape.vocab * sizeof(float),
                      hipMemcpyDeviceToHost));
    return GQ8_OK;
}
