// gq8_kernels.hpp -- launch functions for the gfx950 kernels of the Gemma
// Int8Blocks token loop.  Every launcher checks its grid against its buffers
// on the host; positions can come from a device int (pos_ptr, so a captured
// decode step replays at every position) plus a host offset.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace gq8 {

// Q8 row buffer helpers: rows x inner elements in the Int8Blocks layout.
inline int64_t q8_bytes(int64_t rows, int64_t inner)
{
    return rows * inner + rows * inner / 16;
}

// elements fp32 values -> q[elements] bytes and scales[elements / 32] fp16
// bits (the two regions of an Int8Blocks buffer, given separately so a piece
// of a larger tensor can be quantized in place).
hipError_t launch_quantize(const float *x, int64_t elements, uint8_t *q, uint16_t *scales,
                           hipStream_t stream);

hipError_t launch_embed(const uint32_t *tokens, const int *pos_ptr, int rows,
                        const uint8_t *table, int vocab, int width, float scale, float *out,
                        hipStream_t stream);

// y (optional) fp32 and q8 (optional) Q8 row buffer of rows x width.
hipError_t launch_rmsnorm(const float *x, const float *weight, int rows, int width,
                          float epsilon, float *y, uint8_t *q8, hipStream_t stream);

hipError_t launch_rope(float *x, int row_stride, int heads, int head_dim, const int *pos_ptr,
                       int pos_value, int rows, const float *cosines, const float *sines,
                       hipStream_t stream);

// The fused-qkv epilogue of a step: rotate q (in place, heads) and k (kv
// heads), store k and v as fp16 into the caches at the step's positions.
hipError_t launch_rope_kv(float *qkv, int qkv_stride, int heads, int kv_heads, int head_dim,
                          const int *pos_ptr, int pos_value, int rows, const float *cosines,
                          const float *sines, uint16_t *key_cache, uint16_t *value_cache,
                          hipStream_t stream);

hipError_t launch_kv_store(const float *k, const float *v, int src_stride, int rows,
                           int kv_width, uint16_t *key_cache, uint16_t *value_cache,
                           const int *pos_ptr, int pos_value, hipStream_t stream);

// x8: Q8 row buffer of x_rows_total rows; rows [x_row0, x_row0 + rows) are used.
// Steps of kGemmMinRows rows or more whose inner size is a whole number of
// 256-byte chunks run on the int8 MFMA GEMM (gq8_gemm.hip).
constexpr int kGemmMinRows = 32;
bool q8_gemm_supported(int rows, int inner, int outputs);
// The gate|up product of a fused [2 F, inner] weight with GeGLU and its Q8
// folded into the GEMM's epilogue: q8_out receives the [rows, F] Q8 row
// buffer of the activations, debug_out (optional) their fp32 values.
bool q8_gemm_geglu_supported(int rows, int inner, int intermediate);
hipError_t launch_q8_gemm_geglu(const uint8_t *x8, int64_t x_elements, int x_row0, int rows,
                                const uint8_t *w8, int inner, int intermediate, uint8_t *q8_out,
                                float *debug_out, hipStream_t stream);
hipError_t launch_q8_gemm(const uint8_t *x8, int64_t x_elements, int x_row0, int rows,
                          const uint8_t *w8, int inner, int outputs, float *y, int y_stride,
                          int residual, hipStream_t stream);
hipError_t launch_q8_product(const uint8_t *x8, int x_rows_total, int x_row0, int rows,
                             const uint8_t *w8, int inner, int outputs, float *y, int y_stride,
                             int residual, hipStream_t stream);

constexpr int kAttentionSplits = 64; // workgroups over one query row's keys
constexpr int kMaxHeads = 16;
constexpr int kMaxHeadDim = 256;

size_t mqa_workspace_bytes(int rows, int heads, int head_dim, int max_keys);

// Blocks of kPrefillAttentionMinRows rows or more with a head width of 64, 128
// or 256 take the fp64-MFMA prefill kernel (gq8_prefill_attention.hip; no
// workspace) when its 16-byte loads and stores fit the buffers: queries, caches,
// out and q8 16-byte aligned, q_stride a multiple of 4.
constexpr int kPrefillAttentionMinRows = 16;
bool prefill_attention_supported(int head_dim, const float *queries, int q_stride,
                                 const uint16_t *key_cache, const uint16_t *value_cache,
                                 const float *out, const uint8_t *q8);
hipError_t launch_prefill_attention(const float *queries, int q_stride, const uint16_t *key_cache,
                                    const uint16_t *value_cache, int heads, int kv_heads,
                                    int head_dim, int rows, const int *pos_ptr, int pos_value,
                                    float scale, float *out, uint8_t *q8, hipStream_t stream);

// Rows of queries (row stride q_stride) at positions base + r where
// base = (*pos_ptr if pos_ptr) + pos_value; row r attends keys [0, base + r].
// max_keys bounds base + rows (sizes the grid so a captured step fits every
// position).  out: fp32 [rows, heads * head_dim] (optional), q8: Q8 row buffer
// of the same (optional).
hipError_t launch_mqa(const float *queries, int q_stride, const uint16_t *key_cache,
                      const uint16_t *value_cache, int heads, int kv_heads, int head_dim,
                      int rows, const int *pos_ptr, int pos_value, int max_keys, float scale,
                      float *out, uint8_t *q8, void *workspace, size_t workspace_bytes,
                      hipStream_t stream);

hipError_t launch_geglu(const float *fused, int rows, int intermediate, float *out,
                        uint8_t *q8, hipStream_t stream);

size_t argmax_workspace_bytes(int rows, int length);
// indices[(pos_ptr ? *pos_ptr : 0) + index_offset + row] for each row.
hipError_t launch_argmax(const float *logits, const float *mask, int rows, int length,
                         uint32_t *indices, const int *pos_ptr, int index_offset,
                         void *workspace, size_t workspace_bytes, hipStream_t stream);

hipError_t launch_advance(int *pos_ptr, int amount, hipStream_t stream);

// ---- lockstep sequences (one step of up to kBatchRows independent sequences
// over one weight set) ----------------------------------------------------------
// Row r: sequence r, at position positions[r]; its token slots start at
// slots + r * slot_stride.
constexpr int kBatchRows = 16;

// With row_angles, also the RoPE table rows (half pairs, cosines then sines)
// of each row's position, for the step's attention (RowsAttentionArgs).
hipError_t launch_embed_slots(const uint32_t *slots, int64_t slot_stride, const int *positions,
                              int rows, const uint8_t *table, int vocab, int width, float scale,
                              float *out, const float *cosines, const float *sines, int half,
                              float *row_angles, hipStream_t stream);

// y[m, n] (+)= the Int8Blocks product of up to kBatchRows activation rows (a
// Q8 row buffer of x_rows rows, rows [0, rows) used) on int8 MFMA.  Products
// too small to fill the chip split their blocks over several workgroups:
// partials (rows_workspace_bytes) and tickets (rows_ticket_count ints, zero
// between launches) carry the split.
size_t rows_workspace_bytes(int inner, int outputs);
int rows_ticket_count(int outputs);
hipError_t launch_q8_rows(const uint8_t *x8, int x_rows, int rows, const uint8_t *w8, int inner,
                          int outputs, float *y, int y_stride, int residual, double *partials,
                          size_t partial_bytes, int *tickets, hipStream_t stream,
                          const uint8_t *w8_tiled = nullptr, unsigned long long *best = nullptr);
// The greedy pick fused into a streamed product (rows_pick_supported: the
// lm_head's shape): with best (rows_pick_bytes, zero between steps), every
// workgroup folds its tiles' (logit key, complemented column) maxima of each
// row into one of the row's slots; launch_batch_pick_advance then takes each
// row's largest (the lowest column among equal logits), stores it in chosen
// and in the row's next slot, advances the position and clears the slots.
bool rows_pick_supported(const uint8_t *w8, const uint8_t *w8_tiled, int inner, int outputs);
size_t rows_pick_bytes();
hipError_t launch_batch_pick_advance(unsigned long long *best, uint32_t *chosen, uint32_t *slots,
                                     int64_t slot_stride, int *positions, int rows,
                                     hipStream_t stream);

// The fragment-ordered copy of an [outputs, inner] Int8Blocks weight that
// the lockstep products stream about a third faster than the row-major
// layout (w8_tiled above; rows_tiled_bytes bytes, 16-byte aligned, inner a
// multiple of 256).  A copy, so it holds the weight as it was when made.
bool rows_tiled_supported(int inner, int outputs);
size_t rows_tiled_bytes(int inner, int outputs);
hipError_t launch_tile_weights(const uint8_t *w8, int inner, int outputs, uint8_t *out,
                               hipStream_t stream);

// Attention of the lockstep rows with the step's RoPE and cache append
// (multi-query: one KV head).  qkv row r holds sequence r's unrotated
// q | k | v; the keys [0, positions[r]] of sequence r's caches (the layer's
// base for sequence 0, cache_stride elements a sequence) are attended after
// the new key and value are appended at positions[r].  The merged row goes to
// row r of a Q8 row buffer of q8_rows rows.  per_split is
// rows_attention_split_keys(max_positions); ws_o / ws_ml hold
// rows_attention_workspace_doubles.
constexpr int kRowsMaxSplits = 32;
struct RowsAttentionArgs {
    const float *qkv;
    int qkv_stride;
    const int *positions;
    const float *row_angles;  // row r's RoPE cosines [2 r half ..] and sines [(2 r + 1) half ..]
    uint16_t *key_cache, *value_cache;
    int64_t cache_stride;
    int max_positions;        // rows of each cache (the bound of speculative reads)
    int heads, head_dim;
    float scale;
    int per_split;
    double *ws_o, *ws_ml;
    uint8_t *q8;
    int q8_rows;
};
bool rows_attention_supported(int heads, int kv_heads, int head_dim, int max_positions);
int rows_attention_split_keys(int max_positions);
size_t rows_attention_workspace_doubles(int rows, int heads, int head_dim);
hipError_t launch_rows_attention(const RowsAttentionArgs &a, int rows, int max_positions,
                                 hipStream_t stream);

// The gate | up product with GeGLU fused: w8 is the stacked [gate; up]
// tensor (2 intermediate rows), and GeGLU of row m's products goes, as Q8, to
// row m of geglu8 (a Q8 row buffer of x_rows rows of intermediate).
bool rows_geglu_supported(int inner, int intermediate);
hipError_t launch_q8_rows_geglu(const uint8_t *x8, int x_rows, int rows, const uint8_t *w8,
                                int inner, int intermediate, uint8_t *geglu8, hipStream_t stream,
                                const uint8_t *w8_tiled = nullptr);

// After the argmax of a step: slot positions[r] + 1 of sequence r takes
// chosen[r], and positions[r] advances by one.
hipError_t launch_batch_advance(const uint32_t *chosen, uint32_t *slots, int64_t slot_stride,
                                int *positions, int rows, hipStream_t stream);

// ---- sampling (Sampler::sample, Sampler.cpp:78-213) ----------------------------
struct SampleArgs {
    const float *logits;   // one row of fp32 [vocab]
    const float *mask;     // nonzero: the token is never chosen (optional)
    int vocab;
    float temperature;     // > 0 (zero is the argmax)
    int top_k;             // 0: no cut
    float top_p;           // 1: no cut
    const double *draws;   // uniform draws in [0, 1), one a sample
    int draw_count;        // the index is clamped to the last draw
    int *draw_index;       // the draw this sample takes; advanced by one
    uint32_t *sequence;    // the chosen id goes to sequence[*position + offset] (optional)
    const int *position;
    int offset;
    uint32_t *token_out;   // and to *token_out (optional)
};

size_t sample_workspace_bytes(int vocab);
bool sampling_options_valid(float temperature, int top_k, float top_p);
hipError_t launch_sample(const SampleArgs &a, void *workspace, size_t workspace_bytes,
                         hipStream_t stream);

} // namespace gq8
