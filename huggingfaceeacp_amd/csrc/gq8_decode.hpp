// gq8_decode.hpp -- the fused one-token decode step (see gq8_decode.hip).
#pragma once

#include "gq8_kernels.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace gq8 {

constexpr int kFusedMaxWidth = 2048; // a normalised row held in LDS as Q8
constexpr int kDecodeSplits = 64;    // attention workgroups over one row's keys
constexpr int kDecodeCounters = 64; // attention head-group tickets
constexpr int kHeadSlots = 64;       // lm_head argmax words (one wave folds them)
constexpr int kHeadSlotStride = 16;  // 128 bytes between words

struct QkvArgs {
    const float *hidden;      // the residual stream row (unused when embedding)
    const uint32_t *sequence; // with embedding: the id at sequence[*position] is gathered
    const uint8_t *embedding; // non-null on the first layer: gather instead of hidden
    int64_t vocab;
    float embed_scale;
    float *hidden_out;        // the gathered row is stored here (first layer)
    const float *norm_weight;
    int width;
    float epsilon;
    const uint8_t *weights;   // fused q|k|v, Int8Blocks [(H + 2 KV) * D, width]
    int heads, kv_heads, head_dim;
    const int *position;
    const float *cosines, *sines;
    float *query;             // rotated q, fp32 [H * D]
    uint16_t *key_cache, *value_cache; // this layer's [max_positions, KV * D]
    float *debug_normalised;  // optional
    uint8_t *debug_q8;        // optional
};

struct AttentionArgs {
    const float *query;
    const uint16_t *key_cache, *value_cache;
    int heads, kv_heads, head_dim;
    const int *position;      // keys [0, *position] are attended
    float scale;
    double *ws_o, *ws_ml;     // kDecodeSplits partials
    int *counter;             // one a head group (kDecodeCounters), zero between launches
    float *out;               // optional fp32 row
    uint8_t *q8;              // Q8 row for o_proj
};

struct GateUpArgs {
    const float *hidden;
    const float *norm_weight;
    int width;
    float epsilon;
    const uint8_t *weights;   // fused gate|up, Int8Blocks [2 F, width]
    int intermediate;
    uint8_t *q8;              // Q8 row of the GeGLU output for down_proj
    float *debug_activated;   // optional
};

struct HeadArgs {
    const float *hidden;
    const float *norm_weight;
    int width;
    float epsilon;
    const uint8_t *weights;   // the tied embedding, Int8Blocks [vocab, width]
    int vocab;
    uint8_t *q8;              // the final-norm row's Q8 (written, then read by the lm_head)
    float *logits;            // fp32 [vocab]
    float *normalised_out;    // the final-norm row (hiddenStates)
    unsigned long long *best; // kHeadSlots packed (logit key, complemented row) maxima,
                              // kHeadSlotStride apart, zero between launches
    uint32_t *sequence;       // the argmax goes to sequence[*position + 1] (optional)
    int *position;
    int advance;              // nonzero: *position += 1 after the argmax
};

bool fused_decode_supported(int width, int heads, int kv_heads, int head_dim, int intermediate,
                            int max_positions);
size_t decode_workspace_bytes(int heads, int head_dim);

hipError_t launch_qkv_rope(const QkvArgs &a, hipStream_t stream);
hipError_t launch_attention(const AttentionArgs &a, hipStream_t stream);
hipError_t launch_gateup_geglu(const GateUpArgs &a, hipStream_t stream);
hipError_t launch_final_norm(const HeadArgs &a, hipStream_t stream);    // one workgroup
hipError_t launch_lmhead_argmax(const HeadArgs &a, hipStream_t stream); // logits + packed maximum
hipError_t launch_head_finalize(const HeadArgs &a, hipStream_t stream); // id, position, clear

} // namespace gq8
