// gq8_decode.hpp -- the fused one-token decode step (see gq8_decode.hip).
#pragma once

#include "gq8_kernels.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace gq8 {

constexpr int kFusedMaxWidth = 2048; // a normalised row held in LDS as Q8
constexpr int kDecodeSplits = 64;    // attention workgroups over one row's keys
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
    uint32_t *tag_epoch;      // advanced by one each launch (the attention launch's tag)
};

struct AttentionArgs {
    const float *query;
    const uint16_t *key_cache, *value_cache;
    int heads, kv_heads, head_dim;
    int max_positions;        // rows of the cache (the bound of speculative reads)
    const int *position;      // keys [0, *position] are attended
    float scale;
    uint64_t *part_ll;        // split partials as tagged words: [kDecodeSplits][H D][2]
    uint64_t *ml_ll;          // their (max, sum): [kDecodeSplits][H][4] tagged words
    const uint32_t *tag_epoch; // the launch's tag (advanced by the q|k|v launch before it)
    int *error;               // set when a merge's wait gives up
    float *out;               // optional fp32 row
    uint8_t *q8;              // Q8 row for o_proj
    int grid_splits;          // the launch's key splits (attention_grid_splits of the step's
                              // key-count range)
    int rounds;               // 32-key rounds a split takes at most (attention_rounds)
    int spec_keys;            // rounds * 32: the keys of a split loaded before the position
                              // is known
};

// The one-token attention launch for steps of `keyCount` keys, by key-count
// range (attention_graph_range: at most 512, 1024, 2048, 4096 keys, and
// beyond): its key splits (16, 32, 64, 64, 64) and the 32-key rounds a split
// takes at most (1, 1, 1, 2, 4), whose rows its workgroups load before the
// position arrives.  A captured step replays within the range it was
// captured for; attention_key_range is the largest key count of that range.
constexpr int kAttentionRanges = 5;
int attention_graph_range(int keyCount);
int attention_grid_splits(int keyCount);
int attention_rounds(int keyCount);
int attention_key_range(int keyCount, int maxPositions);
// Query heads a workgroup of the split attention (2 of a KV head's, or 1).
int attention_group_heads(int heads, int kv_heads);
// Workgroups of the split attention's launch for steps of keyCount keys.
int attention_grid(int heads, int kv_heads, int keyCount);
// Whether the split attention takes the shape (head width 64, 128 or 256, a
// window of at most 64 splits of 128 keys).
bool split_attention_supported(int heads, int kv_heads, int head_dim, int max_positions);
// Whether every launch the window reaches fits the workgroups that can be
// resident at once, by range: the launch's workgroups wait on each other.
bool split_attention_fits(int heads, int kv_heads, int head_dim, int max_positions,
                          const int (&resident)[kAttentionRanges]);
// The resident workgroups of each range's kernel on `device` (occupancy of
// the instance times the compute units); false if unknown.
bool split_attention_resident(int device, int heads, int kv_heads, int head_dim, int max_positions,
                              int (&resident)[kAttentionRanges]);

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
    uint8_t *q8;              // the final-norm row's Q8 (written by workgroup 0: the debug view)
    float *logits;            // fp32 [vocab]
    float *normalised_out;    // the final-norm row (hiddenStates)
    unsigned long long *best; // kHeadSlots packed (logit key, complemented row) maxima,
                              // kHeadSlotStride apart, zero between launches
    uint32_t *sequence;       // the argmax goes to sequence[*position + 1] (optional)
    int *position;
    int advance;              // nonzero: *position += 1 after the argmax
};

// Whether the fused one-token kernels (q|k|v + RoPE, gate|up + GeGLU, the
// head) take the shape; the attention between them is the split attention
// where it fits, else the partial/merge pair of gq8_kernels.hip.
bool fused_decode_supported(int width, int heads, int kv_heads, int head_dim, int intermediate);

hipError_t launch_qkv_rope(const QkvArgs &a, hipStream_t stream);
hipError_t launch_attention(const AttentionArgs &a, hipStream_t stream);
hipError_t launch_gateup_geglu(const GateUpArgs &a, hipStream_t stream);
hipError_t launch_lmhead_argmax(const HeadArgs &a, hipStream_t stream); // final norm, logits, maximum
hipError_t launch_head_finalize(const HeadArgs &a, hipStream_t stream); // id, position, clear

} // namespace gq8
