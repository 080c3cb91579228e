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
    int round_keys;           // keys a round of the launch (attention_round_keys: 32 or 64)
    int spec_keys;            // keys of a split loaded before the position is known
                              // (attention_spec_keys of the same range)
};

// The one-token attention launch for steps of `keyCount` keys, by key-count
// range (attention_graph_range: at most 512, 1024, 2048, 4096 keys, and
// beyond): its key splits (16, 32, 64, 64, 64), the keys of its rounds (32
// while at most 2048 keys, then 64: 4 or 8 keys a wave), and the keys a split
// is expected to cover, whose rows its workgroups load before the position
// arrives (one round; two past 4096 keys).  A split of another size loads its
// rows again once the position is known.  Splits past the step's keys exit
// after their speculative loads, so a launch sized to the range keeps those
// loads few.  A captured step replays within the range it was captured for;
// attention_key_range is the largest key count of that range.
constexpr int kAttentionRanges = 5;
int attention_graph_range(int keyCount);
int attention_grid_splits(int keyCount);
int attention_round_keys(int keyCount);
int attention_spec_keys(int keyCount);
int attention_key_range(int keyCount, int maxPositions);

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

// ---- the dataflow decode step: one launch a token --------------------------------
// Every piece of work of a one-token step (the q|k|v rows, the attention
// splits, the o, gate|up and down rows of every layer, the final norm, the
// lm_head rows and the id) is one workgroup, in dependency order; a workgroup
// issues its weight loads, then waits (a bounded spin) until the phase it
// reads from has finished, computes and publishes its outputs with
// agent-scope (cross-L2 coherent) stores before counting itself done.
constexpr int kFlowThreads = 512;
constexpr int kFlowCounters = 2;       // the lm_head items, the idle attention splits
// A counter is a tree of 128-byte lines: a top line, kFlowFlagLines completion
// flags (waiters spread their polling over them) and kFlowSubLines
// sub-counters of at most kFlowFanIn arrivals each.
constexpr int kFlowLineInts = 32;
constexpr int kFlowFanIn = 16;
constexpr int kFlowFlagLines = 16;
constexpr int kFlowSubLines = 1024;
constexpr int kFlowCounterLines = 1 + kFlowFlagLines + kFlowSubLines;
constexpr int64_t kFlowCounterInts = (int64_t) kFlowCounters * kFlowCounterLines * kFlowLineInts;
constexpr int kFlowMaxLayers = 127;    // residual-row versions 0 .. 2 layers fit a tag's 8 bits

struct FlowArgs {
    int layers, width, heads, kv_heads, head_dim, intermediate, vocab, max_positions;
    float epsilon, embed_scale, attn_scale;
    const uint8_t *embedding;                 // Int8Blocks [vocab, width], also the lm_head
    // layer l of a kind at base + l * stride (bytes for the Int8Blocks
    // tensors, floats for the norms): addresses the compiler knows are global
    const uint8_t *qkv, *out, *gate_up, *down; // fused q|k|v, o, fused gate|up, down
    int64_t qkv_stride, out_stride, gate_up_stride, down_stride;
    const float *input_norm, *post_norm;
    int64_t norm_stride;
    const float *final_norm;
    uint16_t *key_cache, *value_cache;        // [layers][max_positions][kv_heads * head_dim]
    const float *cosines, *sines;
    uint32_t *sequence;
    int *position;
    uint32_t *epoch;                          // the launch's tag epoch (never 0)
    // rows handed between items, one tagged word (value | tag << 32) an element
    uint64_t *hidden_ll;                      // the residual row [width]
    uint64_t *q_ll;                           // the rotated q row [heads * head_dim]
    uint64_t *k_ll, *v_ll;                    // this step's fp16 K and V rows, two halves a word
    uint64_t *part_ll;                        // attention partial outputs [kDecodeSplits][q width] doubles
    uint64_t *part_ml_ll;                     // their max and sum [kDecodeSplits][heads] double pairs
    uint64_t *attn_ll, *act_ll, *head_ll;     // Q8 rows: bytes (four a word), then one scale word a block
    float *logits;
    unsigned long long *best;                 // argmax slots
    int *counters;                            // kFlowCounters counter trees
    int *error;                               // nonzero after a wait gave up
    int attn_splits;                          // attention split items a head group
    int sample;                               // nonzero: the id goes to sequence[position + 1]
    int qkv_items, attn_items, o_items, gate_up_items, down_items, head_items;
};

// ---- the persistent decode step: one launch a token, one workgroup a CU -------
// Every workgroup runs the whole step's program on its share of every phase
// (gq8_persist.hip).  Four prefetch waves stream its share of the gate|up,
// down and lm_head weights into an LDS ring; four compute waves run the
// dependent chain and hand rows on in tagged words.
constexpr int kPersistThreads = 512;
constexpr int kPersistMaxSplits = 64;   // attention key splits of a row
constexpr int kPersistMaxLayers = 127;  // residual-row versions 0 .. 2 layers fit a tag's 8 bits

struct PersistArgs {
    int layers, width, heads, kv_heads, head_dim, intermediate, vocab, max_positions;
    float epsilon, embed_scale, attn_scale;
    const uint8_t *embedding;                 // Int8Blocks [vocab, width], also the lm_head
    // layer l of a kind at base + l * stride (bytes for the Int8Blocks
    // tensors, floats for the norms)
    const uint8_t *qkv, *out, *gate_up, *down;
    int64_t qkv_stride, out_stride, gate_up_stride, down_stride;
    const float *input_norm, *post_norm;
    int64_t norm_stride;
    const float *final_norm;
    uint16_t *key_cache, *value_cache;        // [layers][max_positions][kv_heads * head_dim]
    const float *cosines, *sines;
    uint32_t *sequence;
    int *position;
    uint32_t *epoch;                          // the launch's tag epoch (never 0)
    // tagged rows (value | tag << 32, one element a word)
    uint64_t *hid_ll;                         // the residual row [width]
    uint64_t *q_ll;                           // the rotated q row [heads * head_dim]
    uint64_t *kv_ll;                          // this step's k then v row, fp16 bits [2 kv width]
    uint64_t *part_ll;                        // attention partials [split][head][head_dim], doubles as
                                              // (low, high) word pairs
    uint64_t *ml_ll;                          // their (max, sum) [split][head], four words
    uint64_t *attn_ll, *act_ll;               // Q8 rows: bytes four a word, then a scale word a block
    uint64_t *cand_ll;                        // a workgroup's argmax candidate, two words
    float *logits;                            // fp32 [vocab]
    int *error;                               // nonzero after a wait gave up
    int sample;                               // nonzero: the id goes to sequence[position + 1]
    int grid;                                 // workgroups: one a compute unit, all resident
};

// Tagged words the persistent step needs, by row (the runtime carves them
// from one allocation).
struct PersistWords {
    int64_t hid, q, kv, part, ml, attn, act, cand;
};
PersistWords persist_words(int width, int heads, int kv_heads, int head_dim, int intermediate, int grid);
// Whether the shape fits the persistent step's partition on `grid` workgroups.
bool persist_decode_supported(int layers, int width, int heads, int kv_heads, int head_dim,
                              int intermediate, int vocab, int max_positions, int grid);
// The workgroups of the persistent step on `device` (its compute units, when
// one workgroup fits a unit), or 0.
int persist_grid(int device);
hipError_t launch_persist_step(const PersistArgs &a, hipStream_t stream);

bool flow_decode_supported(int layers, int width, int heads, int kv_heads, int head_dim, int intermediate,
                           int vocab, int max_positions);
int flow_attention_splits(int max_positions);
// Fills the item counts of a; returns the grid size.
int flow_items(FlowArgs &a);
hipError_t launch_flow_step(const FlowArgs &a, hipStream_t stream);

bool fused_decode_supported(int width, int heads, int kv_heads, int head_dim, int intermediate,
                            int max_positions);

hipError_t launch_qkv_rope(const QkvArgs &a, hipStream_t stream);
hipError_t launch_attention(const AttentionArgs &a, hipStream_t stream);
hipError_t launch_gateup_geglu(const GateUpArgs &a, hipStream_t stream);
hipError_t launch_final_norm(const HeadArgs &a, hipStream_t stream);    // one workgroup
hipError_t launch_lmhead_argmax(const HeadArgs &a, hipStream_t stream); // logits + packed maximum
hipError_t launch_head_finalize(const HeadArgs &a, hipStream_t stream); // id, position, clear

} // namespace gq8
