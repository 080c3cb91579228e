/*
 * gemma_oracle.h -- CPU oracle for the Gemma-2B Int8Blocks ("Q8") token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the GPU path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or the timed CPU
 * baseline: nothing in the shipped product calls it.
 *
 * It restates, as plain C, the arithmetic of eyalamirmusic/HuggingFaceEACP
 * (file:line citations on each function in gemma_oracle.c), plus the two
 * storage rules the MI355X path adds and the reference does not have:
 *
 *   - activation Q8: every product input row is quantized with the
 *     reference's own Int8Blocks rule (Lib/HuggingFaceEACP/Kernels/
 *     Int8Blocks.cpp:25-47) before the product, and the product is the
 *     exact int8 dot per 32-block times (weight scale * activation scale);
 *   - an fp16 key/value cache (IEEE binary16, round to nearest even).
 *
 * Arithmetic rule of the Q8 path ("double compute, fp32 storage"): every
 * operation is evaluated in IEEE double and its result is rounded to fp32 at
 * the points where the reference's GPU decoder stores an fp32 buffer
 * (hidden, normalised, queries, attended, fused, activated, logits;
 * Lib/HuggingFaceEACP/Decoder/Decoder.cpp:172-218).  The reference's own CPU
 * oracle, Tests/Decoder/ReferenceDecoder.h:294-375, is the double-precision
 * form of the same chain with fp32 activations and no fp32 storage points;
 * GOR_MODE_REFERENCE restates that one.
 *
 * Parity pins for each function are listed in the tests (tests/test_oracle_*.py).
 */
#ifndef GEMMA_ORACLE_H
#define GEMMA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE binary16 -------------------------------------------------- */
uint16_t gor_half_from_float(float value);
float gor_half_to_float(uint16_t bits);

/* ---- Int8Blocks format (Int8Blocks.h:56-88, Int8Blocks.cpp:25-124) -- */
enum { GOR_BLOCK = 32 };
int64_t gor_int8_block_count(int64_t element_count);
int64_t gor_int8_blocks_byte_count(int64_t element_count);
int gor_quantizes_as_int8_blocks(int64_t contiguous_extent, int64_t element_count);
uint16_t gor_block_scale_bits(const float *block);
int8_t gor_quantized_byte(float value, float scale);
void gor_quantize_int8_blocks(const float *values, int64_t value_count, int64_t first,
                              int64_t element_count, uint8_t *destination);
void gor_dequantize_int8_blocks(const uint8_t *stored, int64_t element_count,
                                float *values);
/* One activation row under the same rule, stored as the two regions of the
 * format in two arrays: q[n] and scale bits [n / 32]. */
void gor_quantize_row(const float *x, int64_t n, int8_t *q, uint16_t *scale_bits);

/* ---- seeded synthetic inputs ------------------------------------------ */
typedef struct gor_mt64 {
    uint64_t state[312];
    int index;
} gor_mt64;
void gor_mt64_seed(gor_mt64 *engine, uint64_t seed);
uint64_t gor_mt64_next(gor_mt64 *engine);
/* N(0, sigma) fp32 values of one tensor (Box-Muller in double over
 * mt19937_64, one engine per 2^20-element chunk, seeded
 * (tensor_seed << 32) | chunk). */
void gor_normal_fill(uint64_t tensor_seed, double sigma, float *out, int64_t count);
/* Prompt ids: mt19937_64(seed), id = next() % vocab. */
void gor_prompt_ids(uint64_t seed, int vocab, int count, int32_t *out);

/* ---- small kernels' arithmetic ------------------------------------------ */
void gor_rotary_table(int max_positions, int head_dim, double theta, float *cosines,
                      float *sines);
void gor_rmsnorm_row(const float *x, const float *weight, int n, float epsilon,
                     float *out);
double gor_tanh_gelu(double x);
float gor_geglu(float gate, float up);
void gor_rope_row(float *x, int row_stride, int heads, int head_dim, int position,
                  const float *cosines, const float *sines);
/* Q8 x Q8 product of one activation row against rows [0, rows) of an
 * Int8Blocks tensor in the reference's split-region layout. */
void gor_q8_matvec(const int8_t *xq, const uint16_t *xs, const uint8_t *weights,
                   int64_t rows, int64_t inner, float *out);
/* first maximum among unmasked entries, 0 when all are masked
 * (Argmax.h:14-38; Sampler.cpp:60-76). mask may be NULL. */
int gor_argmax(const float *logits, const float *mask, int n);
/* Sampler::uniform (Sampler.cpp:209-212). */
double gor_mt64_uniform(gor_mt64 *engine);
/* Sampler::sample with the draw given (Sampler.cpp:78-213). */
int gor_sample(const float *logits, const float *mask, int n, float temperature, int top_k,
               float top_p, double uniform);
/* One query row (heads x head_dim) over key_count cached fp16 keys/values. */
void gor_mqa_row_f16(const float *query, const uint16_t *keys, const uint16_t *values,
                     int heads, int kv_heads, int head_dim, int key_count, float scale,
                     float *out);

/* ---- the decoder --------------------------------------------------------- */
typedef struct gor_shape {
    int width, heads, kv_heads, head_dim, layers, intermediate, vocab, max_positions;
    float rms_epsilon;
    double rope_theta;
    float embedding_scale;
} gor_shape;

enum {
    GOR_MODE_Q8 = 0,        /* activation Q8 + fp16 KV, double compute, fp32 storage */
    GOR_MODE_REFERENCE = 1, /* ReferenceDecoder.h: double activations, no Q8, double KV */
    GOR_MODE_Q8_PATH_F32 = 2 /* the Q8 path's code with the two new storage rules off:
                                fp32 product inputs and an fp32 KV cache (a check of
                                that code path's composition) */
};

/* Tensor indices in GemmaTensors::all order (GemmaTensors.cpp:30-57):
 * 0 embedding; layer l at 1 + 9l + {q,k,v,o,gate,up,down,input_norm,post_norm};
 * final norm at 1 + 9 * layers. */
enum {
    GOR_T_Q = 0, GOR_T_K, GOR_T_V, GOR_T_O, GOR_T_GATE, GOR_T_UP, GOR_T_DOWN,
    GOR_T_INPUT_NORM, GOR_T_POST_NORM, GOR_T_PER_LAYER
};
int gor_tensor_count(const gor_shape *shape);
int64_t gor_tensor_elements(const gor_shape *shape, int index);
int gor_tensor_is_norm(const gor_shape *shape, int index);
uint64_t gor_tensor_seed(int index);
double gor_tensor_sigma(const gor_shape *shape, int index);

typedef struct gor_model gor_model;
gor_model *gor_model_create(const gor_shape *shape, int mode);
void gor_model_destroy(gor_model *model);
/* values: fp32 tensor; projections and the embedding are Int8Blocks-quantized
 * on the way in (TensorLoader.cpp:120-228), norms are kept as fp32. */
int gor_model_set_tensor(gor_model *model, int index, const float *values);
/* Generate every tensor with gor_normal_fill (sigma 0.02 projections and
 * embedding, 0.1 norms) and set it. */
int gor_model_fill_synthetic(gor_model *model);
/* Quantized bytes of a projection / embedding tensor (NULL for norms). */
const uint8_t *gor_model_tensor_bytes(const gor_model *model, int index);
void gor_model_begin(gor_model *model);
int gor_model_position(const gor_model *model);
/* One decoder step over n tokens at positions position..position+n-1.
 * logits: n x vocab (or NULL); hidden: n x width after the final norm (or
 * NULL); returns 0 or a negative refusal code (see gemma_oracle.c). */
/* The Q8 path's step over a block of n tokens with the products taken over
 * all rows at once (the same arithmetic as n single steps, bit for bit);
 * logits receives the last logits_rows rows (0: none).  -1 outside the Q8
 * mode. */
int gor_model_step_block(gor_model *model, const int32_t *tokens, int n, float *logits,
                         int logits_rows);
int gor_model_step(gor_model *model, const int32_t *tokens, int n, float *logits,
                   float *hidden);
/* Intermediates of the last token of the last step, for bisecting. */
const float *gor_model_debug(const gor_model *model, int which, int layer);
enum { GOR_DBG_NORMALISED = 0, GOR_DBG_ATTENDED, GOR_DBG_ACTIVATED, GOR_DBG_HIDDEN };
/* Q8 bytes of the last product inputs (Q8 mode): which as above. */
const int8_t *gor_model_debug_q(const gor_model *model, int which, int layer);
const uint16_t *gor_model_debug_s(const gor_model *model, int which, int layer);

/* Greedy generation (Gemma.cpp:395-543): prefill, then one token per step,
 * EOS stops and is excluded when eos >= 0, limit = min(max_tokens,
 * max_positions - prompt_length).  Returns count, or a negative refusal. */
int gor_generate(gor_model *model, const int32_t *prompt, int prompt_length,
                 int max_tokens, int eos, int32_t *out, float *out_margins);

/* ---- checks that pin the oracle (test infrastructure) ------------------- */
/* Exhaustive fp32 -> fp16 comparison against the CPU's F16C conversion;
 * returns the number of disagreeing bit patterns (NaNs compare by NaN-ness). */
int64_t gor_check_half_exhaustive(void);
/* All 65536 halves: half -> float -> half is the identity (NaN-ness kept). */
int64_t gor_check_half_roundtrip(void);

#ifdef __cplusplus
}
#endif
#endif
