/*
 * gemma_q8.h -- C ABI of the MI355X (gfx950) Gemma-2B Int8Blocks token loop.
 *
 * One shared library, huggingfaceeacp_amd/libgemma_q8.so, with two layers:
 *
 *   1. op-level entry points, one per kernel of the reference's decoder
 *      (the headers under Lib/HuggingFaceEACP/Kernels), taking device pointers, sizes and a
 *      HIP stream (passed as void *);
 *   2. the decoder runtime: the counterparts of HF::Decoder
 *      (Lib/HuggingFaceEACP/Decoder/Decoder.h:69-319) and of the greedy loop
 *      of HF::Gemma (Lib/HuggingFaceEACP/Generation/Gemma.h:65-342).
 *
 * Conventions.  Every function returns an int status (GQ8_OK = 0, a negative
 * gq8_status otherwise) and never throws; gq8_last_error() names the last
 * failure.  Refusals are checked on the host before anything is launched, so a
 * refused call leaves every output untouched (the reference throws before it
 * records: Decoder.cpp:644-675).  Device pointers belong to the caller unless
 * a function says otherwise.
 *
 * Int8Blocks layout (Lib/HuggingFaceEACP/Kernels/Int8Blocks.h:19-31): a tensor
 * of E elements is one buffer of E + E / 16 bytes: E signed bytes, then E / 32
 * little-endian fp16 scales, the scale of block b at half index E / 2 + b.  An
 * activation "Q8 row buffer" of R rows of K is the same layout over R * K
 * elements.
 */
#ifndef GEMMA_Q8_H
#define GEMMA_Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum gq8_status {
    GQ8_OK = 0,
    GQ8_ERR_ARGUMENT = -1,      /* null pointer, negative or inconsistent size */
    GQ8_ERR_SHAPE = -2,         /* DecoderShape::validate refusals (DecoderShape.cpp:41-92) */
    GQ8_ERR_CAPACITY = -3,      /* rows past the step capacity (Decoder.cpp:655-664) */
    GQ8_ERR_WINDOW = -4,        /* position + rows past maxPositions (Decoder.cpp:666-675) */
    GQ8_ERR_TOKEN = -5,         /* token id outside the vocabulary (Gemma.cpp:418-424) */
    GQ8_ERR_UNQUANTIZABLE = -6, /* quantizesAsInt8Blocks refusal (Int8Blocks.cpp:80-85) */
    GQ8_ERR_NOT_PREPARED = -7,  /* weights missing (Decoder.cpp:286-300) */
    GQ8_ERR_EMPTY = -8,         /* a step or prompt of zero tokens (Decoder.cpp:650-651) */
    GQ8_ERR_DEVICE = -9,        /* a HIP call failed */
    GQ8_ERR_MEMORY = -10,       /* device allocation failed */
    GQ8_ERR_FORMAT = -11        /* a malformed or mismatched checkpoint file (SafeTensors.h:85-101) */
} gq8_status;

const char *gq8_status_string(int status);
/* The message of the last failure on this thread ("" if none). */
const char *gq8_last_error(void);
/* Library identity: "gemma_q8 <version> gfx950". */
const char *gq8_version(void);

/* ======================================================================= */
/* Int8Blocks format on the host (Int8Blocks.h:58-88).                     */
/* ======================================================================= */
int64_t gq8_int8_block_count(int64_t element_count);       /* Int8Blocks.h:60 */
int64_t gq8_int8_blocks_byte_count(int64_t element_count); /* Int8Blocks.h:61 */
/* 1 if a tensor of this shape is storable (Int8Blocks.h:69), else 0. */
int gq8_quantizes_as_int8_blocks(int64_t contiguous_extent, int64_t element_count);
/* quantizeInt8Blocks, both overloads (Int8Blocks.h:72-82): values holds
 * value_count elements starting at element `first` of a tensor of
 * element_count, destination is that whole tensor's bytes.  Runs on all host
 * cores (TensorLoader.cpp:190-228). */
int gq8_quantize_int8_blocks_host(const float *values, int64_t value_count, int64_t first,
                                  int64_t element_count, uint8_t *destination);
/* dequantizeInt8Blocks (Int8Blocks.h:88). */
int gq8_dequantize_int8_blocks_host(const uint8_t *stored, int64_t element_count,
                                    float *values);
/* makeRotaryTable (RoPE.h:116-117): cos/sin [max_positions, head_dim / 2]. */
int gq8_rotary_table_host(int max_positions, int head_dim, double theta, float *cosines,
                          float *sines);

/* ======================================================================= */
/* Op-level entry points (device pointers, stream = hipStream_t or NULL).  */
/* ======================================================================= */

/* Int8Blocks quantization of rows x inner fp32 values into one Q8 row
 * buffer; bit-exact with quantizeInt8Blocks (Int8Blocks.cpp:87-110).  Used
 * for activations and for quantize-on-upload of weights. */
int gq8_quantize_rows(const float *x, int64_t rows, int64_t inner, uint8_t *q8, void *stream);

/* EmbedProgram<Int8Blocks> (Embed.h:45-82): out[t, c] = scale * W[token[t], c]
 * for a [vocab, width] Int8Blocks table. */
int gq8_embed(const uint32_t *tokens, int rows, const uint8_t *table, int vocab, int width,
              float scale, float *out, void *stream);

/* RMSNorm (RMSNorm.h:37-90): y = x / sqrt(mean(x^2) + eps) * (1 + w), per row.
 * y may be NULL when q8 is given; q8 (optional) receives the Q8 row buffer of
 * y (the fused norm + activation quantization of the Q8 path). */
int gq8_rmsnorm(const float *x, const float *weight, int rows, int width, float epsilon,
                float *y, uint8_t *q8, void *stream);

/* RoPE (RoPE.h:50-94): rotate-half in place over rows x heads heads of
 * head_dim at row_stride, row r at position first_position + r, from the
 * [max_positions, head_dim / 2] tables. */
int gq8_rope(float *x, int row_stride, int heads, int head_dim, int first_position, int rows,
             const float *cosines, const float *sines, void *stream);

/* The Int8Blocks product of SplitLinearProgram / TiledMatMulProgram
 * (Linear.h:128-357, TiledMatMul.h:167-650) with Q8 activations:
 *   y[r, o] = sum_b scale_w[o, b] * scale_x[r, b] * dot8(w[o, b], x[r, b])  (+ y[r, o])
 * x8: Q8 row buffer [rows, inner]; w8: Int8Blocks [outputs, inner];
 * y: fp32 [rows, y_stride] (y_stride >= outputs); residual != 0 adds the
 * existing y (Linear.h:284-298).  Exact int8 dots, double accumulation. */
int gq8_q8_product(const uint8_t *x8, const uint8_t *w8, int rows, int inner, int outputs,
                   float *y, int y_stride, int residual, void *stream);

/* fp16 KV-cache append (the ranged bind of Decoder.cpp:450-466, with fp16
 * storage): rows of k and v (fp32, row stride src_stride) written at cache
 * rows position .. position + rows - 1 of [max_positions, kv_width] caches. */
int gq8_kv_store_f16(const float *k, const float *v, int src_stride, int rows, int kv_width,
                     uint16_t *key_cache, uint16_t *value_cache, int position, void *stream);

/* MultiQueryDecodeAttention (MultiQueryAttention.h:317-341): one query row of
 * heads x head_dim over key_count fp16 cached rows, split over key chunks with
 * an exact online-softmax merge.  workspace >= gq8_mqa_workspace_bytes(). */
size_t gq8_mqa_workspace_bytes(int rows, int heads, int head_dim, int max_keys);
int gq8_mqa_decode(const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
                   int heads, int kv_heads, int head_dim, int key_count, float scale, float *out,
                   void *workspace, size_t workspace_bytes, void *stream);

/* gq8_mqa_decode without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The split partials live in a static device array of
 * gq8_mqa_decode_noalloc_limit_bytes() bytes per GPU (1 064 960: one query
 * row of at most 16 heads and 2048 channels), held until the process ends;
 * a shape past 16 heads or a 2048-wide query row is refused with
 * GQ8_ERR_SHAPE (the shape check every attention entry point makes, which
 * keeps the partials within the array).  Every call on one
 * GPU shares that array, so calls that overlap on one GPU (two streams, two
 * threads) race. */
size_t gq8_mqa_decode_noalloc_limit_bytes(void);
int gq8_mqa_decode_noalloc(const float *query, const uint16_t *key_cache,
                           const uint16_t *value_cache, int heads, int kv_heads, int head_dim,
                           int key_count, float scale, float *out, void *stream);

/* MultiQueryPrefillAttention (MultiQueryAttention.h:275-308): rows query rows
 * at positions position_offset + r, row r over keys [0, position_offset + r]. */
int gq8_mqa_prefill(const float *queries, const uint16_t *key_cache,
                    const uint16_t *value_cache, int heads, int kv_heads, int head_dim,
                    int rows, int position_offset, float scale, float *out, void *workspace,
                    size_t workspace_bytes, void *stream);

/* GeGLU (GeGLU.h:50-73): out[r, c] = gelu_tanh(f[r, c]) * f[r, inter + c]
 * over fused [rows, 2 * inter]; out (fp32) and/or q8 (Q8 row buffer). */
int gq8_geglu(const float *fused, int rows, int intermediate, float *out, uint8_t *q8,
              void *stream);

/* SamplingOptions (Sampling/Sampler.h:33-51): temperature 0 is the argmax,
 * top_k 0 and top_p 1 switch their cut off, seed seeds std::mt19937_64. */
typedef struct gq8_sampling {
    float temperature;
    int top_k;
    float top_p;
    uint64_t seed;
} gq8_sampling;

/* Sampler::sample (Sampler.cpp:78-213) on the device: one token from one row
 * of vocab fp32 logits (device), the mask (device, optional, nonzero =
 * suppressed) applied first, scores logit / temperature in double, the top-k
 * then top-p cuts over the ranking (score descending, token ascending), the
 * softmax over what is left and the first candidate whose running mass
 * passes `uniform` (in [0, 1): one Sampler::uniform draw).  The id goes to
 * *token (device).  Options are refused as SamplingError refuses them
 * (Sampler.cpp:28-41): GQ8_ERR_ARGUMENT.  Synchronous. */
size_t gq8_sample_workspace_bytes(int vocab);
int gq8_sample_row(const float *logits, const float *mask, int vocab,
                   const gq8_sampling *options, double uniform, uint32_t *token,
                   void *workspace, size_t workspace_bytes, void *stream);

/* ArgmaxPartial + ArgmaxFinal (Argmax.h:47-257): per row the first maximum
 * over unmasked entries (mask may be NULL; nonzero = suppressed), 0 if none. */
size_t gq8_argmax_workspace_bytes(int rows, int length);
int gq8_argmax_rows(const float *logits, const float *mask, int rows, int length,
                    uint32_t *indices, void *workspace, size_t workspace_bytes, void *stream);

/* ======================================================================= */
/* Decoder runtime (HF::Decoder, Decoder.h:69-319).                        */
/* ======================================================================= */
typedef struct gq8_shape {
    int width, heads, kv_heads, head_dim, layers, intermediate, vocab, max_positions;
    int max_step_rows; /* 0 = max_positions (DecoderShape.h:85-89) */
    float rms_epsilon;
    double rope_theta;
    float embedding_scale;
} gq8_shape;

/* DecoderShape::validate (DecoderShape.cpp:41-92) plus the Int8Blocks shape
 * rule for every product weight. */
int gq8_shape_validate(const gq8_shape *shape);
/* DecoderShape::fromConfig for google/gemma-2b (GemmaConfig.h:41-92). */
gq8_shape gq8_gemma_2b_shape(int layers, int max_positions, int max_step_rows);

typedef struct gq8_decoder gq8_decoder;

/* Decoder::prepare (Decoder.cpp:172-218): validates, allocates the step
 * buffers, the per-layer fp16 KV caches and the rotary tables on the current
 * device.  Weights are loaded separately. */
int gq8_decoder_create(const gq8_shape *shape, gq8_decoder **out);
void gq8_decoder_destroy(gq8_decoder *decoder);

/* Tensor catalogue in GemmaTensors::all order (GemmaTensors.cpp:30-57):
 * 0 embedding; layer l at 1 + 9 l + {q, k, v, o, gate, up, down,
 * input_layernorm, post_attention_layernorm}; the final norm last. */
int gq8_tensor_count(const gq8_shape *shape);
int64_t gq8_tensor_elements(const gq8_shape *shape, int index);
int gq8_tensor_is_norm(const gq8_shape *shape, int index);

/* TensorLoader::loadProjectionWeight / loadStackedProjectionWeights /
 * loadFloatTensor (TensorLoader.cpp:186-347): fp32 host values, quantized on
 * the device (bit-exact with quantizeInt8Blocks) and placed in the layer's
 * fused q|k|v or gate|up tensor; norms stay fp32. */
int gq8_decoder_load_tensor(gq8_decoder *decoder, int index, const float *host_values);
/* The same tensor already quantized: Int8Blocks bytes from the host. */
int gq8_decoder_load_tensor_q8(gq8_decoder *decoder, int index, const uint8_t *host_bytes);
/* Seeded synthetic N(0, sigma) weights for every tensor (sigma 0.02 for the
 * projections and embedding, 0.1 for norms): Box-Muller in double over
 * std::mt19937_64, one engine per 2^20-element chunk seeded
 * ((0x5EED0000 + index) << 32) | chunk; generated on host threads, quantized
 * on the device.  threads <= 0 uses every hardware thread. */
int gq8_decoder_fill_synthetic(gq8_decoder *decoder, int threads);
/* The generator of gq8_decoder_fill_synthetic for one tensor, on the host:
 * count N(0, sigma) fp32 values from tensor_seed (all host threads). */
int gq8_normal_fill_host(uint64_t tensor_seed, double sigma, float *out, int64_t count);
/* Seeded uniform prompt ids: std::mt19937_64(seed), id = next() % vocab. */
int gq8_prompt_ids(uint64_t seed, int vocab, int count, int32_t *out);
/* The tensor's Int8Blocks bytes (or fp32 norm values) read back to the host. */
int gq8_decoder_read_tensor(gq8_decoder *decoder, int index, void *host_out, size_t bytes);

/* Decoder::beginSequence / position (Decoder.h:93-104). */
int gq8_decoder_begin_sequence(gq8_decoder *decoder);
int gq8_decoder_position(const gq8_decoder *decoder);
/* The position word on the device, after the decoder's stream has finished
 * (steps advance it on the device; it equals gq8_decoder_position after every
 * synchronous call).  Decoder::position (Decoder.h:101-104) read where the
 * steps keep it. */
int gq8_decoder_device_position(gq8_decoder *decoder);

/* Decoder::step (Decoder.cpp:644-706): n token ids (device, uint32) at
 * positions position .. position + n - 1; logits (device, fp32) receives
 * [n, vocab] when logits_rows == n, or only the last row when logits_rows == 1,
 * or nothing when logits == NULL.  Synchronous on the decoder's stream. */
int gq8_decoder_step(gq8_decoder *decoder, const uint32_t *tokens, int n, float *logits,
                     int logits_rows);
/* One-token steps run through the fused kernels (five launches a layer)
 * when the shape allows; 0 selects the unfused kernels (both compute the same
 * arithmetic).  On by default. */
int gq8_decoder_set_fused(gq8_decoder *decoder, int enabled);
/* The attention of the fused one-token step: 1 when it is the split kernel
 * (one workgroup a key split and group of query heads loads the split's K/V
 * rows once for all the heads, and the workgroups of a launch merge each
 * other's partials), 0 when it is the two-launch partial/merge pair (no
 * waits between workgroups), -1 when the shape has no fused step.  Replaces
 * MultiQueryDecodeAttention's dispatch (MultiQueryAttention.cpp:66-77). */
int gq8_decoder_attention_path(const gq8_decoder *decoder);
/* The choice behind gq8_decoder_attention_path for a shape, on the host:
 * 1 when the shape takes the split kernel and each of its launches (up to 64
 * key splits x KV heads x query-head groups workgroups, by key-count range)
 * fits `resident_workgroups` workgroups resident at once, else 0; negative
 * for a shape gq8_shape_validate refuses.  The decoder passes the kernel's
 * occupancy times the device's compute units.  No reference counterpart:
 * the reference's attention workgroups never wait on each other
 * (MultiQueryAttention.cpp:66-77). */
int gq8_decode_attention_fits(const gq8_shape *shape, int resident_workgroups);
/* Sets the split attention's error word, as a bounded wait does when it gives
 * up: the next step's waits give up at once, every kernel still exits, and
 * the check after it reports GQ8_ERR_DEVICE and puts the device and host
 * positions back to where that step began.  For tests of that path;
 * GQ8_ERR_SHAPE when the decoder's attention is not the split kernel.  No
 * reference counterpart (the reference has no waits between workgroups). */
int gq8_decoder_inject_wait_failure(gq8_decoder *decoder);
/* Gemma::setSampling (Generation/Gemma.cpp:198-202): how gq8_generate and
 * gq8_decoder_decode choose each id.  Temperature 0 (the default) is the
 * argmax; above it, each id is drawn on the device (gq8_sample_row's rule)
 * and written to its sequence slot, so no logits come back to the host
 * (Gemma::generateBySampling, Gemma.cpp:546-595, reads them back).  Every
 * sequence draws from the seed afresh (Gemma.cpp:549), one draw a sampled
 * token.  GQ8_ERR_ARGUMENT as SamplingError. */
int gq8_decoder_set_sampling(gq8_decoder *decoder, const gq8_sampling *options);
/* Decoder::hiddenStates (Decoder.h:119-121): the last step's rows after the
 * final norm, [rows, width] fp32, copied to the host. */
int gq8_decoder_hidden(gq8_decoder *decoder, float *host_out, int rows);
/* Intermediates of the last row of the last step, for bisecting against the
 * oracle: which = 0 normalised (input norm output), 1 attended, 2 activated
 * (GeGLU output), 3 hidden after the layer; fp32 values and their Q8 bytes
 * (q8 may be NULL).  Only kept when debug capture is on. */
int gq8_decoder_set_debug(gq8_decoder *decoder, int enabled);
int gq8_decoder_debug(gq8_decoder *decoder, int which, int layer, float *host_values,
                      uint8_t *host_q8);

/* ======================================================================= */
/* Greedy token loop (HF::Gemma::generate at temperature 0,                 */
/* Gemma.cpp:395-543).                                                      */
/* ======================================================================= */
typedef struct gq8_run_stats {
    double prefill_seconds;  /* Gemma::lastPrefillSeconds */
    double decode_seconds;   /* Gemma::lastDecodeSeconds  */
    int step_count;          /* Gemma::lastStepCount      */
    int generated;           /* tokens written to out     */
} gq8_run_stats;

/* Prefill the prompt in blocks of max_step_rows, then one token per step with
 * the id chosen on the device and fed back through the sequence slots; eos >=
 * 0 stops the run and is excluded (Gemma.cpp:503-504), eos < 0 never stops.
 * The run's limit is min(max_tokens, max_positions - prompt_length)
 * (Gemma.cpp:395-400; max_tokens <= 0 means the window).  use_graph != 0
 * replays each decode step as one captured hipGraph.  out receives up to the
 * limit token ids; returns the count (>= 0) or a negative status. */
int gq8_generate(gq8_decoder *decoder, const int32_t *prompt, int prompt_length,
                 int max_tokens, int eos, int use_graph, int32_t *out, gq8_run_stats *stats);
/* Gemma::onToken (Generation/Gemma.h:179-183): called once a generated id is
 * known, in order, on the thread that runs the loop (an EOS that stops the
 * run is not passed). */
typedef void (*gq8_token_callback)(int32_t token, void *user);
/* gq8_generate with the callback (NULL: none).  With eos >= 0 each id is
 * passed as it is read back, while the step after it runs; with eos < 0 the
 * steps are enqueued back to back and the ids are passed once the run ends. */
int gq8_generate_streaming(gq8_decoder *decoder, const int32_t *prompt, int prompt_length,
                           int max_tokens, int eos, int use_graph, int32_t *out,
                           gq8_run_stats *stats, gq8_token_callback on_token, void *user);

/* Continue the greedy loop `steps` tokens from the current position: each
 * step embeds the id in the slot at the position, runs the decoder and writes
 * its argmax into the next slot (Gemma.cpp:320-333, on-device feedback); no
 * EOS check.  Synchronous.  gq8_decoder_tokens reads slots back. */
int gq8_decoder_decode(gq8_decoder *decoder, int steps, int use_graph);
int gq8_decoder_tokens(gq8_decoder *decoder, int first, int count, int32_t *host_out);

/* Stage timing: every launch of a stage whose bit is set in stage_mask (0
 * turns timing off) that a step records outside a graph is bracketed by HIP
 * events on the decoder's stream.  Stages: 0 embed, 1 norm, 2 qkv product,
 * 3 rope+kv, 4 attention, 5 o product, 6 gate|up product, 7 geglu, 8 down
 * product, 9 lm_head product, 10 argmax.  Bracketing only the stages of
 * interest keeps the other launches free of event packets.
 * gq8_decoder_timing fills per-stage totals (milliseconds) and launch counts
 * since the last reset, and resets.  No reference counterpart: measurement. */
enum { GQ8_STAGE_COUNT = 11 };
int gq8_decoder_set_timing(gq8_decoder *decoder, int stage_mask);
int gq8_decoder_timing(gq8_decoder *decoder, double *milliseconds, int *launches);
/* Times one fused one-token kernel alone (stage 6 gate|up, 8 down or 9
 * lm_head): `repeats` rounds over every layer's weights (the lm_head: one
 * launch a round) back to back between two HIP events on the decoder's
 * stream; fills the milliseconds and the launch count.  Writes scratch only
 * (the sequence, the position and the KV cache are untouched).  No reference
 * counterpart: measurement. */
int gq8_decoder_time_kernel(gq8_decoder *decoder, int stage, int repeats, double *milliseconds,
                            int *launches);

/* ======================================================================= */
/* Checkpoint files: safetensors (Model/SafeTensors.h:78-183) and Gemma's   */
/* config.json (Model/GemmaConfig.h:41-92).  Host only; no GPU needed.      */
/* ======================================================================= */
/* dtype tags in Model/TensorType.h:12-27 order */
enum {
    GQ8_DTYPE_BOOL, GQ8_DTYPE_U8, GQ8_DTYPE_I8, GQ8_DTYPE_U16, GQ8_DTYPE_I16, GQ8_DTYPE_F16,
    GQ8_DTYPE_BF16, GQ8_DTYPE_U32, GQ8_DTYPE_I32, GQ8_DTYPE_F32, GQ8_DTYPE_U64, GQ8_DTYPE_I64,
    GQ8_DTYPE_F64
};
typedef struct gq8_safetensors gq8_safetensors;
/* SafeTensors::fromFile (a read-only mapping: nothing is resident before it
 * is read) and SafeTensors::fromBytes (a copy).  Every header rule is checked
 * before a byte is trusted (SafeTensors.h:85-101): a malformed length, JSON,
 * entry, dtype, byte range, shape/range mismatch or metadata value is
 * GQ8_ERR_FORMAT. */
int gq8_safetensors_open(const char *path, gq8_safetensors **out);
int gq8_safetensors_from_bytes(const uint8_t *bytes, uint64_t size, gq8_safetensors **out);
void gq8_safetensors_close(gq8_safetensors *file);
/* SafeTensors::tensors (sorted by name) / find (GQ8_ERR_FORMAT when absent) */
int gq8_safetensors_count(const gq8_safetensors *file);
int gq8_safetensors_find(const gq8_safetensors *file, const char *name);
/* TensorInfo of entry `index`; name stays valid while the file is open; up to
 * shape_capacity dimensions are written. */
int gq8_safetensors_info(const gq8_safetensors *file, int index, const char **name, int *dtype,
                         int *rank, int64_t *shape, int shape_capacity, uint64_t *byte_count);
/* widenTensorElements (SafeTensors.h:71-76): elements [first, first + count)
 * widened to fp32 (F16 and BF16 exactly); GQ8_ERR_FORMAT for integer dtypes. */
int gq8_safetensors_read_floats(const gq8_safetensors *file, int index, int64_t first,
                                int64_t count, float *out);
/* SafeTensors::rawBytes: the entry's bytes in the mapping (NULL if no such entry). */
const uint8_t *gq8_safetensors_raw(const gq8_safetensors *file, int index);
/* SafeTensors::metadata: the __metadata__ string pairs, sorted by key. */
int gq8_safetensors_metadata_count(const gq8_safetensors *file);
int gq8_safetensors_metadata(const gq8_safetensors *file, int index, const char **key,
                             const char **value);

typedef struct gq8_token_ids {
    int bos, eos, pad;
} gq8_token_ids;
/* GemmaConfig::fromJson (GemmaConfig.cpp:140-205) and DecoderShape::fromConfig:
 * every field defaults to google/gemma-2b's value; model_type must be
 * "gemma"; token ids are a number or the first of a list.  max_positions > 0
 * caps the window below max_position_embeddings.  An untied output projection
 * is GQ8_ERR_SHAPE (this decoder's lm_head is the embedding). */
int gq8_gemma_config_parse(const char *json_text, size_t length, int max_positions,
                           int max_step_rows, gq8_shape *shape, gq8_token_ids *tokens);
/* TensorLoader::load (TensorLoader.cpp:186-347) over the checkpoint's shards:
 * every tensor of the catalogue is found by its checkpoint name
 * ("model.embed_tokens.weight", "model.layers.N.self_attn.q_proj.weight", ...,
 * "model.norm.weight"; GemmaTensors.h:29-44) and checked against the shape
 * before anything is uploaded (GemmaTensors::checkAgainst), then widened to
 * fp32 on the host in pieces and quantized to Int8Blocks on the device. */
int gq8_decoder_load_safetensors(gq8_decoder *decoder, gq8_safetensors *const *shards,
                                 int shard_count);

/* ======================================================================= */
/* Lockstep decode of up to 16 independent sequences over one decoder's     */
/* weights.  The reference has no batch dimension: a batch stands for S     */
/* separate HF::Decoders (Decoder.h:69-319, one sequence and one cache      */
/* each) run by S greedy loops (Gemma.cpp:459-543), and every sequence's     */
/* ids equal its own one-sequence run's.                                    */
/* ======================================================================= */
typedef struct gq8_batch gq8_batch;
/* S in [1, 16] sequences, each with its own fp16 cache and max_positions + 1
 * token slots; the decoder's weights are shared, so the decoder must outlive
 * the batch.  Where every product's inner size is a multiple of 256 the batch
 * also keeps a copy of the weights in the products' MFMA fragment order
 * (about the size of the weights: 2.98 GB for Gemma-2B), made at its first
 * decode and again at a decode after any weight upload to the decoder.
 * GQ8_ERR_SHAPE where the one-token attention layout does not cover the
 * decoder's shape. */
int gq8_batch_create(gq8_decoder *decoder, int sequences, gq8_batch **out);
void gq8_batch_destroy(gq8_batch *batch);
/* Gemma::generate's prefill (Gemma.cpp:350-380, 402-424) of one sequence,
 * restarting it: the prompt goes through the decoder's own step path in
 * blocks of max_step_rows, and the last row's argmax fills slot
 * prompt_length.  Refusals as gq8_generate's.  Synchronous. */
int gq8_batch_prefill(gq8_batch *batch, int sequence, const int32_t *prompt, int prompt_length);
/* `steps` lockstep steps: each takes every sequence's token at its position,
 * writes its argmax into the next slot and advances the position (the
 * greedy loop's step, Gemma.cpp:320-333, for every sequence at once); no EOS
 * check.  GQ8_ERR_NOT_PREPARED if a sequence has no prompt, GQ8_ERR_WINDOW if
 * one would pass max_positions.  use_graph != 0 replays one captured step.
 * Synchronous. */
int gq8_batch_decode(gq8_batch *batch, int steps, int use_graph);
int gq8_batch_sequences(const gq8_batch *batch);
/* The position of the sequence's next step (prompt length + steps so far). */
int gq8_batch_position(const gq8_batch *batch, int sequence);
/* Slots [first, first + count) of one sequence (prompt, then generated ids). */
int gq8_batch_tokens(gq8_batch *batch, int sequence, int first, int count, int32_t *host_out);
/* The last lockstep step's logits, [S, vocab] fp32, copied to the host. */
int gq8_batch_logits(gq8_batch *batch, float *host_out);

/* ======================================================================= */
/* Tokenizer: Gemma's SentencePiece BPE from tokenizer.json, on the host    */
/* (Tokenizer/Tokenizer.h:35-124; Metaspace.h; ByteFallback.h).             */
/* ======================================================================= */
typedef struct gq8_tokenizer gq8_tokenizer;
/* SpecialTokens (Tokenizer/SpecialTokens.h:16-24): -1 where the file has none. */
typedef struct gq8_special_tokens {
    int32_t pad, eos, bos, unk, start_of_turn, end_of_turn;
} gq8_special_tokens;
/* Tokenizer::fromJsonText / fromFile (Tokenizer.cpp:206-301): GQ8_ERR_FORMAT
 * for malformed JSON, a missing model.vocab or model.merges, or a bad merge
 * rule, with the reason in gq8_last_error. */
int gq8_tokenizer_from_json(const char *text, size_t length, gq8_tokenizer **out);
int gq8_tokenizer_open(const char *path, gq8_tokenizer **out);
void gq8_tokenizer_destroy(gq8_tokenizer *tokenizer);
/* Tokenizer::encode / encodeWithBos (Tokenizer.cpp:565-609) of `length`
 * bytes of text: returns the number of ids (or a negative status) and writes
 * the first min(count, capacity) of them. */
int gq8_tokenizer_encode(const gq8_tokenizer *tokenizer, const char *text, size_t length,
                         int with_bos, int32_t *out, int capacity);
/* Tokenizer::decode / decodeKeepingSpecialTokens (Tokenizer.cpp:611-683):
 * *length receives the text's byte length; the first min(length, capacity)
 * bytes go to out (no terminator).  Ids outside the vocabulary are skipped. */
int gq8_tokenizer_decode(const gq8_tokenizer *tokenizer, const int32_t *tokens, int count,
                         int keep_special, char *out, size_t capacity, size_t *length);
int gq8_tokenizer_vocabulary_size(const gq8_tokenizer *tokenizer);
int gq8_tokenizer_specials(const gq8_tokenizer *tokenizer, gq8_special_tokens *out);
int gq8_tokenizer_is_special(const gq8_tokenizer *tokenizer, int32_t token);
/* Tokenizer::textForToken: the piece as the vocabulary spells it (empty
 * outside the vocabulary); tokenForText: the id of a piece, or -1. */
int gq8_tokenizer_token_text(const gq8_tokenizer *tokenizer, int32_t token, char *out,
                             size_t capacity, size_t *length);
int32_t gq8_tokenizer_token_for_text(const gq8_tokenizer *tokenizer, const char *text,
                                     size_t length);
/* Tokenizer::metaspace (Metaspace.h:14-45): the replacement for a space, the
 * dummy prefix and the per-word split, as read from the file. */
int gq8_tokenizer_metaspace(const gq8_tokenizer *tokenizer, char *replacement, size_t capacity,
                            size_t *length, int *prepends, int *splits);

/* ======================================================================= */
/* Model directory runtime: HF::Gemma (Generation/Gemma.h:65-251) over a    */
/* Hugging Face Gemma directory (Model/ModelFiles.h:11-66).                 */
/* ======================================================================= */
typedef struct gq8_gemma gq8_gemma;
/* ModelFiles' files (ModelFileNames, ModelFiles.h:13-27) */
enum {
    GQ8_FILE_CONFIG, GQ8_FILE_GENERATION_CONFIG, GQ8_FILE_SHARD_INDEX, GQ8_FILE_TOKENIZER_JSON,
    GQ8_FILE_TOKENIZER_MODEL, GQ8_FILE_GGUF, GQ8_FILE_SHARD
};
int gq8_gemma_create(gq8_gemma **out);
void gq8_gemma_destroy(gq8_gemma *gemma);
/* Gemma::load(modelDirectory) (Gemma.cpp:64-84): ModelFiles::fromDirectory
 * (config.json required; model.safetensors.index.json naming its shards by
 * plain file name, else model.safetensors, required; generation_config.json,
 * tokenizer.json, tokenizer.model and gemma-2b.gguf recorded when present,
 * ModelFiles.cpp:77-99), GemmaConfig::fromModelFiles (generation_config.json's
 * bos / eos / pad over config.json's, GemmaConfig.cpp:204-223), the tokenizer
 * (required, and no larger than the config's vocabulary, Gemma.cpp:120-139)
 * and every shard mapped.  The maximum token count returns to 0 and a
 * prepared decoder is dropped.  GQ8_ERR_FORMAT names the file at fault.
 * Host only. */
int gq8_gemma_load(gq8_gemma *gemma, const char *model_directory);
/* ModelFiles::directoryFromEnvironment (ModelFiles.cpp:100-106): the
 * GEMMA_MODEL_DIR variable, empty when unset.  *length gets its byte length;
 * up to capacity bytes go to out (no terminator). */
int gq8_gemma_directory_from_environment(char *out, size_t capacity, size_t *length);
int gq8_gemma_is_loaded(const gq8_gemma *gemma);
int gq8_gemma_is_prepared(const gq8_gemma *gemma);
/* A located file's path (which = GQ8_FILE_*, index selects the shard):
 * *length is 0 for a file the directory does not hold. */
int gq8_gemma_file(const gq8_gemma *gemma, int which, int index, char *out, size_t capacity,
                   size_t *length);
int gq8_gemma_shard_count(const gq8_gemma *gemma);
/* GemmaConfig's shape and token ids after load (config.json with
 * generation_config.json applied). */
int gq8_gemma_config(const gq8_gemma *gemma, gq8_shape *shape, gq8_token_ids *tokens);
/* Gemma::setMaximumTokens / setPromptCapacity (Gemma.cpp:164-179): a
 * negative count or a capacity below one row is GQ8_ERR_ARGUMENT.  The
 * capacity is taken at prepare. */
int gq8_gemma_set_maximum_tokens(gq8_gemma *gemma, int count);
int gq8_gemma_maximum_tokens(const gq8_gemma *gemma);
int gq8_gemma_set_prompt_capacity(gq8_gemma *gemma, int rows);
int gq8_gemma_prompt_capacity(const gq8_gemma *gemma);
/* Gemma::setSampling (Gemma.cpp:195-202); validated as SamplingError does. */
int gq8_gemma_set_sampling(gq8_gemma *gemma, const gq8_sampling *options);
/* Gemma::onToken: NULL restores the no-op. */
int gq8_gemma_set_on_token(gq8_gemma *gemma, gq8_token_callback on_token, void *user);
/* Gemma::prepare (Gemma.cpp:207-243): the decoder of shape
 * DecoderShape::fromConfig with maxStepRows = min(prompt capacity, window),
 * its weights read from the shards by checkpoint name and quantized to
 * Int8Blocks on the device, and the sampling options.  GQ8_ERR_NOT_PREPARED
 * before load. */
int gq8_gemma_prepare(gq8_gemma *gemma);
/* The prepared decoder (NULL before prepare), for the op-level calls. */
gq8_decoder *gq8_gemma_decoder(gq8_gemma *gemma);
/* The loaded tokenizer (NULL before load). */
const gq8_tokenizer *gq8_gemma_tokenizer(const gq8_gemma *gemma);
/* Gemma::generate (Gemma.cpp:402-457): the generated ids with the EOS
 * excluded, up to min(maximum tokens or the window, max_positions - prompt
 * length), stopping at the config's eos.  Returns the count (or a negative
 * status); the first min(count, capacity) ids go to out.  Refusals as
 * gq8_generate's; GQ8_ERR_NOT_PREPARED before prepare. */
int gq8_gemma_generate(gq8_gemma *gemma, const int32_t *prompt, int prompt_length, int32_t *out,
                       int capacity);
/* Gemma::generateFromText (Gemma.cpp:596-603): the text encoded with the
 * BOS in front, then generate. */
int gq8_gemma_generate_from_text(gq8_gemma *gemma, const char *text, size_t length, int32_t *out,
                                 int capacity);
/* Gemma::generateText (Gemma.cpp:605-609): generateFromText decoded back
 * with the special tokens dropped.  *length gets the text's byte length; up
 * to capacity bytes go to out. */
int gq8_gemma_generate_text(gq8_gemma *gemma, const char *text, size_t length, char *out,
                            size_t capacity, size_t *out_length);
/* Gemma::textForTokens (Gemma.cpp:611-615): after load. */
int gq8_gemma_text_for_tokens(const gq8_gemma *gemma, const int32_t *tokens, int count, char *out,
                              size_t capacity, size_t *length);
/* lastPrefillSeconds / lastDecodeSeconds / lastStepCount of the last run. */
int gq8_gemma_last_stats(const gq8_gemma *gemma, gq8_run_stats *stats);

#ifdef __cplusplus
}
#endif
#endif
