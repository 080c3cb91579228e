/*
 * gemma_oracle.c -- CPU oracle for the Gemma-2B Int8Blocks token loop.
 *
 * TEST INFRASTRUCTURE ONLY (see gemma_oracle.h).  Reference citations are
 * relative to the root of eyalamirmusic/HuggingFaceEACP.
 *
 * Built with -ffp-contract=off so every double expression below is evaluated
 * exactly as written (no fused multiply-adds the source does not spell).
 */
#include "gemma_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================================================================== */
/* IEEE binary16, written from IEEE 754-2008 section 3.6 (binary16: 1 sign,  */
/* 5 exponent bits biased by 15, 10 fraction bits) with round to nearest,    */
/* ties to even -- the conversion eacp's halfFromFloat/halfToFloat perform   */
/* (used at Lib/HuggingFaceEACP/Kernels/Int8Blocks.cpp:32-33, 101, 121).   */
/* ======================================================================== */
uint16_t gor_half_from_float(float value)
{
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);

    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t exponent = (bits >> 23) & 0xFFu;
    uint32_t mantissa = bits & 0x7FFFFFu;

    if (exponent == 0xFFu) {
        if (mantissa == 0)
            return (uint16_t) (sign | 0x7C00u);
        /* a NaN stays a NaN: quiet bit set, top payload bits kept */
        return (uint16_t) (sign | 0x7E00u | (mantissa >> 13));
    }

    const int halfExponent = (int) exponent - 127 + 15;

    if (halfExponent >= 31)
        return (uint16_t) (sign | 0x7C00u);

    if (halfExponent <= 0) {
        /* below 2^-25 every value rounds to zero (2^-25 itself ties to 0) */
        if (halfExponent < -10)
            return (uint16_t) sign;

        mantissa |= 0x800000u;
        const int shift = 14 - halfExponent; /* 14 .. 24 */
        uint32_t half = mantissa >> shift;
        const uint32_t rest = mantissa & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);

        if (rest > halfway || (rest == halfway && (half & 1u)))
            ++half; /* may carry into the smallest normal: still correct */

        return (uint16_t) (sign | half);
    }

    uint32_t half = sign | ((uint32_t) halfExponent << 10) | (mantissa >> 13);
    const uint32_t rest = mantissa & 0x1FFFu;

    if (rest > 0x1000u || (rest == 0x1000u && (half & 1u)))
        ++half; /* a carry into the exponent is the correct rounding, up to inf */

    return (uint16_t) half;
}

float gor_half_to_float(uint16_t half)
{
    const uint32_t sign = ((uint32_t) half & 0x8000u) << 16;
    const uint32_t exponent = ((uint32_t) half >> 10) & 0x1Fu;
    uint32_t mantissa = (uint32_t) half & 0x3FFu;
    uint32_t bits;

    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            /* subnormal: normalise into an fp32 normal */
            int e = -1;
            do {
                ++e;
                mantissa <<= 1;
            } while ((mantissa & 0x400u) == 0);
            bits = sign | ((uint32_t) (127 - 15 - e) << 23) | ((mantissa & 0x3FFu) << 13);
        }
    } else if (exponent == 0x1Fu) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent - 15 + 127) << 23) | (mantissa << 13);
    }

    float value;
    memcpy(&value, &bits, sizeof value);
    return value;
}

static float g_half_table[65536];
static int g_half_table_ready = 0;

static void ensure_half_table(void)
{
    if (g_half_table_ready)
        return;
    for (uint32_t h = 0; h < 65536u; ++h)
        g_half_table[h] = gor_half_to_float((uint16_t) h);
    g_half_table_ready = 1;
}

/* ======================================================================== */
/* Int8Blocks (Lib/HuggingFaceEACP/Kernels/Int8Blocks.h:9-88,                */
/* Int8Blocks.cpp:70-124).                                                   */
/* ======================================================================== */
int64_t gor_int8_block_count(int64_t element_count)
{
    return element_count / GOR_BLOCK; /* Int8Blocks.cpp:70-73 */
}

int64_t gor_int8_blocks_byte_count(int64_t element_count)
{
    return element_count + 2 * gor_int8_block_count(element_count); /* :164-167 */
}

int gor_quantizes_as_int8_blocks(int64_t contiguous_extent, int64_t element_count)
{
    /* Int8Blocks.cpp:80-85 */
    return contiguous_extent > 0 && element_count > 0
           && contiguous_extent % GOR_BLOCK == 0
           && element_count % (2 * GOR_BLOCK) == 0;
}

/* blockScaleBits, Int8Blocks.cpp:25-36: the largest magnitude over 127 as a
 * float division, narrowed to fp16; a scale that is zero, infinite or NaN is
 * stored as zero.  std::max(largest, |x|) keeps `largest` when |x| is a NaN,
 * which is what the comparison below does too. */
uint16_t gor_block_scale_bits(const float *block)
{
    float largest = 0.f;

    for (int index = 0; index < GOR_BLOCK; ++index) {
        const float magnitude = fabsf(block[index]);
        if (largest < magnitude)
            largest = magnitude;
    }

    const uint16_t bits = gor_half_from_float(largest / (float) 127.0);
    const float scale = gor_half_to_float(bits);

    return (scale > 0.f && isfinite(scale)) ? bits : (uint16_t) 0u;
}

/* quantizedByte, Int8Blocks.cpp:41-47: round to nearest, ties to even, of
 * the double quotient by the narrowed scale, clamped to [-127, 127].  The
 * reference leaves a NaN element undefined (a NaN cast to an integer); here it
 * is stored as zero. */
int8_t gor_quantized_byte(float value, float scale)
{
    const double rounded = nearbyint((double) value / (double) scale);

    if (rounded != rounded)
        return 0;
    if (rounded < -127.0)
        return -127;
    if (rounded > 127.0)
        return 127;
    return (int8_t) rounded;
}

/* quantizeInt8Blocks, Int8Blocks.cpp:87-110: `values` holds value_count
 * elements beginning at element `first` of a tensor of element_count, whose
 * bytes are `destination` in the two-region layout. */
void gor_quantize_int8_blocks(const float *values, int64_t value_count, int64_t first,
                              int64_t element_count, uint8_t *destination)
{
    for (int64_t at = 0; at < value_count; at += GOR_BLOCK) {
        const float *block = values + at;
        const uint16_t bits = gor_block_scale_bits(block);
        const float scale = gor_half_to_float(bits);
        const int64_t element = first + at;
        const int64_t scaleAt = element_count + 2 * (element / GOR_BLOCK);

        destination[scaleAt] = (uint8_t) (bits & 0xFFu);
        destination[scaleAt + 1] = (uint8_t) (bits >> 8);

        for (int index = 0; index < GOR_BLOCK; ++index)
            destination[element + index] =
                bits == 0 ? 0u : (uint8_t) gor_quantized_byte(block[index], scale);
    }
}

/* dequantizeInt8Blocks, Int8Blocks.cpp:112-124: the widened fp16 scale times
 * the sign-extended byte, as an fp32 product. */
void gor_dequantize_int8_blocks(const uint8_t *stored, int64_t element_count,
                                float *values)
{
    for (int64_t index = 0; index < element_count; ++index) {
        const int64_t at = element_count + 2 * (index / GOR_BLOCK);
        const uint16_t bits = (uint16_t) (stored[at] | ((uint32_t) stored[at + 1] << 8));
        const float signedByte = (float) ((int) (stored[index] ^ 0x80u) - 128);

        values[index] = gor_half_to_float(bits) * signedByte;
    }
}

void gor_quantize_row(const float *x, int64_t n, int8_t *q, uint16_t *scale_bits)
{
    for (int64_t b = 0; b < n / GOR_BLOCK; ++b) {
        const float *block = x + b * GOR_BLOCK;
        const uint16_t bits = gor_block_scale_bits(block);
        const float scale = gor_half_to_float(bits);

        scale_bits[b] = bits;
        for (int i = 0; i < GOR_BLOCK; ++i)
            q[b * GOR_BLOCK + i] = bits == 0 ? 0 : gor_quantized_byte(block[i], scale);
    }
}

/* ======================================================================== */
/* Seeded synthetic inputs.                                                  */
/* MT19937-64 from Matsumoto & Nishimura's published algorithm (the engine   */
/* std::mt19937_64 specifies: w=64 n=312 m=156 r=31 a=0xB5026F5AA96619E9     */
/* u=29 d=0x5555555555555555 s=17 b=0x71D67FFFEDA60000 t=37                  */
/* c=0xFFF7EEE000000000 l=43 f=6364136223846793005).                         */
/* ======================================================================== */
void gor_mt64_seed(gor_mt64 *engine, uint64_t seed)
{
    engine->state[0] = seed;
    for (int i = 1; i < 312; ++i)
        engine->state[i] = 6364136223846793005ULL
                               * (engine->state[i - 1] ^ (engine->state[i - 1] >> 62))
                           + (uint64_t) i;
    engine->index = 312;
}

uint64_t gor_mt64_next(gor_mt64 *engine)
{
    static const uint64_t upper = 0xFFFFFFFF80000000ULL;
    static const uint64_t lower = 0x7FFFFFFFULL;

    if (engine->index >= 312) {
        for (int i = 0; i < 312; ++i) {
            const uint64_t x = (engine->state[i] & upper)
                               | (engine->state[(i + 1) % 312] & lower);
            uint64_t next = x >> 1;
            if (x & 1u)
                next ^= 0xB5026F5AA96619E9ULL;
            engine->state[i] = engine->state[(i + 156) % 312] ^ next;
        }
        engine->index = 0;
    }

    uint64_t y = engine->state[engine->index++];
    y ^= (y >> 29) & 0x5555555555555555ULL;
    y ^= (y << 17) & 0x71D67FFFEDA60000ULL;
    y ^= (y << 37) & 0xFFF7EEE000000000ULL;
    y ^= y >> 43;
    return y;
}

enum { GOR_CHUNK = 1 << 20 };

static double unit_interval(gor_mt64 *engine)
{
    return (double) (gor_mt64_next(engine) >> 11) * (1.0 / 9007199254740992.0);
}

/* Box-Muller in double: r = sqrt(-2 ln(1 - u1)), theta = 2 pi u2; the pair
 * (r cos theta, r sin theta) fills two consecutive elements. */
void gor_normal_fill(uint64_t tensor_seed, double sigma, float *out, int64_t count)
{
    const int64_t chunks = (count + GOR_CHUNK - 1) / GOR_CHUNK;
    const double twoPi = 6.283185307179586476925286766559;

#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t chunk = 0; chunk < chunks; ++chunk) {
        gor_mt64 engine;
        gor_mt64_seed(&engine, (tensor_seed << 32) | (uint64_t) chunk);

        const int64_t begin = chunk * GOR_CHUNK;
        const int64_t end = begin + GOR_CHUNK < count ? begin + GOR_CHUNK : count;

        for (int64_t at = begin; at < end; at += 2) {
            const double u1 = unit_interval(&engine);
            const double u2 = unit_interval(&engine);
            const double radius = sqrt(-2.0 * log(1.0 - u1));
            const double angle = twoPi * u2;

            out[at] = (float) (sigma * (radius * cos(angle)));
            if (at + 1 < end)
                out[at + 1] = (float) (sigma * (radius * sin(angle)));
        }
    }
}

void gor_prompt_ids(uint64_t seed, int vocab, int count, int32_t *out)
{
    gor_mt64 engine;
    gor_mt64_seed(&engine, seed);
    for (int i = 0; i < count; ++i)
        out[i] = (int32_t) (gor_mt64_next(&engine) % (uint64_t) vocab);
}

/* ======================================================================== */
/* Small kernels.                                                            */
/* ======================================================================== */

/* makeRotaryTable, Lib/HuggingFaceEACP/Kernels/RoPE.cpp:7-34: inverse
 * frequency 1 / theta^(2i / headDim) in double, angle = position * it, cos and
 * sin in double narrowed to fp32; [maxPositions, headDim / 2] row-major. */
void gor_rotary_table(int max_positions, int head_dim, double theta, float *cosines,
                      float *sines)
{
    const int half = head_dim / 2;

    for (int channel = 0; channel < half; ++channel) {
        const double exponent = 2.0 * channel / (double) head_dim;
        const double inverseFrequency = 1.0 / pow(theta, exponent);

        for (int position = 0; position < max_positions; ++position) {
            const double angle = (double) position * inverseFrequency;
            const int64_t at = (int64_t) position * half + channel;

            cosines[at] = (float) cos(angle);
            sines[at] = (float) sin(angle);
        }
    }
}

/* RMSNorm, Lib/HuggingFaceEACP/Kernels/RMSNorm.h:7-56 and
 * Tests/Decoder/ReferenceDecoder.h:108-133: x * 1/sqrt(mean(x^2) + eps) *
 * (1 + w), the sum in double, the output rounded to fp32 once. */
void gor_rmsnorm_row(const float *x, const float *weight, int n, float epsilon,
                     float *out)
{
    double squares = 0.0;

    for (int i = 0; i < n; ++i)
        squares += (double) x[i] * (double) x[i];

    const double scale = 1.0 / sqrt(squares / (double) n + (double) epsilon);

    for (int i = 0; i < n; ++i)
        out[i] = (float) (((double) x[i] * scale) * (1.0 + (double) weight[i]));
}

/* tanh GELU, Lib/HuggingFaceEACP/Kernels/Gelu.h:27-46 with the double
 * constants of Tests/Kernels/Common.h:170-175; the tanh argument saturates to
 * +-1 at |z| >= 10 as eacp's saturatingTanh does (Gelu.h:27-38). */
double gor_tanh_gelu(double x)
{
    const double rootTwoOverPi = 0.7978845608028654;
    const double inner = rootTwoOverPi * (x + 0.044715 * x * x * x);
    const double t = inner >= 10.0 ? 1.0 : (inner <= -10.0 ? -1.0 : tanh(inner));

    return 0.5 * x * (1.0 + t);
}

/* GeGLU, Lib/HuggingFaceEACP/Kernels/GeGLU.h:50-73: gelu(gate) * up. */
float gor_geglu(float gate, float up)
{
    return (float) (gor_tanh_gelu((double) gate) * (double) up);
}

/* RoPE, Lib/HuggingFaceEACP/Kernels/RoPE.h:59-81: rotate-half of every head
 * of one row at `position`, from the fp32 table, in double, rounded once. */
void gor_rope_row(float *x, int row_stride, int heads, int head_dim, int position,
                  const float *cosines, const float *sines)
{
    const int half = head_dim / 2;
    (void) row_stride;

    for (int head = 0; head < heads; ++head) {
        float *base = x + head * head_dim;
        for (int pair = 0; pair < half; ++pair) {
            const double c = (double) cosines[(int64_t) position * half + pair];
            const double s = (double) sines[(int64_t) position * half + pair];
            const double lo = (double) base[pair];
            const double hi = (double) base[pair + half];

            base[pair] = (float) (lo * c - hi * s);
            base[pair + half] = (float) (hi * c + lo * s);
        }
    }
}

/* The Q8 product of one activation row: per 32-block the exact int8 dot
 * times (fp16 weight scale * fp16 activation scale), summed over the blocks in
 * double, rounded to fp32 once.  The weight is in the split-region layout of
 * Int8Blocks.h:19-31 (bytes of row r at r * inner, the scale of block b of row
 * r at half index rows * inner / 2 + r * inner / 32 + b).  This is the product
 * of SplitLinearProgram<Int8Blocks> (Lib/HuggingFaceEACP/Kernels/Linear.h:
 * 128-357) with the activation row taken through Int8Blocks as well. */
/* Built for three instruction sets, picked at load time by the CPU (the
 * integer dots vectorize; the double sum stays in block order on each). */
__attribute__((target_clones("avx512f", "avx2", "default")))
static double q8_row_dot(const int8_t *xq, const double *xs, const uint8_t *weights,
                         int64_t rows, int64_t inner, int64_t row)
{
    const int8_t *w = (const int8_t *) weights + row * inner;
    const uint8_t *scaleBytes = weights + rows * inner + 2 * (row * (inner / GOR_BLOCK));
    double total = 0.0;

    for (int64_t b = 0; b < inner / GOR_BLOCK; ++b) {
        int32_t dot = 0;
        const int8_t *wb = w + b * GOR_BLOCK;
        const int8_t *xb = xq + b * GOR_BLOCK;

        for (int i = 0; i < GOR_BLOCK; ++i)
            dot += (int32_t) wb[i] * (int32_t) xb[i];

        const uint16_t bits =
            (uint16_t) (scaleBytes[2 * b] | ((uint32_t) scaleBytes[2 * b + 1] << 8));
        const double scale = (double) g_half_table[bits] * xs[b];

        total += scale * (double) dot;
    }

    return total;
}

static void q8_matvec_double(const int8_t *xq, const uint16_t *xs,
                             const uint8_t *weights, int64_t rows, int64_t inner,
                             double *out)
{
    ensure_half_table();

    double *activationScales = (double *) malloc(sizeof(double) * (size_t) (inner / GOR_BLOCK));
    for (int64_t b = 0; b < inner / GOR_BLOCK; ++b)
        activationScales[b] = (double) g_half_table[xs[b]];

#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < rows; ++row)
        out[row] = q8_row_dot(xq, activationScales, weights, rows, inner, row);

    free(activationScales);
}

void gor_q8_matvec(const int8_t *xq, const uint16_t *xs, const uint8_t *weights,
                   int64_t rows, int64_t inner, float *out)
{
    double *exact = (double *) malloc(sizeof(double) * (size_t) rows);
    q8_matvec_double(xq, xs, weights, rows, inner, exact);
    for (int64_t row = 0; row < rows; ++row)
        out[row] = (float) exact[row];
    free(exact);
}

/* Argmax.h:14-38 and Sampler.cpp:60-76: the first maximum over the unmasked
 * entries (a strictly greater value replaces the best), 0 if all are masked. */
int gor_argmax(const float *logits, const float *mask, int n)
{
    int best = -1;

    for (int token = 0; token < n; ++token) {
        if (mask && mask[token] != 0.f)
            continue;
        if (best < 0 || logits[token] > logits[best])
            best = token;
    }

    return best < 0 ? 0 : best;
}

/* ---- Sampler.cpp:78-213: one token from one row of logits --------------
 * Temperature 0 is the argmax.  Otherwise the unmasked tokens become
 * candidates scored logit * (1 / temperature) in double (token order);
 * top-k keeps the k best by (score descending, token ascending) and orders
 * them; top-p orders the candidates, takes their softmax, and keeps the
 * shortest prefix whose running mass reaches p (the boundary kept); the
 * survivors' softmax is drawn from by walking them in their order until the
 * running mass passes the uniform draw, the last one when rounding leaves the
 * total short.  The ordered k best are what nth_element + sort leave, since
 * the order is total; a full sort finds the same prefix. */
typedef struct {
    int token;
    double score;
} sample_candidate;

static int ranks_before(const void *l, const void *r)
{
    const sample_candidate *a = (const sample_candidate *) l, *b = (const sample_candidate *) r;
    if (a->score != b->score)
        return a->score > b->score ? -1 : 1;
    return a->token < b->token ? -1 : (a->token > b->token);
}

static void sample_softmax(const sample_candidate *c, int n, double *p)
{
    double largest = -DBL_MAX, total = 0.0;
    for (int i = 0; i < n; ++i)
        if (c[i].score > largest)
            largest = c[i].score;
    for (int i = 0; i < n; ++i) {
        p[i] = exp(c[i].score - largest);
        total += p[i];
    }
    for (int i = 0; i < n; ++i)
        p[i] /= total;
}

int gor_sample(const float *logits, const float *mask, int n, float temperature, int top_k,
               float top_p, double uniform)
{
    if (temperature == 0.f)
        return gor_argmax(logits, mask, n);
    sample_candidate *c = (sample_candidate *) malloc(sizeof(sample_candidate) * (size_t) n);
    double *p = (double *) malloc(sizeof(double) * (size_t) n);
    const double inverse = 1.0 / (double) temperature;
    int count = 0;
    for (int token = 0; token < n; ++token) {
        if (mask && mask[token] != 0.f)
            continue;
        c[count].token = token;
        c[count].score = (double) logits[token] * inverse;
        ++count;
    }
    int chosen = 0;
    if (count > 0) {
        if (top_k > 0 && top_k < count) {
            qsort(c, (size_t) count, sizeof(sample_candidate), ranks_before);
            count = top_k;
        }
        if (top_p < 1.f) {
            qsort(c, (size_t) count, sizeof(sample_candidate), ranks_before);
            sample_softmax(c, count, p);
            const double wanted = (double) top_p;
            double mass = 0.0;
            int kept = 0;
            while (kept < count && mass < wanted)
                mass += p[kept++];
            count = kept;
        }
        sample_softmax(c, count, p);
        double mass = 0.0;
        chosen = c[count - 1].token;
        for (int i = 0; i < count; ++i) {
            mass += p[i];
            if (uniform < mass) {
                chosen = c[i].token;
                break;
            }
        }
    }
    free(c);
    free(p);
    return chosen;
}

/* Sampler::uniform (Sampler.cpp:209-212): the top 53 bits of one engine draw. */
double gor_mt64_uniform(gor_mt64 *engine)
{
    return (double) (gor_mt64_next(engine) >> 11) * 0x1.0p-53;
}

/* Multi-query attention of one query row over key_count cached rows
 * (Lib/HuggingFaceEACP/Kernels/MultiQueryAttention.h:138-260 and
 * Tests/Decoder/ReferenceDecoder.h:208-272): query head h reads KV head
 * h / (heads / kv_heads); scores scale * q.k in double, softmax by the
 * maximum, the output the weighted value sum divided by the weight sum,
 * rounded to fp32 once.  Keys and values are fp16. */
typedef double (*cache_reader)(const void *cache, int64_t index);

static double read_half_cache(const void *cache, int64_t index)
{
    return (double) g_half_table[((const uint16_t *) cache)[index]];
}

static double read_float_cache(const void *cache, int64_t index)
{
    return (double) ((const float *) cache)[index];
}

static void mqa_row(const float *query, const void *keys, const void *values,
                    cache_reader read, int heads, int kv_heads, int head_dim, int key_count,
                    float scale, float *out)
{
    ensure_half_table();

    const int kvWidth = kv_heads * head_dim;
    const int perKv = heads / kv_heads;
    double *weights = (double *) malloc(sizeof(double) * (size_t) key_count);
    double *acc = (double *) malloc(sizeof(double) * (size_t) head_dim);

    for (int head = 0; head < heads; ++head) {
        const float *q = query + head * head_dim;
        const int kvColumn = (head / perKv) * head_dim;
        double largest = -INFINITY;

        for (int key = 0; key < key_count; ++key) {
            const int64_t k = (int64_t) key * kvWidth + kvColumn;
            double total = 0.0;
            for (int c = 0; c < head_dim; ++c)
                total += (double) q[c] * read(keys, k + c);
            weights[key] = (double) scale * total;
            if (weights[key] > largest)
                largest = weights[key];
        }

        double denominator = 0.0;
        for (int key = 0; key < key_count; ++key) {
            weights[key] = exp(weights[key] - largest);
            denominator += weights[key];
        }

        for (int c = 0; c < head_dim; ++c)
            acc[c] = 0.0;
        for (int key = 0; key < key_count; ++key) {
            const int64_t v = (int64_t) key * kvWidth + kvColumn;
            for (int c = 0; c < head_dim; ++c)
                acc[c] += weights[key] * read(values, v + c);
        }
        for (int c = 0; c < head_dim; ++c)
            out[head * head_dim + c] = (float) (acc[c] / denominator);
    }

    free(acc);
    free(weights);
}

/* Multi-query attention of one query row over key_count cached rows
 * (Lib/HuggingFaceEACP/Kernels/MultiQueryAttention.h:138-260 and
 * Tests/Decoder/ReferenceDecoder.h:208-272): query head h reads KV head
 * h / (heads / kv_heads); scores scale * q.k in double, softmax by the
 * maximum, the output the weighted value sum divided by the weight sum,
 * rounded to fp32 once.  Keys and values are fp16. */
void gor_mqa_row_f16(const float *query, const uint16_t *keys, const uint16_t *values,
                     int heads, int kv_heads, int head_dim, int key_count, float scale,
                     float *out)
{
    mqa_row(query, keys, values, read_half_cache, heads, kv_heads, head_dim, key_count, scale,
            out);
}

/* ======================================================================== */
/* The decoder.                                                              */
/* ======================================================================== */
int gor_tensor_count(const gor_shape *shape)
{
    return 2 + GOR_T_PER_LAYER * shape->layers;
}

static int is_final_norm(const gor_shape *shape, int index)
{
    return index == 1 + GOR_T_PER_LAYER * shape->layers;
}

int gor_tensor_is_norm(const gor_shape *shape, int index)
{
    if (index == 0)
        return 0;
    if (is_final_norm(shape, index))
        return 1;
    const int role = (index - 1) % GOR_T_PER_LAYER;
    return role == GOR_T_INPUT_NORM || role == GOR_T_POST_NORM;
}

int64_t gor_tensor_elements(const gor_shape *shape, int index)
{
    const int64_t width = shape->width;
    const int64_t queries = (int64_t) shape->heads * shape->head_dim;
    const int64_t kv = (int64_t) shape->kv_heads * shape->head_dim;
    const int64_t inter = shape->intermediate;

    if (index == 0)
        return (int64_t) shape->vocab * width;
    if (is_final_norm(shape, index))
        return width;

    switch ((index - 1) % GOR_T_PER_LAYER) {
    case GOR_T_Q: return queries * width;
    case GOR_T_K: return kv * width;
    case GOR_T_V: return kv * width;
    case GOR_T_O: return width * queries;
    case GOR_T_GATE: return inter * width;
    case GOR_T_UP: return inter * width;
    case GOR_T_DOWN: return width * inter;
    default: return width;
    }
}

uint64_t gor_tensor_seed(int index)
{
    return 0x5EED0000ULL + (uint64_t) index;
}

double gor_tensor_sigma(const gor_shape *shape, int index)
{
    return gor_tensor_is_norm(shape, index) ? 0.1 : 0.02;
}

static int64_t inner_of(const gor_shape *shape, int index)
{
    if (index == 0)
        return shape->width;
    switch ((index - 1) % GOR_T_PER_LAYER) {
    case GOR_T_O: return (int64_t) shape->heads * shape->head_dim;
    case GOR_T_DOWN: return shape->intermediate;
    default: return shape->width;
    }
}

typedef struct gor_layer_debug {
    float *normalised, *attended, *activated, *hidden;
    int8_t *normalisedQ, *attendedQ, *activatedQ, *hiddenQ;
    uint16_t *normalisedS, *attendedS, *activatedS, *hiddenS;
} gor_layer_debug;

struct gor_model {
    gor_shape shape;
    int mode;
    int position;
    int tensorCount;
    uint8_t **bytes;   /* Int8Blocks tensors (NULL for norms) */
    float **norms;     /* fp32 norm tensors (NULL for projections) */
    int *present;
    float *cosines, *sines;
    uint16_t *keyCache, *valueCache; /* Q8 mode: [layers][maxPos][kvWidth] fp16 */
    float *keyCacheF, *valueCacheF;  /* Q8-path-f32 mode */
    double *keyCacheD, *valueCacheD; /* reference mode */
    gor_layer_debug *debug;           /* layers + 1 entries (last: final norm) */
};

gor_model *gor_model_create(const gor_shape *shape, int mode)
{
    gor_model *model = (gor_model *) calloc(1, sizeof(gor_model));
    model->shape = *shape;
    model->mode = mode;
    model->tensorCount = gor_tensor_count(shape);
    model->bytes = (uint8_t **) calloc((size_t) model->tensorCount, sizeof(uint8_t *));
    model->norms = (float **) calloc((size_t) model->tensorCount, sizeof(float *));
    model->present = (int *) calloc((size_t) model->tensorCount, sizeof(int));

    const int half = shape->head_dim / 2;
    model->cosines = (float *) malloc(sizeof(float) * (size_t) shape->max_positions * (size_t) half);
    model->sines = (float *) malloc(sizeof(float) * (size_t) shape->max_positions * (size_t) half);
    gor_rotary_table(shape->max_positions, shape->head_dim, shape->rope_theta,
                     model->cosines, model->sines);

    const size_t cacheElements = (size_t) shape->layers * (size_t) shape->max_positions
                                 * (size_t) (shape->kv_heads * shape->head_dim);
    if (mode == GOR_MODE_Q8) {
        model->keyCache = (uint16_t *) calloc(cacheElements, sizeof(uint16_t));
        model->valueCache = (uint16_t *) calloc(cacheElements, sizeof(uint16_t));
    } else if (mode == GOR_MODE_Q8_PATH_F32) {
        model->keyCacheF = (float *) calloc(cacheElements, sizeof(float));
        model->valueCacheF = (float *) calloc(cacheElements, sizeof(float));
    } else {
        model->keyCacheD = (double *) calloc(cacheElements, sizeof(double));
        model->valueCacheD = (double *) calloc(cacheElements, sizeof(double));
    }

    const int qw = shape->heads * shape->head_dim;
    model->debug = (gor_layer_debug *) calloc((size_t) shape->layers + 1, sizeof(gor_layer_debug));
    for (int l = 0; l <= shape->layers; ++l) {
        gor_layer_debug *d = &model->debug[l];
        d->normalised = (float *) calloc((size_t) shape->width, sizeof(float));
        d->attended = (float *) calloc((size_t) qw, sizeof(float));
        d->activated = (float *) calloc((size_t) shape->intermediate, sizeof(float));
        d->hidden = (float *) calloc((size_t) shape->width, sizeof(float));
        d->normalisedQ = (int8_t *) calloc((size_t) shape->width, 1);
        d->attendedQ = (int8_t *) calloc((size_t) qw, 1);
        d->activatedQ = (int8_t *) calloc((size_t) shape->intermediate, 1);
        d->hiddenQ = (int8_t *) calloc((size_t) shape->width, 1);
        d->normalisedS = (uint16_t *) calloc((size_t) shape->width / GOR_BLOCK + 1, 2);
        d->attendedS = (uint16_t *) calloc((size_t) qw / GOR_BLOCK + 1, 2);
        d->activatedS = (uint16_t *) calloc((size_t) shape->intermediate / GOR_BLOCK + 1, 2);
        d->hiddenS = (uint16_t *) calloc((size_t) shape->width / GOR_BLOCK + 1, 2);
    }
    return model;
}

void gor_model_destroy(gor_model *model)
{
    if (!model)
        return;
    for (int i = 0; i < model->tensorCount; ++i) {
        free(model->bytes[i]);
        free(model->norms[i]);
    }
    for (int l = 0; l <= model->shape.layers; ++l) {
        gor_layer_debug *d = &model->debug[l];
        free(d->normalised); free(d->attended); free(d->activated); free(d->hidden);
        free(d->normalisedQ); free(d->attendedQ); free(d->activatedQ); free(d->hiddenQ);
        free(d->normalisedS); free(d->attendedS); free(d->activatedS); free(d->hiddenS);
    }
    free(model->debug);
    free(model->bytes);
    free(model->norms);
    free(model->present);
    free(model->cosines);
    free(model->sines);
    free(model->keyCache);
    free(model->valueCache);
    free(model->keyCacheF);
    free(model->valueCacheF);
    free(model->keyCacheD);
    free(model->valueCacheD);
    free(model);
}

int gor_model_set_tensor(gor_model *model, int index, const float *values)
{
    if (index < 0 || index >= model->tensorCount)
        return -1;

    const int64_t count = gor_tensor_elements(&model->shape, index);

    if (gor_tensor_is_norm(&model->shape, index)) {
        free(model->norms[index]);
        model->norms[index] = (float *) malloc(sizeof(float) * (size_t) count);
        memcpy(model->norms[index], values, sizeof(float) * (size_t) count);
    } else {
        /* TensorLoader.cpp:274-296 refuses a tensor the format cannot hold */
        if (!gor_quantizes_as_int8_blocks(inner_of(&model->shape, index), count))
            return -5;
        free(model->bytes[index]);
        model->bytes[index] = (uint8_t *) malloc((size_t) gor_int8_blocks_byte_count(count));
        const int64_t piece = (int64_t) GOR_CHUNK;
        const int64_t pieces = (count + piece - 1) / piece;
        uint8_t *destination = model->bytes[index];
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t p = 0; p < pieces; ++p) {
            const int64_t first = p * piece;
            const int64_t n = first + piece < count ? piece : count - first;
            gor_quantize_int8_blocks(values + first, n, first, count, destination);
        }
    }
    model->present[index] = 1;
    return 0;
}

int gor_model_fill_synthetic(gor_model *model)
{
    for (int index = 0; index < model->tensorCount; ++index) {
        const int64_t count = gor_tensor_elements(&model->shape, index);
        float *values = (float *) malloc(sizeof(float) * (size_t) count);
        gor_normal_fill(gor_tensor_seed(index), gor_tensor_sigma(&model->shape, index),
                        values, count);
        const int status = gor_model_set_tensor(model, index, values);
        free(values);
        if (status != 0)
            return status;
    }
    return 0;
}

const uint8_t *gor_model_tensor_bytes(const gor_model *model, int index)
{
    if (index < 0 || index >= model->tensorCount)
        return NULL;
    return model->bytes[index];
}

void gor_model_begin(gor_model *model)
{
    model->position = 0; /* Decoder.h:93-96: no reallocation, position reset */
}

int gor_model_position(const gor_model *model)
{
    return model->position;
}

const float *gor_model_debug(const gor_model *model, int which, int layer)
{
    if (layer < 0 || layer > model->shape.layers)
        return NULL;
    const gor_layer_debug *d = &model->debug[layer];
    switch (which) {
    case GOR_DBG_NORMALISED: return d->normalised;
    case GOR_DBG_ATTENDED: return d->attended;
    case GOR_DBG_ACTIVATED: return d->activated;
    default: return d->hidden;
    }
}

const int8_t *gor_model_debug_q(const gor_model *model, int which, int layer)
{
    if (layer < 0 || layer > model->shape.layers)
        return NULL;
    const gor_layer_debug *d = &model->debug[layer];
    switch (which) {
    case GOR_DBG_NORMALISED: return d->normalisedQ;
    case GOR_DBG_ATTENDED: return d->attendedQ;
    case GOR_DBG_ACTIVATED: return d->activatedQ;
    default: return d->hiddenQ;
    }
}

const uint16_t *gor_model_debug_s(const gor_model *model, int which, int layer)
{
    if (layer < 0 || layer > model->shape.layers)
        return NULL;
    const gor_layer_debug *d = &model->debug[layer];
    switch (which) {
    case GOR_DBG_NORMALISED: return d->normalisedS;
    case GOR_DBG_ATTENDED: return d->attendedS;
    case GOR_DBG_ACTIVATED: return d->activatedS;
    default: return d->hiddenS;
    }
}

static const uint8_t *layer_bytes(const gor_model *model, int layer, int role)
{
    return model->bytes[1 + GOR_T_PER_LAYER * layer + role];
}

static const float *layer_norm(const gor_model *model, int layer, int role)
{
    return model->norms[1 + GOR_T_PER_LAYER * layer + role];
}

/* ---- Q8 path: one token ------------------------------------------------ */
static double dequantized(const uint8_t *bytes, int64_t elements, int64_t index);

/* A product input row: quantized in the Q8 mode (kept for the debug view),
 * left as fp32 in the Q8-path-f32 mode. */
static void product_input(const gor_model *model, const float *x, int n, int8_t *xq,
                          uint16_t *xs)
{
    if (model->mode == GOR_MODE_Q8) {
        gor_quantize_row(x, n, xq, xs);
    } else {
        memset(xq, 0, (size_t) n);
        memset(xs, 0, sizeof(uint16_t) * (size_t) (n / GOR_BLOCK));
    }
}

/* The fp32 row against one dequantized weight row (Linear.h:128-357 with
 * the Int8Blocks read of WeightStorage.h:80-191), a block at a time: the
 * products x * q are exact in double, a block's 32 are summed in eight
 * partial sums (element k in sum k % 8, combined in a fixed tree), then
 * scaled by the block's fp16 scale and summed over the blocks in double.
 * Built for three instruction sets like q8_row_dot. */
__attribute__((target_clones("avx512f", "avx2", "default")))
static double f32_row_dot(const float *x, const uint8_t *weights, int64_t elements, int64_t inner,
                          int64_t row)
{
    const int64_t blocks = inner / GOR_BLOCK;
    const int8_t *q = (const int8_t *) weights + row * inner;
    const uint8_t *scales = weights + elements + 2 * row * blocks;
    double total = 0.0;
    for (int64_t b = 0; b < blocks; ++b) {
        const float *xb = x + b * GOR_BLOCK;
        const int8_t *qb = q + b * GOR_BLOCK;
        double p[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
        for (int k = 0; k < GOR_BLOCK; k += 8)
            for (int u = 0; u < 8; ++u)
                p[u] += (double) xb[k + u] * (double) qb[k + u];
        const double block = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
        const uint16_t bits = (uint16_t) (scales[2 * b] | ((uint32_t) scales[2 * b + 1] << 8));
        total += block * (double) g_half_table[bits];
    }
    return total;
}

static void product(const gor_model *model, const float *x, const int8_t *xq,
                    const uint16_t *xs, const uint8_t *weights, int64_t rows, int64_t inner,
                    double *out)
{
    if (model->mode == GOR_MODE_Q8) {
        q8_matvec_double(xq, xs, weights, rows, inner, out);
        return;
    }
    const int64_t elements = rows * inner;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        out[r] = f32_row_dot(x, weights, elements, inner, r);
}

static void q8_token(gor_model *model, int32_t token, float *logits, float *hiddenOut)
{
    const gor_shape *s = &model->shape;
    const int width = s->width;
    const int qw = s->heads * s->head_dim;
    const int kvw = s->kv_heads * s->head_dim;
    const int inter = s->intermediate;
    const int position = model->position;
    const int64_t embedElements = (int64_t) s->vocab * width;
    const int64_t maxCacheRow = (int64_t) s->max_positions * kvw;

    float *h = (float *) malloc(sizeof(float) * (size_t) width);
    float *n = (float *) malloc(sizeof(float) * (size_t) width);
    float *q = (float *) malloc(sizeof(float) * (size_t) qw);
    float *k = (float *) malloc(sizeof(float) * (size_t) kvw);
    float *v = (float *) malloc(sizeof(float) * (size_t) kvw);
    float *att = (float *) malloc(sizeof(float) * (size_t) qw);
    float *gate = (float *) malloc(sizeof(float) * (size_t) inter);
    float *up = (float *) malloc(sizeof(float) * (size_t) inter);
    float *act = (float *) malloc(sizeof(float) * (size_t) inter);
    int maxInner = inter > qw ? inter : qw;
    if (width > maxInner)
        maxInner = width;
    int8_t *xq = (int8_t *) malloc((size_t) maxInner);
    uint16_t *xs = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) (maxInner / GOR_BLOCK + 1));
    int64_t maxRows = s->vocab > inter ? s->vocab : inter;
    double *y = (double *) malloc(sizeof(double) * (size_t) maxRows);

    ensure_half_table();

    /* Embed.h:45-82 with Decoder.cpp:319-362: scale * dequantized row, fp32 */
    {
        const uint8_t *table = model->bytes[0];
        for (int c = 0; c < width; ++c) {
            const int64_t e = (int64_t) token * width + c;
            const int64_t at = embedElements + 2 * (e / GOR_BLOCK);
            const uint16_t bits = (uint16_t) (table[at] | ((uint32_t) table[at + 1] << 8));
            const float gathered = g_half_table[bits] * (float) (int8_t) table[e];
            h[c] = (float) ((double) s->embedding_scale * (double) gathered);
        }
    }

    for (int layer = 0; layer < s->layers; ++layer) {
        gor_layer_debug *dbg = &model->debug[layer];

        /* Decoder.cpp:579-642, encodeLayer: pre-norm attention sublayer */
        gor_rmsnorm_row(h, layer_norm(model, layer, GOR_T_INPUT_NORM), width,
                        s->rms_epsilon, n);
        product_input(model, n, width, xq, xs);
        memcpy(dbg->normalised, n, sizeof(float) * (size_t) width);
        memcpy(dbg->normalisedQ, xq, (size_t) width);
        memcpy(dbg->normalisedS, xs, sizeof(uint16_t) * (size_t) (width / GOR_BLOCK));

        product(model, n, xq, xs, layer_bytes(model, layer, GOR_T_Q), qw, width, y);
        for (int i = 0; i < qw; ++i) q[i] = (float) y[i];
        product(model, n, xq, xs, layer_bytes(model, layer, GOR_T_K), kvw, width, y);
        for (int i = 0; i < kvw; ++i) k[i] = (float) y[i];
        product(model, n, xq, xs, layer_bytes(model, layer, GOR_T_V), kvw, width, y);
        for (int i = 0; i < kvw; ++i) v[i] = (float) y[i];

        /* Decoder.cpp:541-546: rotate the queries and this step's key row */
        gor_rope_row(q, qw, s->heads, s->head_dim, position, model->cosines, model->sines);
        gor_rope_row(k, kvw, s->kv_heads, s->head_dim, position, model->cosines, model->sines);

        const float scale = 1.f / sqrtf((float) s->head_dim);
        if (model->mode == GOR_MODE_Q8) {
            uint16_t *keyRows = model->keyCache + (int64_t) layer * maxCacheRow;
            uint16_t *valueRows = model->valueCache + (int64_t) layer * maxCacheRow;
            for (int i = 0; i < kvw; ++i) {
                keyRows[(int64_t) position * kvw + i] = gor_half_from_float(k[i]);
                valueRows[(int64_t) position * kvw + i] = gor_half_from_float(v[i]);
            }
            /* Decoder.cpp:553-562: decode attention over position + 1 keys */
            mqa_row(q, keyRows, valueRows, read_half_cache, s->heads, s->kv_heads, s->head_dim,
                    position + 1, scale, att);
        } else {
            float *keyRows = model->keyCacheF + (int64_t) layer * maxCacheRow;
            float *valueRows = model->valueCacheF + (int64_t) layer * maxCacheRow;
            memcpy(keyRows + (int64_t) position * kvw, k, sizeof(float) * (size_t) kvw);
            memcpy(valueRows + (int64_t) position * kvw, v, sizeof(float) * (size_t) kvw);
            mqa_row(q, keyRows, valueRows, read_float_cache, s->heads, s->kv_heads,
                    s->head_dim, position + 1, scale, att);
        }
        product_input(model, att, qw, xq, xs);
        memcpy(dbg->attended, att, sizeof(float) * (size_t) qw);
        memcpy(dbg->attendedQ, xq, (size_t) qw);
        memcpy(dbg->attendedS, xs, sizeof(uint16_t) * (size_t) (qw / GOR_BLOCK));

        /* o_proj with the residual folded (Decoder.cpp:595-603) */
        product(model, att, xq, xs, layer_bytes(model, layer, GOR_T_O), width, qw, y);
        for (int i = 0; i < width; ++i)
            h[i] = (float) ((double) h[i] + y[i]);

        /* the feed-forward sublayer (Decoder.cpp:605-641) */
        gor_rmsnorm_row(h, layer_norm(model, layer, GOR_T_POST_NORM), width,
                        s->rms_epsilon, n);
        product_input(model, n, width, xq, xs);
        product(model, n, xq, xs, layer_bytes(model, layer, GOR_T_GATE), inter, width, y);
        for (int i = 0; i < inter; ++i) gate[i] = (float) y[i];
        product(model, n, xq, xs, layer_bytes(model, layer, GOR_T_UP), inter, width, y);
        for (int i = 0; i < inter; ++i) up[i] = (float) y[i];
        for (int i = 0; i < inter; ++i)
            act[i] = gor_geglu(gate[i], up[i]);
        product_input(model, act, inter, xq, xs);
        memcpy(dbg->activated, act, sizeof(float) * (size_t) inter);
        memcpy(dbg->activatedQ, xq, (size_t) inter);
        memcpy(dbg->activatedS, xs, sizeof(uint16_t) * (size_t) (inter / GOR_BLOCK));

        product(model, act, xq, xs, layer_bytes(model, layer, GOR_T_DOWN), width, inter, y);
        for (int i = 0; i < width; ++i)
            h[i] = (float) ((double) h[i] + y[i]);
        memcpy(dbg->hidden, h, sizeof(float) * (size_t) width);
    }

    /* final norm, then the tied lm_head (Decoder.cpp:681-703) */
    {
        gor_layer_debug *dbg = &model->debug[s->layers];
        gor_rmsnorm_row(h, model->norms[1 + GOR_T_PER_LAYER * s->layers], width,
                        s->rms_epsilon, n);
        product_input(model, n, width, xq, xs);
        memcpy(dbg->normalised, n, sizeof(float) * (size_t) width);
        memcpy(dbg->normalisedQ, xq, (size_t) width);
        memcpy(dbg->normalisedS, xs, sizeof(uint16_t) * (size_t) (width / GOR_BLOCK));
        if (hiddenOut)
            memcpy(hiddenOut, n, sizeof(float) * (size_t) width);
        if (logits) {
            product(model, n, xq, xs, model->bytes[0], s->vocab, width, y);
            for (int64_t i = 0; i < s->vocab; ++i)
                logits[i] = (float) y[i];
        }
    }

    free(h); free(n); free(q); free(k); free(v); free(att);
    free(gate); free(up); free(act); free(xq); free(xs); free(y);
}

/* ---- Q8 path: a block of tokens ------------------------------------------
 * The same arithmetic as q8_token for each row of the block, with the
 * products taken over all rows at once so each weight row is read once a
 * block (a prefill of hundreds of rows then costs a few token steps).  Every
 * element is computed by the same expressions in the same order as in
 * q8_token; only the order in which rows and outputs are visited differs, so
 * the results are bit-identical (tests/test_oracle_decoder.py holds them to
 * that).  The debug views keep the block's last row. */
static void q8_products(const int8_t *xq, const uint16_t *xs, int n, int64_t inner,
                        const uint8_t *weights, int64_t rows, double *out)
{
    ensure_half_table();
    const int64_t nb = inner / GOR_BLOCK;
    double *activationScales = (double *) malloc(sizeof(double) * (size_t) (n * nb));
    for (int64_t i = 0; i < (int64_t) n * nb; ++i)
        activationScales[i] = (double) g_half_table[xs[i]];
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < rows; ++row)
        for (int t = 0; t < n; ++t)
            out[(int64_t) t * rows + row] =
                q8_row_dot(xq + (int64_t) t * inner, activationScales + (int64_t) t * nb, weights,
                           rows, inner, row);
    free(activationScales);
}

static void q8_block(gor_model *model, const int32_t *tokens, int n, float *logits,
                     int logitsRows, float *hiddenOut)
{
    const gor_shape *s = &model->shape;
    const int width = s->width;
    const int qw = s->heads * s->head_dim;
    const int kvw = s->kv_heads * s->head_dim;
    const int inter = s->intermediate;
    const int position = model->position;
    const int64_t embedElements = (int64_t) s->vocab * width;
    const int64_t maxCacheRow = (int64_t) s->max_positions * kvw;
    int maxInner = inter > qw ? inter : qw;
    if (width > maxInner)
        maxInner = width;
    int64_t maxOut = inter > qw ? inter : qw;
    if (width > maxOut)
        maxOut = width;

    float *h = (float *) malloc(sizeof(float) * (size_t) n * width);
    float *nrm = (float *) malloc(sizeof(float) * (size_t) n * width);
    float *q = (float *) malloc(sizeof(float) * (size_t) n * qw);
    float *k = (float *) malloc(sizeof(float) * (size_t) n * kvw);
    float *v = (float *) malloc(sizeof(float) * (size_t) n * kvw);
    float *att = (float *) malloc(sizeof(float) * (size_t) n * qw);
    float *gate = (float *) malloc(sizeof(float) * (size_t) n * inter);
    float *up = (float *) malloc(sizeof(float) * (size_t) n * inter);
    float *act = (float *) malloc(sizeof(float) * (size_t) n * inter);
    int8_t *xq = (int8_t *) malloc((size_t) n * maxInner);
    uint16_t *xs = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) n * (maxInner / GOR_BLOCK + 1));
    double *y = (double *) malloc(sizeof(double) * (size_t) n * maxOut);

    ensure_half_table();
    for (int t = 0; t < n; ++t) {
        const uint8_t *table = model->bytes[0];
        for (int c = 0; c < width; ++c) {
            const int64_t e = (int64_t) tokens[t] * width + c;
            const int64_t at = embedElements + 2 * (e / GOR_BLOCK);
            const uint16_t bits = (uint16_t) (table[at] | ((uint32_t) table[at + 1] << 8));
            const float gathered = g_half_table[bits] * (float) (int8_t) table[e];
            h[(int64_t) t * width + c] = (float) ((double) s->embedding_scale * (double) gathered);
        }
    }

    /* the row's norm and its Q8 input, row by row */
#define ORACLE_NORM_ROWS(src, weight, len)                                                   \
    for (int t = 0; t < n; ++t) {                                                            \
        gor_rmsnorm_row((src) + (int64_t) t * width, (weight), width, s->rms_epsilon,       \
                        nrm + (int64_t) t * width);                                          \
        gor_quantize_row(nrm + (int64_t) t * width, width, xq + (int64_t) t * width,        \
                         xs + (int64_t) t * (width / GOR_BLOCK));                            \
    }

    for (int layer = 0; layer < s->layers; ++layer) {
        gor_layer_debug *dbg = &model->debug[layer];
        ORACLE_NORM_ROWS(h, layer_norm(model, layer, GOR_T_INPUT_NORM), width)
        memcpy(dbg->normalised, nrm + (int64_t) (n - 1) * width, sizeof(float) * (size_t) width);
        memcpy(dbg->normalisedQ, xq + (int64_t) (n - 1) * width, (size_t) width);
        memcpy(dbg->normalisedS, xs + (int64_t) (n - 1) * (width / GOR_BLOCK),
               sizeof(uint16_t) * (size_t) (width / GOR_BLOCK));

        q8_products(xq, xs, n, width, layer_bytes(model, layer, GOR_T_Q), qw, y);
        for (int64_t i = 0; i < (int64_t) n * qw; ++i) q[i] = (float) y[i];
        q8_products(xq, xs, n, width, layer_bytes(model, layer, GOR_T_K), kvw, y);
        for (int64_t i = 0; i < (int64_t) n * kvw; ++i) k[i] = (float) y[i];
        q8_products(xq, xs, n, width, layer_bytes(model, layer, GOR_T_V), kvw, y);
        for (int64_t i = 0; i < (int64_t) n * kvw; ++i) v[i] = (float) y[i];

        uint16_t *keyRows = model->keyCache + (int64_t) layer * maxCacheRow;
        uint16_t *valueRows = model->valueCache + (int64_t) layer * maxCacheRow;
        for (int t = 0; t < n; ++t) {
            gor_rope_row(q + (int64_t) t * qw, qw, s->heads, s->head_dim, position + t,
                         model->cosines, model->sines);
            gor_rope_row(k + (int64_t) t * kvw, kvw, s->kv_heads, s->head_dim, position + t,
                         model->cosines, model->sines);
            for (int i = 0; i < kvw; ++i) {
                keyRows[(int64_t) (position + t) * kvw + i] = gor_half_from_float(k[(int64_t) t * kvw + i]);
                valueRows[(int64_t) (position + t) * kvw + i] = gor_half_from_float(v[(int64_t) t * kvw + i]);
            }
        }
        const float scale = 1.f / sqrtf((float) s->head_dim);
#pragma omp parallel for schedule(dynamic, 1)
        for (int t = 0; t < n; ++t)
            mqa_row(q + (int64_t) t * qw, keyRows, valueRows, read_half_cache, s->heads,
                    s->kv_heads, s->head_dim, position + t + 1, scale, att + (int64_t) t * qw);
        for (int t = 0; t < n; ++t)
            gor_quantize_row(att + (int64_t) t * qw, qw, xq + (int64_t) t * qw,
                             xs + (int64_t) t * (qw / GOR_BLOCK));
        memcpy(dbg->attended, att + (int64_t) (n - 1) * qw, sizeof(float) * (size_t) qw);
        memcpy(dbg->attendedQ, xq + (int64_t) (n - 1) * qw, (size_t) qw);
        memcpy(dbg->attendedS, xs + (int64_t) (n - 1) * (qw / GOR_BLOCK),
               sizeof(uint16_t) * (size_t) (qw / GOR_BLOCK));

        q8_products(xq, xs, n, qw, layer_bytes(model, layer, GOR_T_O), width, y);
        for (int64_t i = 0; i < (int64_t) n * width; ++i)
            h[i] = (float) ((double) h[i] + y[i]);

        ORACLE_NORM_ROWS(h, layer_norm(model, layer, GOR_T_POST_NORM), width)
        q8_products(xq, xs, n, width, layer_bytes(model, layer, GOR_T_GATE), inter, y);
        for (int64_t i = 0; i < (int64_t) n * inter; ++i) gate[i] = (float) y[i];
        q8_products(xq, xs, n, width, layer_bytes(model, layer, GOR_T_UP), inter, y);
        for (int64_t i = 0; i < (int64_t) n * inter; ++i) up[i] = (float) y[i];
        for (int64_t i = 0; i < (int64_t) n * inter; ++i)
            act[i] = gor_geglu(gate[i], up[i]);
        for (int t = 0; t < n; ++t)
            gor_quantize_row(act + (int64_t) t * inter, inter, xq + (int64_t) t * inter,
                             xs + (int64_t) t * (inter / GOR_BLOCK));
        memcpy(dbg->activated, act + (int64_t) (n - 1) * inter, sizeof(float) * (size_t) inter);
        memcpy(dbg->activatedQ, xq + (int64_t) (n - 1) * inter, (size_t) inter);
        memcpy(dbg->activatedS, xs + (int64_t) (n - 1) * (inter / GOR_BLOCK),
               sizeof(uint16_t) * (size_t) (inter / GOR_BLOCK));

        q8_products(xq, xs, n, inter, layer_bytes(model, layer, GOR_T_DOWN), width, y);
        for (int64_t i = 0; i < (int64_t) n * width; ++i)
            h[i] = (float) ((double) h[i] + y[i]);
        memcpy(dbg->hidden, h + (int64_t) (n - 1) * width, sizeof(float) * (size_t) width);
    }

    {
        gor_layer_debug *dbg = &model->debug[s->layers];
        ORACLE_NORM_ROWS(h, model->norms[1 + GOR_T_PER_LAYER * s->layers], width)
        memcpy(dbg->normalised, nrm + (int64_t) (n - 1) * width, sizeof(float) * (size_t) width);
        memcpy(dbg->normalisedQ, xq + (int64_t) (n - 1) * width, (size_t) width);
        memcpy(dbg->normalisedS, xs + (int64_t) (n - 1) * (width / GOR_BLOCK),
               sizeof(uint16_t) * (size_t) (width / GOR_BLOCK));
        if (hiddenOut)
            memcpy(hiddenOut, nrm, sizeof(float) * (size_t) n * width);
        if (logits && logitsRows > 0) {
            const int first = n - logitsRows;
            double *row = (double *) malloc(sizeof(double) * (size_t) s->vocab);
            for (int t = first; t < n; ++t) {
                q8_matvec_double(xq + (int64_t) t * width, xs + (int64_t) t * (width / GOR_BLOCK),
                                 model->bytes[0], s->vocab, width, row);
                for (int64_t i = 0; i < s->vocab; ++i)
                    logits[(int64_t) (t - first) * s->vocab + i] = (float) row[i];
            }
            free(row);
        }
    }
#undef ORACLE_NORM_ROWS
    model->position = position + n;

    free(h); free(nrm); free(q); free(k); free(v); free(att);
    free(gate); free(up); free(act); free(xq); free(xs); free(y);
}

/* The block step of the Q8 path (q8_block) in blocks of at most 256 rows:
 * logits for the last logitsRows rows (0: none). */
int gor_model_step_block(gor_model *model, const int32_t *tokens, int n, float *logits,
                         int logitsRows)
{
    for (int i = 0; i < model->tensorCount; ++i)
        if (!model->present[i])
            return -4;
    if (n <= 0 || logitsRows < 0 || logitsRows > n)
        return -1;
    if (model->position + n > model->shape.max_positions)
        return -2;
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= model->shape.vocab)
            return -3;
    if (model->mode != GOR_MODE_Q8)
        return -1;
    const int chunk = 256;
    for (int start = 0; start < n; start += chunk) {
        const int rows = n - start < chunk ? n - start : chunk;
        /* the logits rows that fall in this chunk */
        const int firstLogit = n - logitsRows;
        const int from = firstLogit > start ? firstLogit : start;
        const int want = start + rows > from ? start + rows - from : 0;
        q8_block(model, tokens + start, rows, want ? logits + (int64_t) (from - firstLogit) * model->shape.vocab : NULL,
                 want, NULL);
    }
    return 0;
}

/* ---- reference path: one token, ReferenceDecoder.h:294-375 in double, ---- */
/* ---- cached (prompt == successive single steps, DecoderTests.cpp:116-147) */
static double dequantized(const uint8_t *bytes, int64_t elements, int64_t index)
{
    const int64_t at = elements + 2 * (index / GOR_BLOCK);
    const uint16_t bits = (uint16_t) (bytes[at] | ((uint32_t) bytes[at + 1] << 8));
    return (double) (g_half_table[bits] * (float) (int8_t) bytes[index]);
}

static void reference_linear(const double *x, const uint8_t *bytes, int64_t rows,
                             int64_t inner, double *out)
{
    const int64_t elements = rows * inner;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        double total = 0.0;
        for (int64_t i = 0; i < inner; ++i)
            total += x[i] * dequantized(bytes, elements, r * inner + i);
        out[r] = total;
    }
}

static void reference_norm(const double *x, const float *weight, int n, double epsilon,
                           double *out)
{
    double squares = 0.0;
    for (int i = 0; i < n; ++i)
        squares += x[i] * x[i];
    const double scale = 1.0 / sqrt(squares / n + epsilon);
    for (int i = 0; i < n; ++i)
        out[i] = x[i] * scale * (1.0 + weight[i]);
}

static void reference_rotate(double *x, int heads, int head_dim, int position,
                             double theta)
{
    const int half = head_dim / 2;
    for (int head = 0; head < heads; ++head) {
        for (int pair = 0; pair < half; ++pair) {
            const double exponent = 2.0 * pair / (double) head_dim;
            const double angle = (double) position / pow(theta, exponent);
            const double c = cos(angle), sn = sin(angle);
            double *lo = x + head * head_dim + pair;
            double *hi = lo + half;
            const double a = *lo, b = *hi;
            *lo = a * c - b * sn;
            *hi = b * c + a * sn;
        }
    }
}

static void reference_token(gor_model *model, int32_t token, float *logits, float *hiddenOut)
{
    const gor_shape *s = &model->shape;
    const int width = s->width, qw = s->heads * s->head_dim, kvw = s->kv_heads * s->head_dim;
    const int inter = s->intermediate, position = model->position;
    const int64_t maxCacheRow = (int64_t) s->max_positions * kvw;
    const int perKv = s->heads / s->kv_heads;
    const double scale = 1.0 / sqrt((double) s->head_dim);

    double *h = (double *) malloc(sizeof(double) * (size_t) width);
    double *n = (double *) malloc(sizeof(double) * (size_t) width);
    double *q = (double *) malloc(sizeof(double) * (size_t) qw);
    double *k = (double *) malloc(sizeof(double) * (size_t) kvw);
    double *v = (double *) malloc(sizeof(double) * (size_t) kvw);
    double *att = (double *) malloc(sizeof(double) * (size_t) qw);
    double *gate = (double *) malloc(sizeof(double) * (size_t) inter);
    double *up = (double *) malloc(sizeof(double) * (size_t) inter);
    double *out = (double *) malloc(sizeof(double) * (size_t) (s->vocab > inter ? s->vocab : inter));
    double *w = (double *) malloc(sizeof(double) * (size_t) (position + 1));

    ensure_half_table();
    const int64_t embedElements = (int64_t) s->vocab * width;
    for (int c = 0; c < width; ++c)
        h[c] = (double) s->embedding_scale
               * dequantized(model->bytes[0], embedElements, (int64_t) token * width + c);

    for (int layer = 0; layer < s->layers; ++layer) {
        reference_norm(h, layer_norm(model, layer, GOR_T_INPUT_NORM), width,
                       (double) s->rms_epsilon, n);
        reference_linear(n, layer_bytes(model, layer, GOR_T_Q), qw, width, q);
        reference_linear(n, layer_bytes(model, layer, GOR_T_K), kvw, width, k);
        reference_linear(n, layer_bytes(model, layer, GOR_T_V), kvw, width, v);
        reference_rotate(q, s->heads, s->head_dim, position, s->rope_theta);
        reference_rotate(k, s->kv_heads, s->head_dim, position, s->rope_theta);

        double *keys = model->keyCacheD + (int64_t) layer * maxCacheRow;
        double *values = model->valueCacheD + (int64_t) layer * maxCacheRow;
        memcpy(keys + (int64_t) position * kvw, k, sizeof(double) * (size_t) kvw);
        memcpy(values + (int64_t) position * kvw, v, sizeof(double) * (size_t) kvw);

        for (int head = 0; head < s->heads; ++head) {
            const int qc = head * s->head_dim, kc = (head / perKv) * s->head_dim;
            double largest = -INFINITY;
            for (int j = 0; j <= position; ++j) {
                double total = 0.0;
                for (int c = 0; c < s->head_dim; ++c)
                    total += q[qc + c] * keys[(int64_t) j * kvw + kc + c];
                w[j] = scale * total;
                if (w[j] > largest)
                    largest = w[j];
            }
            double denominator = 0.0;
            for (int j = 0; j <= position; ++j) {
                w[j] = exp(w[j] - largest);
                denominator += w[j];
            }
            for (int c = 0; c < s->head_dim; ++c) {
                double weighted = 0.0;
                for (int j = 0; j <= position; ++j)
                    weighted += w[j] * values[(int64_t) j * kvw + kc + c];
                att[qc + c] = weighted / denominator;
            }
        }

        reference_linear(att, layer_bytes(model, layer, GOR_T_O), width, qw, out);
        for (int i = 0; i < width; ++i) h[i] += out[i];

        reference_norm(h, layer_norm(model, layer, GOR_T_POST_NORM), width,
                       (double) s->rms_epsilon, n);
        reference_linear(n, layer_bytes(model, layer, GOR_T_GATE), inter, width, gate);
        reference_linear(n, layer_bytes(model, layer, GOR_T_UP), inter, width, up);
        for (int i = 0; i < inter; ++i)
            gate[i] = gor_tanh_gelu(gate[i]) * up[i];
        reference_linear(gate, layer_bytes(model, layer, GOR_T_DOWN), width, inter, out);
        for (int i = 0; i < width; ++i) h[i] += out[i];
        for (int i = 0; i < width; ++i) model->debug[layer].hidden[i] = (float) h[i];
    }

    reference_norm(h, model->norms[1 + GOR_T_PER_LAYER * s->layers], width,
                   (double) s->rms_epsilon, n);
    if (hiddenOut)
        for (int i = 0; i < width; ++i) hiddenOut[i] = (float) n[i];
    if (logits) {
        reference_linear(n, model->bytes[0], s->vocab, width, out);
        for (int64_t i = 0; i < s->vocab; ++i) logits[i] = (float) out[i];
    }

    free(h); free(n); free(q); free(k); free(v); free(att);
    free(gate); free(up); free(out); free(w);
}

/* Decoder::step, Decoder.cpp:644-706: every refusal is raised before anything
 * is computed, so a refused step leaves the position and outputs untouched. */
int gor_model_step(gor_model *model, const int32_t *tokens, int n, float *logits,
                   float *hidden)
{
    for (int i = 0; i < model->tensorCount; ++i)
        if (!model->present[i])
            return -4;
    if (n <= 0)
        return -1;
    if (model->position + n > model->shape.max_positions)
        return -2;
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= model->shape.vocab)
            return -3;

    for (int i = 0; i < n; ++i) {
        float *rowLogits = logits ? logits + (int64_t) i * model->shape.vocab : NULL;
        float *rowHidden = hidden ? hidden + (int64_t) i * model->shape.width : NULL;
        if (model->mode != GOR_MODE_REFERENCE)
            q8_token(model, tokens[i], rowLogits, rowHidden);
        else
            reference_token(model, tokens[i], rowLogits, rowHidden);
        model->position += 1;
    }
    return 0;
}

static float top_two_gap(const float *logits, int n, int best)
{
    float second = -INFINITY;
    for (int i = 0; i < n; ++i)
        if (i != best && logits[i] > second)
            second = logits[i];
    return logits[best] - second;
}

/* Gemma::generate / prefill / generateGreedily (Gemma.cpp:350-543). */
int gor_generate(gor_model *model, const int32_t *prompt, int prompt_length,
                 int max_tokens, int eos, int32_t *out, float *out_margins)
{
    const gor_shape *s = &model->shape;

    if (prompt_length <= 0)
        return -1;
    if (prompt_length > s->max_positions)
        return -2;
    for (int i = 0; i < prompt_length; ++i)
        if (prompt[i] < 0 || prompt[i] >= s->vocab)
            return -3;

    gor_model_begin(model);

    const int window = s->max_positions - prompt_length;
    const int limit = max_tokens > 0 ? (max_tokens < window ? max_tokens : window) : window;

    float *logits = (float *) malloc(sizeof(float) * (size_t) s->vocab);
    int status = 0;

    /* the prefill: only its last row's logits are sampled (Gemma.cpp:306-318) */
    if (prompt_length > 1)
        status = gor_model_step(model, prompt, prompt_length - 1, NULL, NULL);
    if (status == 0)
        status = gor_model_step(model, prompt + prompt_length - 1, 1, logits, NULL);
    if (status != 0) {
        free(logits);
        return status;
    }
    if (limit <= 0) {
        free(logits);
        return 0;
    }

    int count = 0;
    int token = gor_argmax(logits, NULL, s->vocab);
    float margin = top_two_gap(logits, s->vocab, token);

    for (int step = 0; step < limit; ++step) {
        if (eos >= 0 && token == eos)
            break;
        out[count] = token;
        if (out_margins)
            out_margins[count] = margin;
        ++count;
        if (step + 1 >= limit)
            break;
        status = gor_model_step(model, &token, 1, logits, NULL);
        if (status != 0)
            break;
        token = gor_argmax(logits, NULL, s->vocab);
        margin = top_two_gap(logits, s->vocab, token);
    }

    free(logits);
    return status != 0 ? status : count;
}
