// gq8_sample.hip -- one token drawn from one row of logits on the device:
// Sampler::sample (Sampler.cpp:78-213) in place of the reference's logits
// readback (Gemma.cpp:545-595).
//
// Candidates are the unmasked tokens, scored logit * (1 / temperature) in
// double.  With top-k or top-p they are ranked (score descending, token
// ascending) by a stable LSD radix sort of a 64-bit order key over the
// token-ordered row: eight passes of an 8-bit digit, each a histogram, a scan
// and a scatter that places every element by its rank among equal digits
// (wave ballots, then wave and round prefixes in LDS), so ties keep token
// order exactly as the reference's comparison does.  One workgroup then
// walks the ranked candidates (or the row in token order when no cut is set,
// as the reference's draw does): the softmax over the survivors, the top-p
// prefix whose running mass reaches p (boundary kept), and the first
// candidate whose running mass passes the draw.  Running sums go a contiguous
// chunk a thread and then chunk by chunk in order, so only the rounding of
// the sums differs from the reference's sequential loop.  The uniform draws
// come from the caller (the top 53 bits of std::mt19937_64 outputs).
#include "gq8_device.hpp"
#include "gq8_kernels.hpp"
#include "gq8_numerics.hpp"

#include <cfloat>
#include <climits>

namespace gq8 {
namespace {

constexpr int kSortThreads = 256;
constexpr int kSortRounds = 8;                          // elements a thread a tile
constexpr int kSortTile = kSortThreads * kSortRounds;   // 2048
constexpr int kDrawThreads = 1024;
constexpr uint64_t kMaskedKey = ~0ull;

struct SampleWorkspace {
    uint64_t *keys[2];
    uint32_t *tokens[2];
    int *hist; // [256][tiles]
    int tiles;
};

int sort_tiles(int vocab)
{
    return (vocab + kSortTile - 1) / kSortTile;
}

size_t align256(size_t n)
{
    return (n + 255) & ~size_t(255);
}

// Scores: +0 for a zero (the reference compares scores by value, so -0 and +0
// tie), the order key descending in score.
__device__ inline double candidate_score(float logit, double inverse)
{
    const double s = (double) logit * inverse;
    return s == 0.0 ? 0.0 : s;
}

__device__ inline uint64_t descending_key(double s)
{
    uint64_t u = (uint64_t) __double_as_longlong(s);
    u = (u >> 63) ? ~u : (u | (1ull << 63));
    return ~u;
}

__device__ inline double score_of_key(uint64_t key)
{
    uint64_t u = ~key;
    u = (u >> 63) ? (u & ~(1ull << 63)) : ~u;
    return __longlong_as_double((long long) u);
}

__global__ __launch_bounds__(kSortThreads) void sample_keys_kernel(SampleArgs a, uint64_t *keys,
                                                                   uint32_t *tokens)
{
    const double inverse = 1.0 / (double) a.temperature;
    for (int r = 0; r < kSortRounds; ++r) {
        const int e = blockIdx.x * kSortTile + r * kSortThreads + threadIdx.x;
        if (e >= a.vocab)
            break;
        const bool masked = a.mask && a.mask[e] != 0.f;
        keys[e] = masked ? kMaskedKey : descending_key(candidate_score(a.logits[e], inverse));
        tokens[e] = (uint32_t) e;
    }
}

__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const uint64_t *keys, int n,
                                                                  int shift, int *hist, int tiles)
{
    __shared__ int counts[256];
    counts[threadIdx.x] = 0;
    __syncthreads();
    for (int r = 0; r < kSortRounds; ++r) {
        const int e = blockIdx.x * kSortTile + r * kSortThreads + threadIdx.x;
        if (e < n)
            atomicAdd(&counts[(keys[e] >> shift) & 255], 1);
    }
    __syncthreads();
    hist[threadIdx.x * tiles + blockIdx.x] = counts[threadIdx.x];
}

// Exclusive scan of the digit-major histogram: offset of (digit, tile).
__global__ __launch_bounds__(kDrawThreads) void radix_scan_kernel(int *hist, int total)
{
    __shared__ int sums[kDrawThreads];
    const int t = threadIdx.x;
    const int chunk = (total + kDrawThreads - 1) / kDrawThreads;
    const int b = min(t * chunk, total), e = min(b + chunk, total);
    int s = 0;
    for (int i = b; i < e; ++i)
        s += hist[i];
    sums[t] = s;
    __syncthreads();
    if (t == 0) {
        int running = 0;
        for (int i = 0; i < kDrawThreads; ++i) {
            const int v = sums[i];
            sums[i] = running;
            running += v;
        }
    }
    __syncthreads();
    int running = sums[t];
    for (int i = b; i < e; ++i) {
        const int v = hist[i];
        hist[i] = running;
        running += v;
    }
}

// Stable scatter: an element's place is its digit's offset for the tile,
// plus the digit's count in earlier rounds of the tile, earlier waves of the
// round, and earlier lanes of the wave (ballots over the digit's bits).
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint64_t *keysIn, const uint32_t *tokensIn, uint64_t *keysOut, uint32_t *tokensOut, int n,
    int shift, const int *offsets, int tiles)
{
    constexpr int kWaves = kSortThreads / 64;
    __shared__ int running[256], base[256];
    __shared__ int waveCount[kWaves][256], wavePrefix[kWaves][256];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    running[t] = 0;
    const uint64_t below = (1ull << lane) - 1;
    for (int r = 0; r < kSortRounds; ++r) {
        const int e = blockIdx.x * kSortTile + r * kSortThreads + t;
        const bool valid = e < n;
        const uint64_t key = valid ? keysIn[e] : 0;
        const uint32_t token = valid ? tokensIn[e] : 0;
        const int d = (int) ((key >> shift) & 255);
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t m = __ballot((d >> b) & 1);
            peers &= ((d >> b) & 1) ? m : ~m;
        }
        const int rank = __popcll(peers & below);
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
            waveCount[w][t] = 0;
        __syncthreads();
        if (valid && (peers >> lane) == 1ull) // the last lane of its digit's peers
            waveCount[wave][d] = __popcll(peers);
        __syncthreads();
        {
            int s = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                wavePrefix[w][t] = s;
                s += waveCount[w][t];
            }
            base[t] = running[t];
            running[t] += s;
        }
        __syncthreads();
        if (valid) {
            const int at = offsets[d * tiles + blockIdx.x] + base[d] + wavePrefix[wave][d] + rank;
            keysOut[at] = key;
            tokensOut[at] = token;
        }
        __syncthreads();
    }
}

// The first i in [0, count) (in order) whose running sum of value(i) makes
// crosses(sum) true, or -1.  Each thread sums a contiguous chunk, the chunk
// sums are scanned in order, and each thread then walks its own chunk from
// its prefix; the smallest index found wins.  crosses is monotone and the
// values are not negative, so this is the sequential walk up to the rounding
// of the sums.  All threads of the workgroup call it.
template <typename Value, typename Crosses>
__device__ int first_crossing(int count, Value value, Crosses crosses, double *sums, int *first)
{
    const int t = threadIdx.x;
    const int chunk = (count + kDrawThreads - 1) / kDrawThreads;
    const int b = min(t * chunk, count), e = min(b + chunk, count);
    double s = 0.0;
    for (int i = b; i < e; ++i)
        s += value(i);
    sums[t] = s;
    if (t == 0)
        *first = INT_MAX;
    __syncthreads();
    if (t == 0) {
        double running = 0.0;
        for (int i = 0; i < kDrawThreads; ++i) {
            const double v = sums[i];
            sums[i] = running;
            running += v;
        }
    }
    __syncthreads();
    double m = sums[t];
    for (int i = b; i < e; ++i) {
        const double v = value(i);
        m += v;
        if (v > 0.0 && crosses(m)) { // a zero term never makes the first crossing
            atomicMin(first, i);
            break;
        }
    }
    __syncthreads();
    const int found = *first;
    __syncthreads(); // sums and first are reused by the next call
    return found == INT_MAX ? -1 : found;
}

// The sum of value(i) over [0, count): chunk sums added in chunk order, the
// same total in every thread.
template <typename Value>
__device__ double ordered_total(int count, Value value, double *sums)
{
    const int t = threadIdx.x;
    const int chunk = (count + kDrawThreads - 1) / kDrawThreads;
    const int b = min(t * chunk, count), e = min(b + chunk, count);
    double s = 0.0;
    for (int i = b; i < e; ++i)
        s += value(i);
    sums[t] = s;
    __syncthreads();
    double total = 0.0;
    for (int i = 0; i < kDrawThreads; ++i)
        total += sums[i];
    __syncthreads();
    return total;
}

// Sampler::sample after the scores (Sampler.cpp:101-205).  `ranked`: the keys
// and tokens hold the row sorted by rank (masked tokens last).
__global__ __launch_bounds__(kDrawThreads) void sample_draw_kernel(SampleArgs a, const uint64_t *keys,
                                                                   const uint32_t *tokens, int ranked)
{
    __shared__ double sums[kDrawThreads];
    __shared__ double sLargest;
    __shared__ int sCount, sFirst, sLast;
    const int t = threadIdx.x, V = a.vocab;
    const double u = a.draws[min(*a.draw_index, a.draw_count - 1)];
    const double inverse = 1.0 / (double) a.temperature;
    auto masked = [&](int i) { return a.mask && a.mask[i] != 0.f; };

    if (t == 0) {
        sCount = 0;
        sLast = -1;
    }
    __syncthreads();
    double largest = -DBL_MAX;
    int count = 0, last = -1;
    for (int i = t; i < V; i += kDrawThreads)
        if (!masked(i)) {
            largest = fmax(largest, candidate_score(a.logits[i], inverse));
            ++count;
            last = i;
        }
    largest = wave_max_d(largest);
    if ((t & 63) == 0)
        sums[t >> 6] = largest;
    atomicAdd(&sCount, count);
    atomicMax(&sLast, last);
    __syncthreads();
    if (t == 0) {
        double m = -DBL_MAX;
        for (int w = 0; w < kDrawThreads / 64; ++w)
            m = fmax(m, sums[w]);
        sLargest = m;
    }
    __syncthreads();
    const int n = sCount;
    const double top = sLargest;
    uint32_t chosen = 0;
    if (n > 0 && (!ranked || !((a.top_k > 0 && a.top_k < n) || a.top_p < 1.f))) {
        // no cut: every unmasked token in token order
        auto weight = [&](int i) -> double {
            return masked(i) ? 0.0 : exp(candidate_score(a.logits[i], inverse) - top);
        };
        const double total = ordered_total(V, weight, sums);
        const int at = first_crossing(
            V, [&](int i) { return weight(i) / total; }, [&](double m) { return u < m; }, sums,
            &sFirst);
        chosen = (uint32_t) (at >= 0 ? at : sLast);
    } else if (n > 0) {
        // the ranked candidates: the top k, then the top-p prefix
        int kept = (a.top_k > 0 && a.top_k < n) ? a.top_k : n;
        auto weight = [&](int i) { return exp(score_of_key(keys[i]) - top); };
        if (a.top_p < 1.f) {
            const double total = ordered_total(kept, weight, sums);
            const double wanted = (double) a.top_p;
            const int at = first_crossing(
                kept, [&](int i) { return weight(i) / total; },
                [&](double m) { return !(m < wanted); }, sums, &sFirst);
            kept = at >= 0 ? at + 1 : kept;
        }
        const double total = ordered_total(kept, weight, sums);
        const int at = first_crossing(
            kept, [&](int i) { return weight(i) / total; }, [&](double m) { return u < m; }, sums,
            &sFirst);
        chosen = tokens[at >= 0 ? at : kept - 1];
    }
    if (t == 0) {
        if (a.sequence)
            a.sequence[*a.position + a.offset] = chosen;
        if (a.token_out)
            *a.token_out = chosen;
        *a.draw_index += 1;
    }
}

SampleWorkspace carve(void *workspace, int vocab)
{
    SampleWorkspace w{};
    w.tiles = sort_tiles(vocab);
    uint8_t *p = static_cast<uint8_t *>(workspace);
    for (int i = 0; i < 2; ++i) {
        w.keys[i] = reinterpret_cast<uint64_t *>(p);
        p += align256((size_t) vocab * 8);
        w.tokens[i] = reinterpret_cast<uint32_t *>(p);
        p += align256((size_t) vocab * 4);
    }
    w.hist = reinterpret_cast<int *>(p);
    return w;
}

} // namespace

size_t sample_workspace_bytes(int vocab)
{
    if (vocab <= 0)
        return 0;
    return 2 * (align256((size_t) vocab * 8) + align256((size_t) vocab * 4))
           + align256((size_t) 256 * sort_tiles(vocab) * 4);
}

bool sampling_options_valid(float temperature, int top_k, float top_p)
{
    // Sampler.cpp:28-41, spelled so that a NaN is refused
    return temperature >= 0.f && top_k >= 0 && top_p > 0.f && top_p <= 1.f;
}

hipError_t launch_sample(const SampleArgs &a, void *workspace, size_t workspace_bytes,
                         hipStream_t stream)
{
    if (!a.logits || a.vocab <= 0 || !a.draws || a.draw_count <= 0 || !a.draw_index
        || !(a.temperature > 0.f)
        || !sampling_options_valid(a.temperature, a.top_k, a.top_p)
        || (!a.sequence && !a.token_out) || (a.sequence && !a.position) || !workspace
        || workspace_bytes < sample_workspace_bytes(a.vocab))
        return hipErrorInvalidValue;
    const SampleWorkspace w = carve(workspace, a.vocab);
    const bool ranked = a.top_k > 0 || a.top_p < 1.f;
    if (ranked) {
        hipLaunchKernelGGL(sample_keys_kernel, dim3(w.tiles), dim3(kSortThreads), 0, stream, a,
                           w.keys[0], w.tokens[0]);
        for (int pass = 0; pass < 8; ++pass) {
            const int in = pass & 1, shift = 8 * pass;
            hipLaunchKernelGGL(radix_hist_kernel, dim3(w.tiles), dim3(kSortThreads), 0, stream,
                               w.keys[in], a.vocab, shift, w.hist, w.tiles);
            hipLaunchKernelGGL(radix_scan_kernel, dim3(1), dim3(kDrawThreads), 0, stream, w.hist,
                               256 * w.tiles);
            hipLaunchKernelGGL(radix_scatter_kernel, dim3(w.tiles), dim3(kSortThreads), 0, stream,
                               w.keys[in], w.tokens[in], w.keys[in ^ 1], w.tokens[in ^ 1], a.vocab,
                               shift, w.hist, w.tiles);
        }
    }
    // eight passes leave the ranked row back in buffer 0
    hipLaunchKernelGGL(sample_draw_kernel, dim3(1), dim3(kDrawThreads), 0, stream, a, w.keys[0],
                       w.tokens[0], ranked ? 1 : 0);
    return hipGetLastError();
}

} // namespace gq8
