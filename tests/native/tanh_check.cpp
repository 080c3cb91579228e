// Host check of gq8_tanh.hpp's tanh_from_exp against libm's tanh: the ulp
// distance over [-10, 10] and the fp32 GeGLU outputs built on each.
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <cstdlib>
#include <random>
#include "gq8_tanh.hpp"
static int64_t ulp(double a, double b) {
    int64_t ia, ib; memcpy(&ia, &a, 8); memcpy(&ib, &b, 8);
    if (ia < 0) ia = INT64_MIN - ia; if (ib < 0) ib = INT64_MIN - ib;
    return ia > ib ? ia - ib : ib - ia;
}
static float geglu(double t, float g, float u) { return (float) (0.5 * g * (1.0 + t) * (double) u); }
int main(int argc, char **argv) {
    const int samples = argc > 1 ? atoi(argv[1]) : 2000000;
    std::mt19937_64 rng(7);
    std::uniform_real_distribution<double> U(-10.0, 10.0);
    std::normal_distribution<double> N(0.0, 1.0);
    int64_t hist[6] = {0}; int64_t worst = 0; double worstX = 0;
    for (int i = 0; i < samples; ++i) {
        const double x = (i & 1) ? U(rng) : N(rng) * 0.5;
        const int64_t d = ulp(gq8::tanh_from_exp(x), std::tanh(x));
        hist[d < 5 ? d : 5]++;
        if (d > worst) { worst = d; worstX = x; }
    }
    printf("ulp distance histogram 0..4,>=5:");
    for (int k = 0; k < 6; ++k) printf(" %lld", (long long) hist[k]);
    printf("\nworst %lld ulp at x = %.17g\n", (long long) worst, worstX);
    // geglu outputs on gate ~ N(0, 1.5), up ~ N(0, 1): fp32 equality with libm's tanh
    int64_t differ = 0, total = 0;
    for (int i = 0; i < samples; ++i) {
        const float g = (float) (N(rng) * 1.5), u = (float) N(rng);
        const double xg = (double) g;
        const double inner = 0.7978845608028654 * (xg + 0.044715 * xg * xg * xg);
        if (inner >= 10.0 || inner <= -10.0) continue;
        ++total;
        differ += geglu(gq8::tanh_from_exp(inner), g, u) != geglu(std::tanh(inner), g, u);
    }
    printf("geglu fp32 differing from libm: %lld of %lld\n", (long long) differ, (long long) total);
    // Where 1 + tanh cancels (tanh argument in [-10, -3]) every fp32 gate,
    // against several up values (large ones included): the GeGLU as both
    // sides round it, (float) ((0.5 g (1 + t)) u)
    const double rootTwoOverPi = 0.7978845608028654;
    const float ups[] = {1.f, -1.f, 3.7f, -0.001f, 1000.f, -12345.678f, 65504.f};
    int64_t sweepDiffer = 0, sweepTotal = 0;
    for (float g = -3.7f; g <= -2.2f; g = std::nextafter(g, 0.f)) {
        const double x = (double) g;
        const double inner = rootTwoOverPi * (x + 0.044715 * x * x * x);
        if (inner < -10.0 || inner > -3.0) continue;
        const double ta = gq8::tanh_from_exp(inner), tb = std::tanh(inner);
        const double ga = 0.5 * x * (1.0 + ta), gb = 0.5 * x * (1.0 + tb);
        for (float u : ups) {
            ++sweepTotal;
            sweepDiffer += (float) (ga * (double) u) != (float) (gb * (double) u);
        }
    }
    printf("dense sweep (tanh argument in [-10, -3]) geglu fp32 differing from libm: %lld of %lld\n",
           (long long) sweepDiffer, (long long) sweepTotal);
}
