// Per-row action samplers, drawing from the env's own xorshift stream.
// Transcendentals come from mg/math.h so that, given the same head row, the
// device and the CPU oracle choose the same action and the same log-prob bits.
#pragma once
#include "common.h"

namespace mg {
namespace dev {

constexpr float kLogSqrt2Pi = 0.9189385332046727f;  // 0.5 * log(2 pi)
constexpr float kPiF = 3.14159265358979323846f;

// model/sample.metal:18-47: inverse-CDF draw; returns the action.
__device__ __forceinline__ int sample_categorical(const float* h, int A, uint32_t& rng, float& logp) {
    float rowMax = -__builtin_huge_valf();
    for (int a = 0; a < A; ++a) rowMax = rowMax < h[a] ? h[a] : rowMax;
    float sum = 0.0f;
    for (int a = 0; a < A; ++a) sum += mg::expf(h[a] - rowMax);
    const float lse = rowMax + mg::logf(sum);
    const float u = (float)(rngNext(rng) >> 8) * (1.0f / 16777216.0f) * sum;
    int chosen = A - 1;
    float acc = 0.0f;
    for (int a = 0; a < A; ++a) {
        acc += mg::expf(h[a] - rowMax);
        if (u < acc) {
            chosen = a;
            break;
        }
    }
    logp = h[chosen] - lse;
    return chosen;
}

// model/gaussian.metal:22-71: Box-Muller pairs, a = mu + exp(log_std) z.
__device__ __forceinline__ void sample_gaussian(const float* h, const float* logStd, int A, uint32_t& rng,
                                                float* act, float& logp) {
    float lp = 0.0f, z0 = 0.0f, z1 = 0.0f;
    for (int k = 0; k < A; ++k) {
        if ((k & 1) == 0) {
            const float u1 = 1.0f - (float)(rngNext(rng) >> 8) * (1.0f / 16777216.0f);
            const float u2 = (float)(rngNext(rng) >> 8) * (1.0f / 16777216.0f);
            const float r = sqrtf(-2.0f * mg::logf(u1));
            const float th = 2.0f * kPiF * u2;
            float st, ct;
            mg::sincosf(th, &st, &ct);  // the bits of mg::sinf and mg::cosf, one reduction
            z0 = r * ct;
            z1 = r * st;
        }
        const float zk = (k & 1) ? z1 : z0;
        const float ls = logStd[k];
        const float mu = h[k];
        const float a = mu + mg::expf(ls) * zk;
        const float d = (a - mu) * mg::expf(-ls);
        act[k] = a;
        lp += -0.5f * d * d - ls - kLogSqrt2Pi;
    }
    logp = lp;
}

}  // namespace dev
}  // namespace mg
