// Test-only envs at the largest policy shape the library accepts: 64
// observation floats and a 64-column head (63 discrete actions, or 63 Gaussian
// means), each plus the value column. They exist to run the collect and train
// kernels at those dimensions; the dynamics only need to move the
// observations and give varied rewards.
#pragma once
#include "mg/env.h"

struct Wide64 {
    struct State {
        float x[64];
        uint32_t steps;
    };
    using Action = int;
    struct Obs {
        float v[64];
    };
    static constexpr uint32_t OBS_DIM = 64;
    static constexpr uint32_t ACT_DIM = 63;
    static constexpr const char* KERNEL = "rollout_test_wide64";

    MG_HD static void reset(State& s, uint32_t& rng) {
        for (int i = 0; i < 64; ++i) s.x[i] = rngUniform(rng, -1.0f, 1.0f);
        s.steps = 0;
    }
    MG_HD static void step(State& s, Action a, Obs& obs, float& reward, uint8_t& done) {
        s.x[a] += 0.25f;
        s.x[63 - a] -= 0.125f;
        s.steps += 1;
        reward = s.x[a] - s.x[0];
        done = s.steps >= 20 ? 1 : 0;
        for (int i = 0; i < 64; ++i) obs.v[i] = s.x[i];
    }
};

struct Wide64Gauss {
    struct State {
        float x[64];
        uint32_t steps;
    };
    struct Action {
        float a[63];
    };
    struct Obs {
        float v[64];
    };
    static constexpr uint32_t OBS_DIM = 64;
    static constexpr uint32_t ACT_DIM = 63;
    static constexpr const char* KERNEL = "rollout_test_wide64_gauss";

    MG_HD static void reset(State& s, uint32_t& rng) {
        for (int i = 0; i < 64; ++i) s.x[i] = rngUniform(rng, -1.0f, 1.0f);
        s.steps = 0;
    }
    MG_HD static void step(State& s, Action a, Obs& obs, float& reward, uint8_t& done) {
        float r = 0.0f;
        for (int i = 0; i < 63; ++i) {
            const float u = a.a[i] > 1.0f ? 1.0f : (a.a[i] < -1.0f ? -1.0f : a.a[i]);
            s.x[i + 1] += 0.1f * u;
            r -= 0.01f * u * u;
        }
        s.steps += 1;
        reward = r + s.x[1];
        done = s.steps >= 20 ? 1 : 0;
        for (int i = 0; i < 64; ++i) obs.v[i] = s.x[i];
    }
};
