// A user-defined env written against mg/env.h: a 16-cell corridor, start at a
// random cell, +1 on reaching the right end, -0.01 per step, 64-step cap.
#pragma once
#include "mg/env.h"

struct Corridor {
    struct State {
        int32_t pos;
        uint32_t steps;
    };
    using Action = int;  // 0 = left, 1 = right
    struct Obs {
        float pos;
        float bias;
    };
    static constexpr uint32_t OBS_DIM = 2;
    static constexpr uint32_t ACT_DIM = 2;
    static constexpr const char* KERNEL = "rollout_corridor";

    MG_HD static void reset(State& s, uint32_t& rng) {
        s.pos = (int32_t)rngInt(rng, 15);
        s.steps = 0;
    }
    MG_HD static void step(State& s, Action a, Obs& obs, float& reward, uint8_t& done) {
        s.pos += a == 1 ? 1 : -1;
        if (s.pos < 0) s.pos = 0;
        s.steps += 1;
        const bool goal = s.pos >= 15;
        reward = goal ? 1.0f : -0.01f;
        done = (goal || s.steps >= 64) ? 1 : 0;
        obs.pos = (float)s.pos / 15.0f;
        obs.bias = 1.0f;
    }
};
