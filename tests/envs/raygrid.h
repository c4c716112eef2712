// Test-only ray-casting envs: RayGrid and RayGridSplit are one env, the second
// also declaring its observation split (OBS_SPLIT, see mg/env.h), so the
// kernels that spread the parts over a workgroup must give the same bits as
// the ones that call step(). A 16 x 16 grid of column heights and an agent
// with a position and heading; 24 depth rays, then position and heading. The
// 272-byte State is too large for registers and small enough for LDS.
#pragma once
#include "mg/env.h"

struct RayGridBase {
    static constexpr uint32_t G = 16, N_RAYS = 24;
    struct State {
        float x, z, yaw;
        uint32_t steps;
        uint8_t h[G * G];
    };
    using Action = int;  // 0 forward, 1 turn left, 2 turn right
    struct Obs {
        float ray[N_RAYS];
        float x, z, sinYaw, cosYaw;
    };
    static constexpr uint32_t OBS_DIM = N_RAYS + 4;
    static constexpr uint32_t ACT_DIM = 3;

    MG_HD static bool inside(float x, float z) { return x >= 0.0f && z >= 0.0f && x < (float)G && z < (float)G; }
    MG_HD static float top(const State& s, float x, float z) { return (float)s.h[(uint32_t)x * G + (uint32_t)z]; }

    MG_HD static void reset(State& s, uint32_t& rng) {
        for (uint32_t i = 0; i < G * G; i++) s.h[i] = (uint8_t)rngInt(rng, 4);
        s.x = rngUniform(rng, 4.0f, 12.0f);
        s.z = rngUniform(rng, 4.0f, 12.0f);
        s.yaw = rngUniform(rng, -3.0f, 3.0f);
        s.steps = 0;
    }
    // ray k: the first of 32 half-cell samples off the grid or on a column of
    // height 3, as a fraction of 16 cells
    MG_HD static float observePart(const State& s, uint32_t k) {
        const float a = s.yaw + ((float)k / (float)(N_RAYS - 1) - 0.5f) * 2.0f;
        const float dx = mg::cosf(a), dz = mg::sinf(a);
        for (uint32_t i = 1; i <= 32; i++) {
            const float t = 0.5f * (float)i;
            const float px = s.x + t * dx, pz = s.z + t * dz;
            if (!inside(px, pz) || top(s, px, pz) >= 3.0f) return t / 16.0f;
        }
        return 1.0f;
    }
    MG_HD static void observeRest(const State& s, Obs& o) {
        o.x = s.x / (float)G;
        o.z = s.z / (float)G;
        o.sinYaw = mg::sinf(s.yaw);
        o.cosYaw = mg::cosf(s.yaw);
    }
    MG_HD static void stepState(State& s, Action a, float& reward, uint8_t& done) {
        if (a == 1) {
            s.yaw -= 0.4f;
        } else if (a == 2) {
            s.yaw += 0.4f;
        } else {
            s.x += 0.5f * mg::cosf(s.yaw);
            s.z += 0.5f * mg::sinf(s.yaw);
        }
        s.steps++;
        const bool out = !inside(s.x, s.z);
        const bool blocked = !out && top(s, s.x, s.z) >= 3.0f;
        reward = out || blocked ? -1.0f : 0.1f;
        done = (out || blocked || s.steps >= 100) ? 1 : 0;
    }
    MG_HD static void step(State& s, Action a, Obs& obs, float& reward, uint8_t& done) {
        stepState(s, a, reward, done);
        for (uint32_t k = 0; k < N_RAYS; k++) obs.ray[k] = observePart(s, k);
        observeRest(s, obs);
    }
};

struct RayGrid : RayGridBase {
    static constexpr const char* KERNEL = "rollout_test_raygrid";
};
struct RayGridSplit : RayGridBase {
    static constexpr uint32_t OBS_SPLIT = N_RAYS;
    // a step writes x, z, yaw and steps; the heights change on reset only
    static constexpr uint32_t STEP_WRITES = 4;
    static constexpr const char* KERNEL = "rollout_test_raygrid_split";
};

// RayField and RayFieldSplit: the same kind of env with a 20-byte State, which
// the kernels hold in registers, the column heights hashed from the cell and a
// per-episode seed instead of stored. Where a State lives in registers the
// kernels must call step() even though the env declares a split observation
// (no other thread can read the state): the two must give the same bits at
// every collect layout.
struct RayFieldBase {
    static constexpr uint32_t G = 16, N_RAYS = 12;
    struct State {
        float x, z, yaw;
        uint32_t steps, seed;
    };
    using Action = int;  // 0 forward, 1 turn left, 2 turn right
    struct Obs {
        float ray[N_RAYS];
        float x, z, sinYaw, cosYaw;
    };
    static constexpr uint32_t OBS_DIM = N_RAYS + 4;
    static constexpr uint32_t ACT_DIM = 3;

    MG_HD static bool inside(float x, float z) { return x >= 0.0f && z >= 0.0f && x < (float)G && z < (float)G; }
    // column height 0 .. 3 of the cell holding (x, z), inside the grid
    MG_HD static uint32_t top(const State& s, float x, float z) {
        uint32_t h = ((uint32_t)x * 73856093u) ^ ((uint32_t)z * 19349663u) ^ s.seed;
        h ^= h >> 13;
        h *= 0x5bd1e995u;
        h ^= h >> 15;
        return h & 3u;
    }
    MG_HD static void reset(State& s, uint32_t& rng) {
        s.seed = rngNext(rng);
        s.x = rngUniform(rng, 4.0f, 12.0f);
        s.z = rngUniform(rng, 4.0f, 12.0f);
        s.yaw = rngUniform(rng, -3.0f, 3.0f);
        s.steps = 0;
    }
    MG_HD static float observePart(const State& s, uint32_t k) {
        const float a = s.yaw + ((float)k / (float)(N_RAYS - 1) - 0.5f) * 2.0f;
        const float dx = mg::cosf(a), dz = mg::sinf(a);
        for (uint32_t i = 1; i <= 24; i++) {
            const float t = 0.5f * (float)i;
            const float px = s.x + t * dx, pz = s.z + t * dz;
            if (!inside(px, pz) || top(s, px, pz) >= 3u) return t / 16.0f;
        }
        return 1.0f;
    }
    MG_HD static void observeRest(const State& s, Obs& o) {
        o.x = s.x / (float)G;
        o.z = s.z / (float)G;
        o.sinYaw = mg::sinf(s.yaw);
        o.cosYaw = mg::cosf(s.yaw);
    }
    MG_HD static void stepState(State& s, Action a, float& reward, uint8_t& done) {
        if (a == 1) {
            s.yaw -= 0.4f;
        } else if (a == 2) {
            s.yaw += 0.4f;
        } else {
            s.x += 0.5f * mg::cosf(s.yaw);
            s.z += 0.5f * mg::sinf(s.yaw);
        }
        s.steps++;
        const bool out = !inside(s.x, s.z);
        const bool blocked = !out && top(s, s.x, s.z) >= 3u;
        reward = out || blocked ? -1.0f : 0.1f;
        done = (out || blocked || s.steps >= 100) ? 1 : 0;
    }
    MG_HD static void step(State& s, Action a, Obs& obs, float& reward, uint8_t& done) {
        stepState(s, a, reward, done);
        for (uint32_t k = 0; k < N_RAYS; k++) obs.ray[k] = observePart(s, k);
        observeRest(s, obs);
    }
};

struct RayField : RayFieldBase {
    static constexpr const char* KERNEL = "rollout_test_rayfield";
};
struct RayFieldSplit : RayFieldBase {
    static constexpr uint32_t OBS_SPLIT = N_RAYS;
    static constexpr const char* KERNEL = "rollout_test_rayfield_split";
};
