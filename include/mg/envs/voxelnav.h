// VoxelNav: the reference's heightmap navigation env
// (examples/VoxelNav/voxelnav.metal:9-174). Terrain is a 32 x 32 grid of uint8
// column heights (0 marks a hole); a trench of holes runs the length of the z
// axis and separates the spawn region from the goal region. Six discrete
// actions move, turn, leap two cells or drop a cobble block in front of the
// agent. Each step it sees 32 depth samples (8 yaw angles x 4 pitch angles,
// marched through the grid) and the goal's position relative to its heading. Same State / Obs layout, constants, RNG draw order and
// arithmetic order as the reference; its Metal sin / cos are replaced by the
// deterministic mg::sinf / mg::cosf so the host oracle and the GPU agree bit
// for bit (the reference's own fast-math bits are not reproducible here).
//
// The state is 1 KB per env (the heightmap), so the rollout kernels update it
// in place in device memory.
#pragma once
#include <math.h>

#include "../env.h"
#include "../math.h"

struct VoxelNav {
    static constexpr uint32_t W = 32;
    static constexpr uint32_t RAY_COLS = 8;
    static constexpr uint32_t RAY_ROWS = 4;
    static constexpr uint32_t N_RAYS = RAY_COLS * RAY_ROWS;
    static constexpr uint32_t OBS_DIM = N_RAYS + 8;
    static constexpr uint32_t ACT_DIM = 6;
    static constexpr uint32_t MAX_STEPS = 250;
    static constexpr float PI = 3.14159265358979323846f;  // Metal's M_PI_F
    static constexpr float FOV = 90.0f * PI / 180.0f;
    static constexpr float MAX_DEPTH = 24.0f;
    static constexpr float EYE = 1.6f;
    static constexpr float GOAL_RADIUS = 1.5f;
    static constexpr uint32_t START_COBBLE = 16;
    static constexpr const char* KERNEL = "rollout_voxelnav";

    struct State {
        float x, z, yaw;
        float gx, gz;
        float prevDist;
        uint32_t steps;
        uint32_t cobble;
        uint8_t height[W * W];  // column height of cell (x, z) at x * W + z; 0 is a hole
    };
    using Action = int;  // 0 step ahead, 1 step back, 2 / 3 yaw -30 / +30 degrees, 4 leap 2 cells, 5 cobble
    struct Obs {
        float ray[N_RAYS];  // depth / MAX_DEPTH, ray c * RAY_ROWS + r
        float goalForward, goalRight, goalUp, goalDist;
        float sinYaw, cosYaw, cobble, height;
    };

    MG_HD static uint32_t cell(int cx, int cz) { return (uint32_t)cx * W + (uint32_t)cz; }
    MG_HD static bool inside(int cx, int cz) { return cx >= 0 && cz >= 0 && cx < (int)W && cz < (int)W; }
    MG_HD static float heightAt(const State& s, float x, float z) {
        const int cx = (int)floorf(x), cz = (int)floorf(z);
        return inside(cx, cz) ? (float)s.height[cell(cx, cz)] : 0.0f;
    }
    MG_HD static float dist(const State& s) {
        const float dx = s.gx - s.x, dz = s.gz - s.z;
        return sqrtf(dx * dx + dz * dz);
    }
    // Metal's mix(x, y, a) = x + (y - x) a
    MG_HD static float mix(float x, float y, float a) { return x + (y - x) * a; }

    MG_HD static void reset(State& s, uint32_t& rng) {
        // base terrain: heights in [3, 9] on a 5 x 5 lattice, bilinearly
        // interpolated to every cell and rounded
        float knot[25];
        for (uint32_t i = 0; i < 25; i++) knot[i] = rngUniform(rng, 3.0f, 9.0f);
        for (uint32_t cx = 0; cx < W; cx++) {
            const float fx = (float)cx / (float)(W - 1) * 4.0f;
            const uint32_t ix = (uint32_t)fx < 3u ? (uint32_t)fx : 3u;
            const float tx = fx - (float)ix;
            for (uint32_t cz = 0; cz < W; cz++) {
                const float fz = (float)cz / (float)(W - 1) * 4.0f;
                const uint32_t iz = (uint32_t)fz < 3u ? (uint32_t)fz : 3u;
                const float tz = fz - (float)iz;
                const float h = mix(mix(knot[ix * 5 + iz], knot[(ix + 1) * 5 + iz], tx),
                                    mix(knot[ix * 5 + iz + 1], knot[(ix + 1) * 5 + iz + 1], tx), tz);
                s.height[cell((int)cx, (int)cz)] = (uint8_t)roundf(h);
            }
        }
        // trench: columns left .. left + width - 1 (width 2-5) become holes, and
        // every column past the trench is raised by 0-2 (capped at 15)
        const uint32_t width = 2 + rngInt(rng, 4);
        const uint32_t left = 12 + rngInt(rng, 6);
        const uint32_t lift = rngInt(rng, 3);
        for (uint32_t cx = 0; cx < W; cx++) {
            for (uint32_t cz = 0; cz < W; cz++) {
                const uint32_t k = cell((int)cx, (int)cz);
                if (cx >= left && cx < left + width) {
                    s.height[k] = 0;
                } else if (cx >= left + width) {
                    const uint32_t lifted = (uint32_t)s.height[k] + lift;
                    s.height[k] = (uint8_t)(lifted < 15u ? lifted : 15u);
                }
            }
        }
        s.x = 2.5f + rngUniform(rng) * (float)(left - 4);
        s.z = 2.5f + rngUniform(rng) * (float)(W - 5);
        s.gx = (float)(left + width) + 2.5f + rngUniform(rng) * (float)(W - 5 - (left + width));
        s.gz = 2.5f + rngUniform(rng) * (float)(W - 5);
        s.yaw = rngUniform(rng, -PI, PI);
        s.prevDist = dist(s);
        s.steps = 0;
        s.cobble = START_COBBLE;
    }

    // Depth of the ray of pitch row r from eye height ey along yaw direction
    // (ca, sa): the first sample t = 0.5, 1, ..., 23.5 off the grid or at or
    // below a column top, else MAX_DEPTH; divided by MAX_DEPTH. The samples go
    // four at a time: the four column heights are read before any is tested,
    // so their memory latencies overlap, and the first hit in sample order
    // wins, as in a sample-by-sample march (t = 0.5 k is exact).
    MG_HD static float march(const State& s, float ey, float ca, float sa, uint32_t r) {
        const float pitches[RAY_ROWS] = {-45.0f, -20.0f, 0.0f, 15.0f};
        const float p = pitches[r] * PI / 180.0f;
        float sp, cp;
        mg::sincosf(p, &sp, &cp);  // the bits of mg::sinf and mg::cosf, one reduction
        const float dx = cp * ca, dy = sp, dz = cp * sa;
        constexpr uint32_t kSamples = 47;  // t = 0.5 k < MAX_DEPTH
        for (uint32_t k0 = 1; k0 <= kSamples; k0 += 4) {
            bool hit[4];
            for (uint32_t u = 0; u < 4; u++) {
                const float t = 0.5f * (float)(k0 + u);
                const float px = s.x + t * dx, py = ey + t * dy, pz = s.z + t * dz;
                const int cx = (int)floorf(px), cz = (int)floorf(pz);
                const bool in = inside(cx, cz);
                const float top = (float)s.height[in ? cell(cx, cz) : 0u];
                hit[u] = k0 + u <= kSamples && (!in || py <= top);
            }
            for (uint32_t u = 0; u < 4; u++)
                if (hit[u]) return 0.5f * (float)(k0 + u) / MAX_DEPTH;
        }
        return MAX_DEPTH / MAX_DEPTH;
    }
    // Yaw of ray column c.
    MG_HD static float rayYaw(const State& s, uint32_t c) {
        return s.yaw + ((float)c / (float)(RAY_COLS - 1) - 0.5f) * FOV;
    }

    // The observation's first N_RAYS floats are independent depth samples, so
    // kernels that hold a tile's states where all its threads can read them
    // may compute them in parallel (observePart), then the rest (observeRest);
    // observe() gives the same floats.
    static constexpr uint32_t OBS_SPLIT = N_RAYS;
    MG_HD static float observePart(const State& s, uint32_t k) {
        const uint32_t c = k / RAY_ROWS, r = k % RAY_ROWS;
        const float a = rayYaw(s, c);
        float sa, ca;
        mg::sincosf(a, &sa, &ca);
        return march(s, heightAt(s, s.x, s.z) + EYE, ca, sa, r);
    }
    MG_HD static void observeRest(const State& s, Obs& o) {
        const float h = heightAt(s, s.x, s.z);
        const float gx = s.gx - s.x, gz = s.gz - s.z;
        float sa, ca;
        mg::sincosf(s.yaw, &sa, &ca);
        o.goalForward = (gx * ca + gz * sa) / (float)W;
        o.goalRight = (-gx * sa + gz * ca) / (float)W;
        o.goalUp = (heightAt(s, s.gx, s.gz) - h) / 8.0f;
        o.goalDist = sqrtf(gx * gx + gz * gz) / (float)W;
        o.sinYaw = sa;
        o.cosYaw = ca;
        o.cobble = (float)s.cobble / (float)START_COBBLE;
        o.height = h / 16.0f;
    }

    MG_HD static void observe(const State& s, Obs& o) {
        const float ey = heightAt(s, s.x, s.z) + EYE;
        for (uint32_t c = 0; c < RAY_COLS; c++) {
            const float a = rayYaw(s, c);
            float sa, ca;
            mg::sincosf(a, &sa, &ca);
            for (uint32_t r = 0; r < RAY_ROWS; r++) o.ray[c * RAY_ROWS + r] = march(s, ey, ca, sa, r);
        }
        observeRest(s, o);
    }

    // A move to (nx, nz): refused off the grid or onto a column more than one
    // above the current one; onto a hole it is taken and reported (true) as a
    // fall.
    MG_HD static bool tryMove(State& s, float nx, float nz) {
        const int cx = (int)floorf(nx), cz = (int)floorf(nz);
        if (!inside(cx, cz)) return false;
        const float here = heightAt(s, s.x, s.z);
        const float there = (float)s.height[cell(cx, cz)];
        if (there == 0.0f) {
            s.x = nx;
            s.z = nz;
            return true;
        }
        if (there > here + 1.0f) return false;
        s.x = nx;
        s.z = nz;
        return false;
    }

    // step() without its observation (the split-observation path).
    MG_HD static void stepState(State& s, Action action, float& reward, uint8_t& done) {
        float sa, ca;
        mg::sincosf(s.yaw, &sa, &ca);
        bool fell = false;
        switch (action) {
            case 0: fell = tryMove(s, s.x + ca, s.z + sa); break;
            case 1: fell = tryMove(s, s.x - ca, s.z - sa); break;
            case 2: s.yaw -= PI / 6.0f; break;
            case 3: s.yaw += PI / 6.0f; break;
            case 4: fell = tryMove(s, s.x + 2.0f * ca, s.z + 2.0f * sa); break;
            case 5: {
                const int cx = (int)floorf(s.x + ca), cz = (int)floorf(s.z + sa);
                if (s.cobble > 0 && inside(cx, cz)) {
                    const uint32_t k = cell(cx, cz);
                    const uint32_t here = (uint32_t)heightAt(s, s.x, s.z);
                    if (s.height[k] == 0) {
                        s.height[k] = (uint8_t)here;
                        s.cobble--;
                    } else if ((uint32_t)s.height[k] <= here) {
                        s.height[k]++;
                        s.cobble--;
                    }
                }
                break;
            }
            default: break;
        }
        if (s.yaw > PI) s.yaw -= 2.0f * PI;
        if (s.yaw < -PI) s.yaw += 2.0f * PI;
        s.steps++;

        const float d = dist(s);
        const float prog = s.prevDist - d;
        reward = -0.05f + 0.2f * (prog < -1.5f ? -1.5f : (prog > 1.5f ? 1.5f : prog));
        s.prevDist = d;
        const bool success = d < GOAL_RADIUS;
        if (success) reward += 10.0f;
        if (fell) reward -= 5.0f;
        done = (success || fell || s.steps >= MAX_STEPS) ? 1 : 0;
    }

    MG_HD static void step(State& s, Action action, Obs& obs, float& reward, uint8_t& done) {
        stepState(s, action, reward, done);
        observe(s, obs);
    }
};
