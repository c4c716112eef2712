// VoxelNav16: a gather-heavy 3-D navigation env.
//
// There is no reference code for this env; it is written from its
// specification. The reference's examples/VoxelNav is a different heightmap
// env. Specification:
//   - each env owns a 16 x 16 x 16 uint8 occupancy grid (1 = occupied), each
//     cell occupied with probability 1/4, drawn from the env's RNG at every reset;
//   - the agent and the goal start on distinct random free cells;
//   - 6 actions: +x, -x, +y, -y, +z, -z; a move into an occupied cell or out of
//     the grid is blocked and the agent stays;
//   - obs = the 3x3x3 occupancy neighbourhood around the agent as 27 floats
//     (out-of-grid cells read as occupied; order z, then y, then x, each -1..1),
//     then the goal delta (goal - agent) / 15 per axis: OBS_DIM = 30;
//   - reward -0.01 per step, -0.1 on a blocked move, +1 on reaching the goal;
//   - the episode ends at the goal or after 256 steps.
//
// RNG use per reset: 256 draws fill the grid (each 32-bit draw gives 16 cells,
// a cell is occupied when its 2-bit field is 3), then rejection draws
// (rngNext & 4095) for the agent cell and then the goal cell, at most 64 each;
// if all 64 land on occupied cells the last drawn cell is cleared.
//
// The state is 4 KB per env, so the kernels keep it in device memory (or a
// rollout's LDS) instead of registers. The 27 neighbourhood cells are declared
// a split observation (OBS_SPLIT, env.h): independent gathers from the grid,
// which the kernels spread over a workgroup's threads.
#pragma once
#include <stddef.h>

#include "../env.h"

struct VoxelNav16 {
    static constexpr int G = 16;
    static constexpr int CELLS = G * G * G;
    struct State {
        int32_t px, py, pz;
        int32_t gx, gy, gz;
        uint32_t steps;
        uint32_t pad;
        uint8_t grid[CELLS];  // index (z * 16 + y) * 16 + x
    };
    using Action = int;
    struct Obs {
        float cells[27];
        float goal[3];
    };

    static constexpr uint32_t OBS_DIM = 30;
    static constexpr uint32_t ACT_DIM = 6;
    static constexpr const char* KERNEL = "rollout_voxelnav16";
    static constexpr uint32_t MAX_STEPS = 256;
    static constexpr int MAX_TRIES = 64;

    MG_HD static int cell(int x, int y, int z) { return (z * G + y) * G + x; }

    MG_HD static bool occupied(const State& s, int x, int y, int z) {
        if (x < 0 || y < 0 || z < 0 || x >= G || y >= G || z >= G) return true;
        return s.grid[cell(x, y, z)] != 0;
    }

    MG_HD static int draw_free_cell(State& s, uint32_t& rng, int avoid) {
        int c = 0;
        for (int t = 0; t < MAX_TRIES; ++t) {
            c = (int)(rngNext(rng) & (uint32_t)(CELLS - 1));
            if (s.grid[c] == 0 && c != avoid) return c;
        }
        if (c == avoid) c = (c + 1) & (CELLS - 1);
        s.grid[c] = 0;
        return c;
    }

    MG_HD static void reset(State& s, uint32_t& rng) {
        for (int w = 0; w < CELLS / 16; ++w) {
            const uint32_t r = rngNext(rng);
            // bit 2 c of f is set iff the 2-bit field c of r is 3; cells 4 q ..
            // 4 q + 3 are bits 8 q, 8 q + 2, 8 q + 4, 8 q + 6 of f, and the
            // multiply by 2^0 + 2^6 + 2^12 + 2^18 moves bit 2 j of x to bit 8 j
            // (the other products land on bits 2 i + 6 k, two at most on one
            // bit, whose carries go to bits 7, 13 and 19, masked off)
            const uint32_t f = r & (r >> 1) & 0x55555555u;
            uint32_t packed[4];
            for (int q = 0; q < 4; ++q) packed[q] = (((f >> (8 * q)) & 0x55u) * 0x41041u) & 0x01010101u;
            __builtin_memcpy(s.grid + 16 * w, packed, 16);
        }
        int a = draw_free_cell(s, rng, -1);
        int g = draw_free_cell(s, rng, a);
        s.px = a % G;
        s.py = (a / G) % G;
        s.pz = a / (G * G);
        s.gx = g % G;
        s.gy = (g / G) % G;
        s.gz = g / (G * G);
        s.steps = 0;
    }

    static constexpr uint32_t OBS_SPLIT = 27;
    // a step moves the agent and counts (px .. pad); the grid changes on reset only
    static constexpr uint32_t STEP_WRITES = 8;
    static_assert(offsetof(State, grid) == 4 * STEP_WRITES, "the grid follows the 8-dword header");

    // neighbourhood cell k = 9 (dz + 1) + 3 (dy + 1) + (dx + 1)
    MG_HD static float observePart(const State& s, uint32_t k) {
        const int dx = (int)(k % 3u) - 1, dy = (int)(k / 3u % 3u) - 1, dz = (int)(k / 9u) - 1;
        return occupied(s, s.px + dx, s.py + dy, s.pz + dz) ? 1.0f : 0.0f;
    }

    // (float)d / 15.0f for an integer d in [-15, 15] (a goal delta): the
    // product with the float nearest 1/15 and one FMA correction give the
    // correctly rounded quotient for each of the 31 values (checked on the
    // host in tests/native/voxelnav16_fill.cpp), in 3 instructions instead of
    // the 10 of an IEEE division.
    MG_HD static float div15(int d) {
        const float x = (float)d, r = 1.0f / 15.0f;
        const float q = x * r;
        return __builtin_fmaf(__builtin_fmaf(-q, 15.0f, x), r, q);
    }

    MG_HD static void observeRest(const State& s, Obs& obs) {
        obs.goal[0] = div15(s.gx - s.px);
        obs.goal[1] = div15(s.gy - s.py);
        obs.goal[2] = div15(s.gz - s.pz);
    }

    MG_HD static void observe(const State& s, Obs& obs) {
        for (uint32_t k = 0; k < OBS_SPLIT; ++k) obs.cells[k] = observePart(s, k);
        observeRest(s, obs);
    }

    MG_HD static void stepState(State& s, Action action, float& reward, uint8_t& done) {
        int a = action < 0 ? 0 : (action > 5 ? 5 : action);
        int sign = (a & 1) ? -1 : 1;
        int axis = a >> 1;
        int nx = s.px + (axis == 0 ? sign : 0);
        int ny = s.py + (axis == 1 ? sign : 0);
        int nz = s.pz + (axis == 2 ? sign : 0);
        bool blocked = occupied(s, nx, ny, nz);
        if (!blocked) {
            s.px = nx;
            s.py = ny;
            s.pz = nz;
        }
        s.steps += 1;
        bool atGoal = s.px == s.gx && s.py == s.gy && s.pz == s.gz;
        reward = atGoal ? 1.0f : (blocked ? -0.1f : -0.01f);
        done = (atGoal || s.steps >= MAX_STEPS) ? 1 : 0;
    }

    MG_HD static void step(State& s, Action action, Obs& obs, float& reward, uint8_t& done) {
        stepState(s, action, reward, done);
        observe(s, obs);
    }
};
