// Environment authoring API.
//
// An environment is one struct compiled for both host and device:
//
//   struct MyEnv {
//       struct State { ... };            // per-env state, lives on the GPU
//       using Action = int;              // 4-byte integer -> softmax head,
//                                        // or a struct of ACT_DIM floats -> Gaussian head
//       struct Obs { float ...; };       // exactly OBS_DIM floats
//       static constexpr uint32_t OBS_DIM = ...;
//       static constexpr uint32_t ACT_DIM = ...;
//       static constexpr const char* KERNEL = "rollout_myenv";   // registry key
//       MG_HD static void reset(State& s, uint32_t& rng);
//       MG_HD static void step(State& s, Action a, Obs& obs, float& reward, uint8_t& done);
//   };
//
// Optional split observation, for an observation made of independent parts
// (e.g. ray casts): an env that also defines
//
//       static constexpr uint32_t OBS_SPLIT = K;   // the first K floats of Obs
//       MG_HD static void stepState(State& s, Action a, float& reward, uint8_t& done);
//       MG_HD static float observePart(const State& s, uint32_t k);   // Obs float k < K
//       MG_HD static void observeRest(const State& s, Obs& obs);      // the floats >= K
//
// promises that step(s, a, obs, r, d) is stepState(s, a, r, d) followed by
// obs float k = observePart(s, k) for every k < K and observeRest(s, obs),
// with the same results. For a State of more than 64 bytes (smaller ones live
// in the env lane's registers) the kernels then spread a tile's K parts per env
// over all of its workgroup's threads: collect (states in LDS, or in device
// memory at two workgroups per CU) and, where the size is a multiple of 4, the
// rollouts (the tile's states staged in LDS). The other shapes call step().
//
// Optional, for a large State whose steps change only its first fields:
//
//       static constexpr uint32_t STEP_WRITES = D;   // dwords
//
// promises that stepState (and step) write nothing past the first D dwords of
// State; reset may write any. The rollouts that stage states in LDS then write
// the rest of an env's state back only if the env reset during the launch.
//
// This mirrors the reference's Env template (README.md:21-66; rollout.h:31-54):
// same member names, same reset/step contract, one struct instead of a Metal
// twin plus a host twin. A .hip file that includes <mg/device/env_kernels.h> and
// writes MG_DEFINE_ENV(MyEnv) instantiates the env's kernels and registers them
// under MyEnv::KERNEL, which is what Gym<MyEnv> looks up (gym.h:43-44).
//
// Per-env random numbers: one uint32 xorshift32 state per env (Marsaglia 2003,
// shifts 13/17/5), shared by resets and by the policy's samplers. The helper
// names and semantics follow rollout.h:9-29.
#pragma once
#include <stdint.h>
#include <type_traits>

#include "math.h"

// xorshift32 step; a zero state stays zero, so seeds are nonzero (rollout.h:9-14)
MG_HD uint32_t rngNext(uint32_t& s) {
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}

// uniform float in [0, 1): the top 24 bits times 2^-24, exact in fp32 (rollout.h:17-19)
MG_HD float rngUniform(uint32_t& s) { return (float)(rngNext(s) >> 8) * (1.0f / 16777216.0f); }

// uniform float in [lo, hi) (rollout.h:22-24)
MG_HD float rngUniform(uint32_t& s, float lo, float hi) { return lo + (hi - lo) * rngUniform(s); }

// uniform int in [0, n) by modulo (rollout.h:27-29)
MG_HD uint32_t rngInt(uint32_t& s, uint32_t n) { return rngNext(s) % n; }

namespace mg {

// Seed of env i. With seed 0 this is the reference's i * 2654435761 + 1
// (gym.h:57-61); other seeds xor in seed * 0x9E3779B9. The one index where the
// result would be 0 gets a fixed nonzero constant, since 0 is absorbing.
MG_HD uint32_t env_seed(uint32_t seed, uint32_t i) {
    uint32_t s = (i * 2654435761u + 1u) ^ (seed * 0x9E3779B9u);
    return s ? s : 0x6D2B79F5u;
}

template <typename Env, typename = void>
struct ObsSplit {
    static constexpr uint32_t value = 0;
};
template <typename Env>
struct ObsSplit<Env, std::void_t<decltype(Env::OBS_SPLIT)>> {
    static constexpr uint32_t value = Env::OBS_SPLIT;
};

template <typename Env, typename = void>
struct StepWrites {
    static constexpr uint32_t value = (uint32_t)((sizeof(typename Env::State) + 3) / 4);
};
template <typename Env>
struct StepWrites<Env, std::void_t<decltype(Env::STEP_WRITES)>> {
    static constexpr uint32_t value = Env::STEP_WRITES;
};

template <typename Env>
struct EnvTraits {
    using State = typename Env::State;
    using Action = typename Env::Action;
    using Obs = typename Env::Obs;
    static constexpr uint32_t OBS_DIM = Env::OBS_DIM;
    static constexpr uint32_t ACT_DIM = Env::ACT_DIM;
    // Integer action -> softmax head; struct of floats -> Gaussian head (model/ppo.h:110)
    static constexpr bool CONTINUOUS = !std::is_integral<Action>::value;
    // Small states are held in registers for a whole T-step rollout; large ones
    // (e.g. a voxel grid) are updated in place in device memory.
    static constexpr bool STATE_IN_REGISTERS = sizeof(State) <= 64;
    static_assert(sizeof(Obs) == OBS_DIM * sizeof(float), "Env::Obs must be exactly OBS_DIM floats");
    static_assert(CONTINUOUS || sizeof(Action) == 4, "the softmax head needs a discrete 4-byte Action");
    static_assert(!CONTINUOUS || sizeof(Action) == ACT_DIM * sizeof(float),
                  "the Gaussian head needs an Action of exactly ACT_DIM floats");
    static_assert(ACT_DIM >= 1 && ACT_DIM + 1 <= 64, "ACT_DIM + value must fit a 64-wide head");
    // the optional split observation's part count (0: none)
    static constexpr uint32_t OBS_SPLIT = ObsSplit<Env>::value;
    static_assert(OBS_SPLIT <= OBS_DIM, "OBS_SPLIT counts floats of Obs");
    // the leading dwords of State a step may write (all of them unless declared)
    static constexpr uint32_t STEP_WRITES = StepWrites<Env>::value;
    static_assert(STEP_WRITES >= 1 && STEP_WRITES <= (sizeof(State) + 3) / 4, "STEP_WRITES counts dwords of State");
};

}  // namespace mg
