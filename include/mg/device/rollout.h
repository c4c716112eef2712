// The rollout<Env> kernel: one lane per env, `steps` env steps per launch with
// the state and RNG held in registers (rollout.h:31-54 runs one step per
// dispatch and round-trips everything through memory).
//
// Per env and step: pick the action (given, or drawn from the env's RNG before
// the reset), reset if the stored done flag is set, Env::step, then coalesced
// [steps][n] slot writes. Obs and reward start at zero before Env::step (the
// reference loads the previous contents of the output slot; step() overwrites
// both in every env).
#pragma once
#include "common.h"

namespace mg {
namespace dev {

template <typename Env, int MODE>
__global__ void __launch_bounds__(256) rollout_kernel(const mg_rollout_args a) {
    using Tr = EnvTraits<Env>;
    using State = typename Env::State;
    using Action = typename Env::Action;
    using Obs = typename Env::Obs;
    constexpr int O = Env::OBS_DIM;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    const uint32_t n = a.n;
    State* states = static_cast<State*>(a.state);
    uint32_t rng = a.rng[i];
    uint8_t done = a.done[i];

    auto run = [&](State& s) {
        for (uint32_t t = 0; t < a.steps; ++t) {
            const size_t k = (size_t)t * n + i;
            Action act;
            if constexpr (MODE == MG_ACTIONS_RANDOM) {
                act = random_action<Env>(rng);
                if (a.actions_out) static_cast<Action*>(a.actions_out)[k] = act;
            } else {
                act = static_cast<const Action*>(a.actions_in)[k];
            }
            if (done) Env::reset(s, rng);
            Obs o{};
            float r = 0.0f;
            Env::step(s, act, o, r, done);
            if (a.obs_out) store_floats<O>(a.obs_out + k * O, reinterpret_cast<const float*>(&o));
            if (a.reward_out) a.reward_out[k] = r;
            if (a.done_out) a.done_out[k] = done;
        }
    };
    if constexpr (Tr::STATE_IN_REGISTERS) {
        State s = states[i];
        run(s);
        states[i] = s;
    } else {
        run(states[i]);
    }
    a.rng[i] = rng;
    a.done[i] = done;
}

// Returns 0, a positive hipError_t on a launch failure, or MG_ERR_INVALID.
template <typename Env>
int launch_rollout(const mg_rollout_args* a) {
    if (!a || a->n == 0 || !a->state || !a->rng || !a->done) return MG_ERR_INVALID;
    if (a->steps == 0) return 0;
    if (a->mode == MG_ACTIONS_GIVEN && !a->actions_in) return MG_ERR_INVALID;
    // one lane per env: below 64 K envs one-wave workgroups spread the waves
    // over more CUs (4096 envs are 64 waves: 64 CUs instead of 16)
    const uint32_t bs = a->n >= 65536u ? 256u : 64u;
    dim3 block(bs), grid((a->n + bs - 1) / bs);
    hipStream_t st = static_cast<hipStream_t>(a->stream);
    if (a->mode == MG_ACTIONS_RANDOM)
        hipLaunchKernelGGL((rollout_kernel<Env, MG_ACTIONS_RANDOM>), grid, block, 0, st, *a);
    else
        hipLaunchKernelGGL((rollout_kernel<Env, MG_ACTIONS_GIVEN>), grid, block, 0, st, *a);
    return (int)hipGetLastError();
}

}  // namespace dev
}  // namespace mg
