// The rollout<Env> kernel: one lane per env, `steps` env steps per launch with
// the state and RNG held in registers (rollout.h:31-54 runs one step per
// dispatch and round-trips everything through memory). Envs with a split
// observation and a large state run rollout_split_kernel instead (below).
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

// The rollout of an env with a split observation (EnvTraits::OBS_SPLIT = K >
// 0) whose State can be staged in LDS: a workgroup of NT threads owns E envs,
// their states in LDS for the whole launch (env e at dword e * STRIDE, an odd
// stride). Per step its first E lanes pick the action, reset if done, run
// Env::stepState and Env::observeRest and write their slots; after a barrier
// the NT threads compute the E x K observation parts from the LDS states.
// Same draws, order and floats as rollout_kernel.
template <typename Env>
struct SplitRollout {
    using State = typename Env::State;
    static constexpr uint32_t K = EnvTraits<Env>::OBS_SPLIT;
    static constexpr uint32_t SD = sizeof(State) / 4;
    static constexpr uint32_t STRIDE = SD % 2 ? SD : SD + 1;
    static constexpr bool OK = K > 0 && !EnvTraits<Env>::STATE_IN_REGISTERS && sizeof(State) % 4 == 0 &&
                               alignof(State) <= 4;
};
template <typename Env, int MODE, int E, int NT = 256>
__global__ void __launch_bounds__(NT) rollout_split_kernel(const mg_rollout_args a) {
    using SR = SplitRollout<Env>;
    using State = typename Env::State;
    using Action = typename Env::Action;
    using Obs = typename Env::Obs;
    constexpr int O = Env::OBS_DIM;
    constexpr uint32_t K = SR::K, SD = SR::SD, STRIDE = SR::STRIDE;
    // an env whose steps write only its first HW dwords writes the rest back
    // only if it reset during the launch (reset_in)
    constexpr uint32_t HW = EnvTraits<Env>::STEP_WRITES;
    constexpr bool PART = HW < SD;
    __shared__ uint32_t lds[E * STRIDE];
    __shared__ uint32_t reset_in[PART ? E : 1];
    const uint32_t n = a.n, tid = threadIdx.x, e0 = blockIdx.x * E;
    const uint32_t ne = n - e0 < (uint32_t)E ? n - e0 : (uint32_t)E;  // envs of this workgroup
    uint32_t* gst = reinterpret_cast<uint32_t*>(static_cast<State*>(a.state) + e0);
    // every thread loads an env's RNG and done flag (the env lanes keep theirs),
    // branch-free and before the states, so all of it is one round trip
    const uint32_t ei = e0 + (tid < ne ? tid : 0);
    uint32_t rng = a.rng[ei];
    uint8_t done = a.done[ei];
    states_to_lds<SD, STRIDE, E, NT>(lds, gst, ne);
    if (PART && tid < (uint32_t)E) reset_in[tid] = 0;
    __syncthreads();
    for (uint32_t t = 0; t < a.steps; ++t) {
        if (tid < ne) {
            State& s = *reinterpret_cast<State*>(lds + tid * STRIDE);
            const size_t k = (size_t)t * n + e0 + tid;
            Action act;
            if constexpr (MODE == MG_ACTIONS_RANDOM) {
                act = random_action<Env>(rng);
                if (a.actions_out) static_cast<Action*>(a.actions_out)[k] = act;
            } else {
                act = static_cast<const Action*>(a.actions_in)[k];
            }
            if (done) {
                Env::reset(s, rng);
                if constexpr (PART) reset_in[tid] = 1;
            }
            Obs o{};
            float r = 0.0f;
            Env::stepState(s, act, r, done);
            Env::observeRest(s, o);
            const float* of = reinterpret_cast<const float*>(&o);
            if (a.obs_out)
#pragma unroll
                for (int q = K; q < O; ++q) a.obs_out[k * O + q] = of[q];
            if (a.reward_out) a.reward_out[k] = r;
            if (a.done_out) a.done_out[k] = done;
        }
        __syncthreads();  // every state is stepped
        const size_t row0 = ((size_t)t * n + e0) * O;
        for (uint32_t q = tid; q < ne * K; q += NT) {
            const uint32_t e = q / K, p = q % K;
            const float v = Env::observePart(*reinterpret_cast<const State*>(lds + e * STRIDE), p);
            if (a.obs_out) a.obs_out[row0 + (size_t)e * O + p] = v;
        }
        __syncthreads();  // the parts are read before the next step writes the states
    }
    if (tid < ne) {
        a.rng[e0 + tid] = rng;
        a.done[e0 + tid] = done;
    }
    states_from_lds<SD, STRIDE, E, NT, HW>(lds, gst, ne, reset_in);  // reset_in: after the loop's last barrier
}

// rollout_split_kernel with E envs per workgroup on NT = 64 ceil(E K / 64)
// threads, so that every observation part of a step runs in one pass. Each
// step is a chain of dependent LDS accesses and two barriers, so the kernel is
// latency-bound and the shape decides how many envs a CU interleaves:
//  - states over 2 KB (VoxelNav16's 4 KB grids: LDS holds 36 to 38 per CU):
//    E = 4 on 128 threads. Random actions, 262144 envs, 32 steps: 771 us
//    against 827 on 256 threads (8 workgroups per CU instead of 9), 870 with
//    E = 2 on 64 threads, 1.02 ms with E = 4 on 64 (two passes of parts);
//  - smaller states (VoxelNav's 1 KB heightmaps, whose parts are ray marches):
//    E = 2 on one wave. 7.23 ms at 262144 envs against 7.46 with E = 8 on 128
//    threads and 8.43 with E = 16 on 256; 515 against 626 us at 4096 envs
//    (E = 4 on 128 threads).
template <typename Env, int MODE, int E>
void launch_split_e(const mg_rollout_args* a, hipStream_t st) {
    constexpr int P = E * (int)SplitRollout<Env>::K;
    constexpr int NT = P <= 64 ? 64 : P <= 128 ? 128 : 256;
    hipLaunchKernelGGL((rollout_split_kernel<Env, MODE, E, NT>), dim3((a->n + E - 1) / E), dim3(NT), 0, st, *a);
}

template <typename Env, int MODE>
void launch_split_rollout(const mg_rollout_args* a, hipStream_t st) {
    constexpr uint32_t bytes = SplitRollout<Env>::STRIDE * 4u;  // LDS per staged state
    constexpr int E = bytes > 2048u ? (bytes * 4u <= 17408u ? 4 : 1) : 2;
    launch_split_e<Env, MODE, E>(a, st);
}

// Returns 0, a positive hipError_t on a launch failure, or MG_ERR_INVALID.
template <typename Env>
int launch_rollout(const mg_rollout_args* a) {
    if (!a || a->n == 0 || !a->state || !a->rng || !a->done) return MG_ERR_INVALID;
    if (a->steps == 0) return 0;
    if (a->mode == MG_ACTIONS_GIVEN && !a->actions_in) return MG_ERR_INVALID;
    // one lane per env: below 64 K envs one-wave workgroups spread the waves
    // over more CUs (4096 envs are 64 waves: 64 CUs instead of 16)
    hipStream_t st = static_cast<hipStream_t>(a->stream);
    if constexpr (SplitRollout<Env>::OK) {
        if (a->mode == MG_ACTIONS_RANDOM)
            launch_split_rollout<Env, MG_ACTIONS_RANDOM>(a, st);
        else
            launch_split_rollout<Env, MG_ACTIONS_GIVEN>(a, st);
        return (int)hipGetLastError();
    }
    const uint32_t bs = a->n >= 65536u ? 256u : 64u;
    dim3 block(bs), grid((a->n + bs - 1) / bs);
    if (a->mode == MG_ACTIONS_RANDOM)
        hipLaunchKernelGGL((rollout_kernel<Env, MG_ACTIONS_RANDOM>), grid, block, 0, st, *a);
    else
        hipLaunchKernelGGL((rollout_kernel<Env, MG_ACTIONS_GIVEN>), grid, block, 0, st, *a);
    return (int)hipGetLastError();
}

}  // namespace dev
}  // namespace mg
