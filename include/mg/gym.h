// Gym<Env>: the env runtime with the reference's API (gym.h:15-122), on the
// metalgym_amd C ABI. Header-only; link with -lmetalgym_amd. Env is a struct
// written against mg/env.h whose kernels were registered with MG_DEFINE_ENV
// (the built-in envs are in the library).
//
// Device buffers belong to the library. The pointers returned by actions(),
// done() and obs() are host mirrors (MI355X memory is not host-shared the way
// Apple unified memory is): actions() is uploaded by run(); done() and obs()
// are downloaded when called. All calls block, as in the reference.
#pragma once
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <vector>

#include "capi.h"
#include "env.h"

namespace mg {

inline void check(int rc, const char* what) {
    if (rc != MG_OK) {
        std::cerr << what << ": " << mg_last_error() << "\n";
        std::exit(1);
    }
}

}  // namespace mg

template <typename Env>
struct Gym {
    using Traits = mg::EnvTraits<Env>;
    using Action = typename Env::Action;
    using Obs = typename Env::Obs;

    mg_gym* handle = nullptr;
    mg_gym_buffers buffers{};
    uint32_t parallels;
    std::vector<Action> actionHost;
    std::vector<Obs> obsHost;
    std::vector<uint8_t> doneHost;
    std::vector<float> rewardHost;

    // gym.h:36-61: n envs, done = 1, actions = 0, rng[i] = hash(seed, i)
    // (seed 0 reproduces the reference's i * 2654435761 + 1).
    explicit Gym(int p, uint32_t seed = 0) : parallels((uint32_t)p) {
        if (p <= 0) {
            std::cerr << "Gym: the env count must be positive\n";
            std::exit(1);
        }
        const mg_env_desc* desc = nullptr;
        if (mg_env_lookup(Env::KERNEL, &desc) != MG_OK) {
            std::cerr << "pipeline for " << Env::KERNEL << " failed: " << mg_last_error() << "\n";
            std::exit(1);
        }
        if (desc->state_bytes != sizeof(typename Env::State) || desc->action_bytes != sizeof(Action) ||
            desc->obs_dim != Env::OBS_DIM || desc->act_dim != Env::ACT_DIM) {
            std::cerr << "Gym: the registered " << Env::KERNEL << " has a different layout than this Env\n";
            std::exit(1);
        }
        mg::check(mg_gym_create(Env::KERNEL, parallels, seed, &handle), "Gym");
        mg::check(mg_gym_buffers_get(handle, &buffers), "Gym");
        actionHost.assign(parallels, Action{});
        obsHost.resize(parallels);
        doneHost.assign(parallels, 1);
        rewardHost.assign(parallels, 0.0f);
    }
    ~Gym() { mg_gym_destroy(handle); }
    Gym(const Gym&) = delete;
    Gym& operator=(const Gym&) = delete;

    // gym.h:86-88
    Action* actions() { return actionHost.data(); }
    uint8_t* done() {
        mg::check(mg_gym_sync(handle), "Gym::done");
        mg::check(mg_memcpy_d2h(doneHost.data(), buffers.done, parallels), "Gym::done");
        return doneHost.data();
    }
    Obs* obs() {
        mg::check(mg_gym_sync(handle), "Gym::obs");
        mg::check(mg_memcpy_d2h(obsHost.data(), buffers.obs, (size_t)parallels * sizeof(Obs)), "Gym::obs");
        return obsHost.data();
    }

    // gym.h:94-108 (encodeStep): one env step reading device actions and writing
    // device obs/reward, e.g. slot t of a rollout buffer. Asynchronous.
    void stepInto(const Action* actionsDev, Obs* obsDev, float* rewardDev) {
        mg::check(mg_gym_step_into(handle, actionsDev, reinterpret_cast<float*>(obsDev), rewardDev), "Gym::stepInto");
    }

    // gym.h:110-121: one blocking env step with actions(); rewards into `reward`.
    void run(std::vector<float>& reward) {
        mg::check(mg_memcpy_h2d(buffers.actions, actionHost.data(), (size_t)parallels * sizeof(Action)), "Gym::run");
        mg::check(mg_gym_run(handle), "Gym::run");
        mg::check(mg_gym_sync(handle), "Gym::run");
        const size_t count = reward.size() < parallels ? reward.size() : parallels;
        if (count) mg::check(mg_memcpy_d2h(reward.data(), buffers.reward, count * sizeof(float)), "Gym::run");
    }

    // T random-policy steps with [T][n] device slot outputs (any may be null).
    void rolloutRandom(uint32_t T, Action* actionsOut, Obs* obsOut, float* rewardOut, uint8_t* doneOut) {
        mg::check(mg_gym_rollout_random(handle, T, actionsOut, reinterpret_cast<float*>(obsOut), rewardOut, doneOut),
                  "Gym::rolloutRandom");
        mg::check(mg_gym_sync(handle), "Gym::rolloutRandom");
    }
};
