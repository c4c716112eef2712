// CartPole with one float action (examples/CartPoleContinuous/cartpole_continuous.metal:7-78).
// The force is 10 * tanh(a). The reference clamps to [-1, 1] instead
// (cartpole_continuous.metal:57); CartPoleContinuousClamp keeps that variant.
#pragma once
#include "cartpole.h"

struct CartPoleContinuous {
    using State = CartPole::State;
    struct Action {
        float force;  // unbounded Gaussian sample, squashed in step()
    };
    using Obs = CartPole::Obs;

    static constexpr uint32_t OBS_DIM = 4;
    static constexpr uint32_t ACT_DIM = 1;
    static constexpr const char* KERNEL = "rollout_cartpole_continuous";

    MG_HD static void reset(State& s, uint32_t& rng) { CartPole::reset(s, rng); }

    MG_HD static void step(State& s, Action action, Obs& obs, float& reward, uint8_t& done) {
        float force = CartPole::FORCE_MAG * mg::tanhf(action.force);
        CartPole::integrate(s, force, obs, reward, done);
    }
};

struct CartPoleContinuousClamp {
    using State = CartPole::State;
    using Action = CartPoleContinuous::Action;
    using Obs = CartPole::Obs;

    static constexpr uint32_t OBS_DIM = 4;
    static constexpr uint32_t ACT_DIM = 1;
    static constexpr const char* KERNEL = "rollout_cartpole_continuous_clamp";

    MG_HD static void reset(State& s, uint32_t& rng) { CartPole::reset(s, rng); }

    MG_HD static void step(State& s, Action action, Obs& obs, float& reward, uint8_t& done) {
        float a = action.force < -1.0f ? -1.0f : (action.force > 1.0f ? 1.0f : action.force);
        CartPole::integrate(s, a * CartPole::FORCE_MAG, obs, reward, done);
    }
};
