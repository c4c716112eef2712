// CartPole (Barto, Sutton & Anderson 1983; Gymnasium CartPole-v1 constants).
// Behaviour follows examples/CartPole/cartpole.metal:5-76: four uniform
// [-0.05, 0.05) reset draws, semi-implicit Euler with tau 0.02, termination at
// |x| > 2.4 or |theta| > 12 degrees, truncation at 500 steps, reward 1 per step.
// The arithmetic keeps the reference's operation order so that host and device
// builds (both -ffp-contract=off) give identical bits.
#pragma once
#include "../env.h"

struct CartPole {
    struct State {
        float x;
        float xDot;
        float theta;
        float thetaDot;
        uint32_t steps;
    };
    using Action = int;  // 0 = push left, 1 = push right
    struct Obs {
        float x;
        float xDot;
        float theta;
        float thetaDot;
    };

    static constexpr uint32_t OBS_DIM = 4;
    static constexpr uint32_t ACT_DIM = 2;
    static constexpr const char* KERNEL = "rollout_cartpole";

    static constexpr float GRAVITY = 9.8f;
    static constexpr float MASS_CART = 1.0f;
    static constexpr float MASS_POLE = 0.1f;
    static constexpr float TOTAL_MASS = MASS_CART + MASS_POLE;
    static constexpr float LENGTH = 0.5f;  // half the pole length
    static constexpr float POLE_MASS_LENGTH = MASS_POLE * LENGTH;
    static constexpr float FORCE_MAG = 10.0f;
    static constexpr float TAU = 0.02f;
    static constexpr float PI_F = 3.14159265358979323846f;
    static constexpr float THETA_THRESHOLD = 12.0f * 2.0f * PI_F / 360.0f;
    static constexpr float X_THRESHOLD = 2.4f;
    static constexpr uint32_t MAX_STEPS = 500;

    MG_HD static void reset(State& s, uint32_t& rng) {
        s.x = rngUniform(rng, -0.05f, 0.05f);
        s.xDot = rngUniform(rng, -0.05f, 0.05f);
        s.theta = rngUniform(rng, -0.05f, 0.05f);
        s.thetaDot = rngUniform(rng, -0.05f, 0.05f);
        s.steps = 0;
    }

    // Shared by CartPole and CartPoleContinuous: one Euler step under `force`.
    MG_HD static void integrate(State& s, float force, Obs& obs, float& reward, uint8_t& done) {
        float sinTheta, cosTheta;
        mg::sincosf(s.theta, &sinTheta, &cosTheta);  // the bits of mg::sinf and mg::cosf, one reduction
        float temp = (force + POLE_MASS_LENGTH * s.thetaDot * s.thetaDot * sinTheta) / TOTAL_MASS;
        float thetaAcc = (GRAVITY * sinTheta - cosTheta * temp) /
                         (LENGTH * (4.0f / 3.0f - MASS_POLE * cosTheta * cosTheta / TOTAL_MASS));
        float xAcc = temp - POLE_MASS_LENGTH * thetaAcc * cosTheta / TOTAL_MASS;

        s.x += TAU * s.xDot;
        s.xDot += TAU * xAcc;
        s.theta += TAU * s.thetaDot;
        s.thetaDot += TAU * thetaAcc;
        s.steps += 1;

        bool terminated = (s.x < 0.0f ? -s.x : s.x) > X_THRESHOLD ||
                          (s.theta < 0.0f ? -s.theta : s.theta) > THETA_THRESHOLD;
        bool truncated = s.steps >= MAX_STEPS;

        obs.x = s.x;
        obs.xDot = s.xDot;
        obs.theta = s.theta;
        obs.thetaDot = s.thetaDot;
        reward = 1.0f;  // 1 on every step, including the terminal one
        done = (terminated || truncated) ? 1 : 0;
    }

    MG_HD static void step(State& s, Action action, Obs& obs, float& reward, uint8_t& done) {
        float force = (action == 1) ? FORCE_MAG : -FORCE_MAG;
        integrate(s, force, obs, reward, done);
    }
};
