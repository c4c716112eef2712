// End-to-end check of the C++ API surface (Gym<Env>, PPOModel<Env>) on the
// GPU: every public call of the reference's API runs once and its result is
// checked for the invariants the reference documents (README.md:100-156).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>

#include "mg/envs/cartpole.h"
#include "mg/envs/cartpole_continuous.h"
#include "mg/ppo.h"

static int failures = 0;
#define CHECK(cond)                                                        \
    do {                                                                   \
        if (!(cond)) {                                                     \
            std::printf("FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                    \
        }                                                                  \
    } while (0)

int main() {
    const uint32_t N = 256, T = 8;
    {  // Gym::stepInto (gym.h:94-108) into slot t of device buffers gives the same
        // steps as Gym::run with the same actions
        const uint32_t S = 40;
        Gym<CartPole> a(N), b(N);
        std::vector<int> acts((size_t)S * N);
        std::mt19937 gen(5);
        for (auto& x : acts) x = (int)(gen() & 1u);
        void *dAct = nullptr, *dObs = nullptr, *dRew = nullptr;
        CHECK(mg_malloc(&dAct, acts.size() * sizeof(int)) == MG_OK);
        CHECK(mg_malloc(&dObs, acts.size() * sizeof(CartPole::Obs)) == MG_OK);
        CHECK(mg_malloc(&dRew, acts.size() * sizeof(float)) == MG_OK);
        CHECK(mg_memcpy_h2d(dAct, acts.data(), acts.size() * sizeof(int)) == MG_OK);
        for (uint32_t t = 0; t < S; t++)
            a.stepInto(static_cast<const int*>(dAct) + (size_t)t * N, static_cast<CartPole::Obs*>(dObs) + (size_t)t * N,
                       static_cast<float*>(dRew) + (size_t)t * N);
        CHECK(mg_gym_sync(a.handle) == MG_OK);
        std::vector<CartPole::Obs> obs(acts.size());
        std::vector<float> rew(acts.size());
        CHECK(mg_memcpy_d2h(obs.data(), dObs, obs.size() * sizeof(CartPole::Obs)) == MG_OK);
        CHECK(mg_memcpy_d2h(rew.data(), dRew, rew.size() * sizeof(float)) == MG_OK);
        std::vector<float> r(N);
        uint32_t ended = 0;
        for (uint32_t t = 0; t < S; t++) {
            for (uint32_t i = 0; i < N; i++) b.actions()[i] = acts[(size_t)t * N + i];
            b.run(r);
            CHECK(std::memcmp(b.obs(), &obs[(size_t)t * N], N * sizeof(CartPole::Obs)) == 0);
            CHECK(std::memcmp(r.data(), &rew[(size_t)t * N], N * sizeof(float)) == 0);
            const uint8_t* db = b.done();
            for (uint32_t i = 0; i < N; i++) ended += db[i];
        }
        CHECK(std::memcmp(a.done(), b.done(), N) == 0);
        CHECK(ended > 0);  // resets happened between the steps
        mg_free(dAct);
        mg_free(dObs);
        mg_free(dRew);
    }
    {
        Gym<CartPole> gym(N);
        const uint8_t* d0 = gym.done();
        for (uint32_t i = 0; i < N; i++) CHECK(d0[i] == 1);  // gym.h:54-55
        std::vector<float> reward(N, 0.0f);
        for (uint32_t i = 0; i < N; i++) gym.actions()[i] = (int)(i & 1);
        gym.run(reward);
        const CartPole::Obs* o = gym.obs();
        for (uint32_t i = 0; i < N; i++) {
            CHECK(reward[i] == 1.0f);
            CHECK(std::fabs(o[i].x) < 0.06f && std::fabs(o[i].theta) < 0.06f);
        }
        PPOModel<CartPole> model(gym, 128, 4, 2, 3e-4f, T);
        CHECK(model.minibatchRows() == N);
        model.collect();
        for (uint32_t t = 0; t < T; t++) {
            for (uint32_t i = 0; i < N; i++) {
                CHECK(model.slotRewards(t)[i] == 1.0f);
                CHECK(model.slotActions(t)[i] == 0 || model.slotActions(t)[i] == 1);
                CHECK(model.slotReturns(t)[i] == model.slotAdvantages(t)[i] + model.slotValues(t)[i]);
                CHECK(std::isfinite(model.slotValues(t)[i]));
            }
        }
        // bootstrap value = head column ACT_DIM of the last forward (model/gae.metal:27)
        const float vT = model.headValue(0, CartPole::ACT_DIM);
        CHECK(model.slotReturns(T - 1)[0] == model.slotAdvantages(T - 1)[0] + model.slotValues(T - 1)[0]);
        CHECK(std::isfinite(vT));
        model.forward();
        std::mt19937 rng(1);
        model.act(rng);
        uint32_t ones = 0;
        for (uint32_t i = 0; i < N; i++) {
            const int a = gym.actions()[i];
            CHECK(a == 0 || a == 1);
            ones += (uint32_t)a;
            CHECK(model.values()[i] == model.headValue(i, CartPole::ACT_DIM));
            // log-probability of the chosen action under the softmax of the head
            const double z0 = model.headValue(i, 0), z1 = model.headValue(i, 1);
            const double m = z0 > z1 ? z0 : z1;
            const double lse = m + std::log(std::exp(z0 - m) + std::exp(z1 - m));
            CHECK(std::fabs(model.logProbs()[i] - ((a ? z1 : z0) - lse)) < 1e-5);
        }
        CHECK(ones > N / 4 && ones < 3 * N / 4);  // the initial policy is close to uniform
        model.actGreedy();
        for (uint32_t i = 0; i < N; i++) {
            const int best = model.headValue(i, 1) > model.headValue(i, 0) ? 1 : 0;
            CHECK(gym.actions()[i] == best);
        }
        model.train(1);
        LossStats s = model.lastStats();
        CHECK(std::isfinite(s.policy) && std::isfinite(s.value) && s.gradNorm > 0.0f);
        CHECK(s.entropy > 0.6f && s.entropy <= 0.6932f);
        CHECK(model.trainStats().size() == T);
        model.trainSlot(3);
        CHECK(model.trainStats().size() == 1);
        model.clip = 0.1f;
        model.collect();
        model.train(1);
        CHECK(std::isfinite(model.lastStats().gradNorm));
    }
    {
        Gym<CartPoleContinuous> gym(N);
        PPOModel<CartPoleContinuous> model(gym, 128, 4, 2, 3e-4f, T);
        CHECK(model.logStdValue(0) == 0.0f);  // model/ppo.h:115
        model.setLogStd(-0.5f);
        CHECK(model.logStdValue(0) == -0.5f);
        model.collect();
        model.train(1);
        LossStats s = model.lastStats();
        CHECK(std::isfinite(s.policy) && s.gradNorm > 0.0f);
        CHECK(model.logStdValue(0) != -0.5f);  // Adam moved it
        std::mt19937 rng(2);
        model.forward();
        model.act(rng);
        // (action - mean) / std is the standard normal draw: sample moments over N rows
        double s1 = 0.0, s2 = 0.0;
        const float sd = std::exp(model.logStdValue(0));
        for (uint32_t i = 0; i < N; i++) {
            CHECK(std::isfinite(gym.actions()[i].force));
            const double z = (gym.actions()[i].force - model.headValue(i, 0)) / sd;
            s1 += z;
            s2 += z * z;
            const double lp = -0.5 * z * z - std::log(sd) - 0.5 * std::log(2.0 * M_PI);
            CHECK(std::fabs(model.logProbs()[i] - lp) < 1e-4);
        }
        CHECK(std::fabs(s1 / N) < 4.0 / std::sqrt((double)N));
        CHECK(std::fabs(s2 / N - 1.0) < 4.0 * std::sqrt(2.0 / N));
        model.actGreedy();
        for (uint32_t i = 0; i < N; i++) CHECK(gym.actions()[i].force == model.headValue(i, 0));
    }
    std::printf(failures ? "api_check FAILED (%d)\n" : "api_check ok\n", failures);
    return failures ? 1 : 0;
}
