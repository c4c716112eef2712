// Drives every entry point of the CPU oracle at small sizes, for every env,
// both precisions and several thread counts, so that a build with
// AddressSanitizer + UndefinedBehaviorSanitizer or ThreadSanitizer checks the
// checker itself (out-of-bounds accesses, undefined arithmetic, races between
// its env-shard and row-shard threads). Exits non-zero if an output is not
// finite.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../oracle/oracle.h"

namespace {

int failures = 0;

void expect_finite(const std::vector<float>& v, const char* what, int env) {
    for (float x : v)
        if (!std::isfinite(x)) {
            std::fprintf(stderr, "env %d: non-finite value in %s\n", env, what);
            ++failures;
            return;
        }
}

void drive_env(int env, uint32_t hidden, uint32_t layers, uint32_t bf16, int threads) {
    orc_env_info info;
    if (orc_env_info_get(env, &info) != 0) {
        std::fprintf(stderr, "env %d: no info\n", env);
        ++failures;
        return;
    }
    const uint32_t n = 64, T = 2, steps = 20, O = info.obs_dim, A = info.act_dim;
    const uint32_t act_words = info.continuous ? A : 1;
    std::vector<uint8_t> state((size_t)n * info.state_bytes), done(n);
    std::vector<uint32_t> rng(n), actions((size_t)n * act_words);
    orc_gym_init(env, n, 7, state.data(), rng.data(), done.data(), actions.data());

    // random and given-action rollouts
    std::vector<uint32_t> acts((size_t)steps * n * act_words);
    std::vector<float> obs((size_t)steps * n * O), rew((size_t)steps * n);
    std::vector<uint8_t> dn((size_t)steps * n);
    orc_rollout(env, n, steps, 1, state.data(), rng.data(), done.data(), nullptr, acts.data(), obs.data(),
                rew.data(), dn.data(), threads);
    orc_rollout(env, n, steps, 0, state.data(), rng.data(), done.data(), acts.data(), nullptr, obs.data(),
                rew.data(), dn.data(), threads);
    expect_finite(obs, "rollout obs", env);

    // parameters, forward on a ragged row count, sampling
    orc_dims d{O, A, 128, hidden, layers, info.continuous, bf16};
    orc_layout lay;
    orc_layout_get(&d, &lay);
    std::vector<float> params(lay.count), m(lay.count), v(lay.count), grad(lay.count);
    orc_init_params(&d, 3, params.data());
    const uint32_t rows = 37;
    std::vector<float> head((size_t)rows * (A + 1)), logp(rows), value(rows);
    std::vector<uint32_t> srng(rows, 12345u), sacts((size_t)rows * act_words);
    orc_forward(&d, params.data(), obs.data(), rows, head.data(), threads);
    orc_sample(&d, params.data(), head.data(), rows, srng.data(), sacts.data(), logp.data(), value.data());
    expect_finite(head, "forward head", env);

    // two collects (the first takes the extra step), GAE inside
    std::vector<float> obs_slots((size_t)(T + 1) * n * O), logp_slots((size_t)T * n), value_slots((size_t)T * n);
    std::vector<float> reward_slots((size_t)T * n), adv((size_t)T * n), ret((size_t)T * n), boot((size_t)n * (A + 1));
    std::vector<uint32_t> action_slots((size_t)T * n * act_words), sampled((size_t)T * n * act_words);
    std::vector<uint8_t> done_slots((size_t)T * n);
    for (int c = 0; c < 2; ++c)
        orc_collect(env, &d, params.data(), n, T, c == 0, 0.99f, 0.95f, state.data(), rng.data(), done.data(),
                    obs_slots.data(), action_slots.data(), logp_slots.data(), value_slots.data(), reward_slots.data(),
                    done_slots.data(), adv.data(), ret.data(), boot.data(), nullptr, sampled.data(), threads);
    orc_gae(reward_slots.data(), done_slots.data(), value_slots.data(), boot.data(), A + 1, A, n, T, 0.99f, 0.95f,
            adv.data(), ret.data());
    expect_finite(adv, "advantages", env);

    // one minibatch, then two shuffled epochs of 64-row minibatches
    orc_hparams hp{0.2f, 0.5f, 0.01f, 0.5f, 0.99f, 0.95f, 3e-4f};
    orc_stats st;
    std::vector<float> mb_head((size_t)64 * (A + 1));
    orc_train_minibatch(&d, &hp, params.data(), m.data(), v.data(), 1, 64, obs_slots.data(), action_slots.data(),
                        adv.data(), ret.data(), logp_slots.data(), grad.data(), &st, mb_head.data(), threads);
    expect_finite(grad, "gradient", env);
    const uint32_t B = 64, epochs = 2, blocks = T * n / B;
    uint64_t shuffle;
    orc_shuffle_state_init(5, &shuffle);
    std::vector<uint32_t> order(blocks);
    for (uint32_t b = 0; b < blocks; ++b) order[b] = b;
    std::vector<orc_stats> stats((size_t)epochs * blocks);
    uint32_t step = 1;
    orc_train(&d, &hp, params.data(), m.data(), v.data(), &step, &shuffle, n, T, B, epochs, obs_slots.data(),
              action_slots.data(), adv.data(), ret.data(), logp_slots.data(), stats.data(), order.data(), threads);
    expect_finite(params, "parameters after training", env);
}

}  // namespace

int main() {
    for (int env = ORC_CARTPOLE; env <= ORC_VOXELNAV; ++env)
        for (uint32_t bf16 = 0; bf16 <= 1; ++bf16) drive_env(env, 128, 2, bf16, 1 + env % 3);
    drive_env(ORC_CARTPOLE, 128, 8, 0, 4);  // the most blocks
    drive_env(ORC_CARTPOLE, 512, 1, 1, 2);  // a wider hidden layer
    std::printf("oracle driver: %d failures\n", failures);
    return failures ? 1 : 0;
}
