// PPOModel<Env> with the reference's API (model/ppo.h:106-1009), on the
// metalgym_amd C ABI: collect(), train(epochs), trainSlot(t), forward(),
// act(rng), actGreedy(), lastStats(), headValue(), logStdValue(), setLogStd(),
// values(), logProbs(), slot*() and the public hyperparameter fields.
//
// All device work runs in the library's kernels on the gym's stream. Host
// accessors return host mirrors that are refreshed lazily after each collect()
// or train(); their pointers stay valid until the model is destroyed.
#pragma once
#include <algorithm>
#include <cmath>
#include <random>
#include <type_traits>
#include <vector>

#include "gym.h"

struct LossStats {  // model/ppo.h:97-104
    float policy;
    float value;
    float entropy;
    float approxKl;
    float clipFrac;
    float gradNorm;
};

template <typename Env>
struct PPOModel {
    using Action = typename Env::Action;
    using Obs = typename Env::Obs;
    static constexpr bool CONTINUOUS = !std::is_integral_v<Action>;
    static_assert(sizeof(Obs) == Env::OBS_DIM * sizeof(float), "Env::Obs must be exactly OBS_DIM floats");
    static_assert(CONTINUOUS || sizeof(Action) == 4, "the softmax head needs a discrete 4-byte Action");
    static_assert(!CONTINUOUS || sizeof(Action) == Env::ACT_DIM * sizeof(float),
                  "the Gaussian head needs an Action of exactly ACT_DIM floats");
    static constexpr float INIT_LOG_STD = 0.0f;
    static constexpr uint32_t HEAD_DIM = Env::ACT_DIM + 1;  // logits or means, then the value
    static constexpr float kHalfLog2Pi = 0.9189385332046727f;  // ln(2 pi) / 2
    static_assert(Env::ACT_DIM + 1 <= 64, "ACT_DIM + value must fit a 64-wide head");

    Gym<Env>& gym;
    mg_ppo* handle = nullptr;
    uint32_t parallels, horizon;

    // model/ppo.h:186-191, read on every call
    float clip = 0.2f;
    float valueCoef = 0.5f;
    float entropyCoef = 0.01f;
    float maxGradNorm = 0.5f;  // 0 disables clipping
    float gamma = 0.99f;
    float lambda = 0.95f;

    // model/ppo.h:274. minibatch: rows per PPO minibatch (multiple of 64 dividing
    // the env count; 0 = min(envs, 4096), which is one whole slot at 4096 envs).
    // precision: MG_PRECISION_FP32, or MG_PRECISION_BF16 for bfloat16 matrix
    // operands in the policy forward (the reference's matmul precision).
    PPOModel(Gym<Env>& g, int e, int s, int layers, float learningRate, int T = 32, uint32_t seed = 0,
             uint32_t minibatch = 0, uint32_t precision = MG_PRECISION_FP32)
        : gym(g), parallels(g.parallels), horizon((uint32_t)(T > 0 ? T : 0)) {
        mg_ppo_config cfg{};
        cfg.embed = (uint32_t)e;
        cfg.scale = (uint32_t)s;
        cfg.layers = (uint32_t)(layers > 0 ? layers : 0);
        cfg.horizon = horizon;
        cfg.minibatch = minibatch;
        cfg.seed = seed;
        cfg.lr = learningRate;
        cfg.precision = precision;
        if (mg_ppo_check_config(Env::KERNEL, parallels, &cfg) != MG_OK) {  // model/ppo.h:290-298
            std::cerr << mg_last_error() << "\n";
            std::exit(1);
        }
        mg::check(mg_ppo_create(gym.handle, &cfg, &handle), "PPOModel");
        mg::check(mg_ppo_slots_get(handle, &slots_), "PPOModel");
        mg::check(mg_ppo_policy(handle, &policy_), "PPOModel");
        valueHost.assign(parallels, 0.0f);
        logProbHost.assign(parallels, 0.0f);
    }
    ~PPOModel() { mg_ppo_destroy(handle); }
    PPOModel(const PPOModel&) = delete;
    PPOModel& operator=(const PPOModel&) = delete;

    // model/ppo.h:716-751: T env steps + GAE, one launch sequence, blocking.
    void collect() {
        pushHParams();
        mg::check(mg_ppo_collect(handle), "collect");
        slotsFresh_ = headFresh_ = false;
    }
    // model/ppo.h:918-923
    void train(uint32_t epochs = 4) {
        pushHParams();
        mg::check(mg_ppo_train(handle, epochs), "train");
        headFresh_ = paramsFresh_ = false;
    }
    // model/ppo.h:906-916: the minibatches of slot t, in row order.
    void trainSlot(uint32_t t) {
        pushHParams();
        const uint32_t per = parallels / minibatchRows();
        for (uint32_t b = 0; b < per; ++b) mg::check(mg_ppo_train_block(handle, t * per + b), "trainSlot");
        headFresh_ = paramsFresh_ = false;
    }
    // model/ppo.h:628-634: policy forward on gym.obs().
    void forward() {
        mg::check(mg_ppo_forward(handle, gym.buffers.obs, parallels), "forward");
        headFresh_ = false;
    }

    // model/ppo.h:636-684: host-side sampling from the last head into
    // gym.actions(), logProbs() and values(). The caller's generator is drawn
    // in row order: one uniform per row for a discrete Action (inverse CDF of
    // the softmax), one standard normal per action dimension for a float
    // Action (mean + exp(log_std) z), as the reference draws it.
    template <typename Rng>
    void act(Rng& rng) {
        const float* head = headHost();
        if constexpr (CONTINUOUS) {
            std::normal_distribution<float> stdNormal(0.0f, 1.0f);
            float logStd[Env::ACT_DIM];
            for (uint32_t k = 0; k < Env::ACT_DIM; ++k) logStd[k] = logStdValue(k);
            float* out = reinterpret_cast<float*>(gym.actions());
            for (uint32_t row = 0; row < parallels; ++row, out += Env::ACT_DIM) {
                const float* mean = head + (size_t)row * HEAD_DIM;
                float logDensity = 0.0f;
                for (uint32_t k = 0; k < Env::ACT_DIM; ++k) {
                    out[k] = mean[k] + std::exp(logStd[k]) * stdNormal(rng);
                    const float z = (out[k] - mean[k]) * std::exp(-logStd[k]);  // the draw, recovered from the action
                    logDensity += -0.5f * z * z - logStd[k] - kHalfLog2Pi;
                }
                logProbHost[row] = logDensity;
                valueHost[row] = mean[Env::ACT_DIM];
            }
        } else {
            std::uniform_real_distribution<float> unit(0.0f, 1.0f);
            float weight[Env::ACT_DIM];
            for (uint32_t row = 0; row < parallels; ++row) {
                const float* logit = head + (size_t)row * HEAD_DIM;
                const float top = *std::max_element(logit, logit + Env::ACT_DIM);
                float total = 0.0f;
                for (uint32_t a = 0; a < Env::ACT_DIM; ++a) total += (weight[a] = std::exp(logit[a] - top));
                // the first action whose cumulative weight exceeds u * total (the last if none does)
                const float target = unit(rng) * total;
                uint32_t pick = 0;
                for (float cum = weight[0]; pick + 1 < Env::ACT_DIM && !(target < cum); cum += weight[++pick]) {
                }
                gym.actions()[row] = (Action)pick;
                logProbHost[row] = logit[pick] - (top + std::log(total));
                valueHost[row] = logit[Env::ACT_DIM];
            }
        }
    }
    // model/ppo.h:686-702: the most probable action (the first of equal ones), or the mean.
    void actGreedy() {
        const float* head = headHost();
        for (uint32_t row = 0; row < parallels; ++row) {
            const float* h = head + (size_t)row * HEAD_DIM;
            if constexpr (CONTINUOUS)
                std::copy(h, h + Env::ACT_DIM, reinterpret_cast<float*>(gym.actions()) + (size_t)row * Env::ACT_DIM);
            else
                gym.actions()[row] = (Action)(std::max_element(h, h + Env::ACT_DIM) - h);
        }
    }

    // model/ppo.h:925-943
    LossStats lastStats() const {
        mg_loss_stats s{};
        mg::check(mg_ppo_last_stats(handle, &s), "lastStats");
        return LossStats{s.policy, s.value, s.entropy, s.approx_kl, s.clip_frac, s.grad_norm};
    }
    // LossStats of every minibatch of the last train() call.
    std::vector<LossStats> trainStats() const {
        uint32_t count = 0;
        mg::check(mg_ppo_train_stats(handle, nullptr, 0, &count), "trainStats");
        std::vector<mg_loss_stats> raw(count);
        mg::check(mg_ppo_train_stats(handle, raw.data(), count, &count), "trainStats");
        std::vector<LossStats> out;
        for (auto& s : raw) out.push_back({s.policy, s.value, s.entropy, s.approx_kl, s.clip_frac, s.grad_norm});
        return out;
    }

    // model/ppo.h:448-476
    float* values() { return valueHost.data(); }
    float* logProbs() { return logProbHost.data(); }
    float headValue(uint32_t row, uint32_t col) { return headHost()[(size_t)row * HEAD_DIM + col]; }
    float logStdValue(uint32_t k) {
        static_assert(CONTINUOUS, "logStdValue needs a continuous Env::Action");
        if (!paramsFresh_) {
            logStdHost.resize(Env::ACT_DIM);
            mg::check(mg_memcpy_d2h(logStdHost.data(), policy_.params + policy_.off_log_std, Env::ACT_DIM * 4),
                      "logStdValue");
            paramsFresh_ = true;
        }
        return logStdHost[k];
    }
    void setLogStd(float value) {
        static_assert(CONTINUOUS, "setLogStd needs a continuous Env::Action");
        mg::check(mg_ppo_set_log_std(handle, value), "setLogStd");
        paramsFresh_ = false;
    }
    Obs* slotObs(uint32_t t) { return reinterpret_cast<Obs*>(slot().obs.data()) + (size_t)t * parallels; }
    Action* slotActions(uint32_t t) { return slot().actions.data() + (size_t)t * parallels; }
    float* slotRewards(uint32_t t) { return slot().reward.data() + (size_t)t * parallels; }
    uint8_t* slotDones(uint32_t t) { return slot().done.data() + (size_t)t * parallels; }
    float* slotValues(uint32_t t) { return slot().value.data() + (size_t)t * parallels; }
    float* slotAdvantages(uint32_t t) { return slot().adv.data() + (size_t)t * parallels; }
    float* slotReturns(uint32_t t) { return slot().ret.data() + (size_t)t * parallels; }

    // Rows per PPO minibatch after defaulting (the reference trains one slot per minibatch).
    uint32_t minibatchRows() const {
        mg_ppo_config cfg{};
        mg::check(mg_ppo_config_get(handle, &cfg), "minibatchRows");
        return cfg.minibatch;
    }

   private:
    struct SlotMirror {
        std::vector<float> obs, reward, value, adv, ret;
        std::vector<Action> actions;
        std::vector<uint8_t> done;
    };
    mg_ppo_slots slots_{};
    mg_policy_view policy_{};
    SlotMirror mirror_;
    std::vector<float> headHost_, logStdHost;
    std::vector<float> valueHost, logProbHost;
    bool slotsFresh_ = false, headFresh_ = false, paramsFresh_ = false;

    void pushHParams() {
        mg_ppo_hparams hp{clip, valueCoef, entropyCoef, maxGradNorm, gamma, lambda};
        mg::check(mg_ppo_set_hparams(handle, &hp), "hyperparameters");
    }
    const float* headHost() {
        if (!headFresh_) {
            const float* dev = nullptr;
            uint32_t rows = 0, hd = 0;
            mg::check(mg_ppo_head(handle, &dev, &rows, &hd), "head");
            headHost_.resize((size_t)rows * hd);
            if (rows) mg::check(mg_memcpy_d2h(headHost_.data(), dev, headHost_.size() * 4), "head");
            headFresh_ = true;
        }
        return headHost_.data();
    }
    SlotMirror& slot() {
        if (!slotsFresh_) {
            const size_t n = parallels, T = horizon;
            auto get = [&](auto& v, const void* src, size_t count) {
                v.resize(count);
                mg::check(mg_memcpy_d2h(v.data(), src, count * sizeof(v[0])), "slot download");
            };
            get(mirror_.obs, slots_.obs, (T + 1) * n * Env::OBS_DIM);
            get(mirror_.actions, slots_.actions, T * n);
            get(mirror_.reward, slots_.reward, T * n);
            get(mirror_.done, slots_.done, T * n);
            get(mirror_.value, slots_.value, T * n);
            get(mirror_.adv, slots_.advantage, T * n);
            get(mirror_.ret, slots_.ret, T * n);
            slotsFresh_ = true;
        }
        return mirror_;
    }
};
