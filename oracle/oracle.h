/*
 * TEST INFRASTRUCTURE ONLY. This is the CPU oracle: a scalar C++ restatement
 * of MetalGym's rollout-and-policy algorithm, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker.
 * The product (libmetalgym_amd.so) never links, loads or calls it.
 *
 * Each function cites the reference file:line it restates. Every function is
 * pinned by a check independent of its own loops (known answers, closed forms,
 * textbook equations, torch float64 fixtures, replays composed of separately
 * pinned pieces; tests/test_cpu_oracle.py, tests/test_cpu_sampling.py,
 * tests/test_cpu_voxelnav.py), and tests/test_cpu_oracle_mutants.py shows the
 * sampler and collect pins reject planted slips. Deliberate
 * differences from the reference (fp32 instead of bf16 storage, the seed hash,
 * uniform init, contiguous minibatch blocks, tanh force) are the build-defined
 * semantics the product implements too.
 */
#ifndef MG_ORACLE_H
#define MG_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* env ids */
enum { ORC_CARTPOLE = 0, ORC_CARTPOLE_CONT = 1, ORC_CARTPOLE_CONT_CLAMP = 2, ORC_VOXELNAV16 = 3, ORC_VOXELNAV = 4 };

typedef struct orc_env_info {
    uint32_t state_bytes;
    uint32_t action_bytes;
    uint32_t obs_dim;
    uint32_t act_dim;
    uint32_t continuous;
} orc_env_info;

typedef struct orc_dims {
    uint32_t obs_dim;
    uint32_t act_dim;
    uint32_t embed;
    uint32_t hidden;
    uint32_t layers;
    uint32_t continuous;
    uint32_t bf16; /* 1: the block GEMMs of the forward take bfloat16 operands */
} orc_dims;

typedef struct orc_layout {
    uint32_t count;
    uint32_t float_group;
    uint32_t head_dim;
    uint32_t off_in_w, off_in_b;
    uint32_t off_ln_gamma[9], off_ln_beta[9];
    uint32_t off_up[8], off_down[8];
    uint32_t off_head, off_log_std;
} orc_layout;

typedef struct orc_hparams {
    float clip, value_coef, entropy_coef, max_grad_norm, gamma, lambda, lr;
} orc_hparams;

typedef struct orc_stats {
    float policy, value, entropy, approx_kl, clip_frac, grad_norm;
} orc_stats;

/* rollout.h:9-29 */
uint32_t orc_rng_next(uint32_t* s);
float orc_rng_uniform(uint32_t* s);
float orc_rng_uniform_range(uint32_t* s, float lo, float hi);
uint32_t orc_rng_int(uint32_t* s, uint32_t n);
/* gym.h:54-61 (+ seed hash) */
void orc_gym_init(int env, uint32_t n, uint32_t seed, void* state, uint32_t* rng, uint8_t* done, void* actions);

int orc_env_info_get(int env, orc_env_info* out);
void orc_env_reset(int env, void* state, uint32_t* rng);
void orc_env_step(int env, void* state, const void* action, float* obs, float* reward, uint8_t* done);

/* rollout.h:31-54 applied `steps` times; random actions drawn before the reset. */
void orc_rollout(int env, uint32_t n, uint32_t steps, int random, void* state, uint32_t* rng, uint8_t* done,
                 const void* actions_in, void* actions_out, float* obs_out, float* reward_out, uint8_t* done_out,
                 int threads);

/* math shared with the product (include/mg/math.h), exported for pinning tests */
float orc_round_bf16(float x); /* bfloat16 rounding (nearest, ties to even) */
float orc_expf(float x);
float orc_logf(float x);
float orc_sinf(float x);
float orc_cosf(float x);
float orc_tanhf(float x);

/* parameters: model/ppo.h:375-423 (layout), D2 init */
int orc_layout_get(const orc_dims* d, orc_layout* out);
void orc_init_params(const orc_dims* d, uint32_t seed, float* params);
uint64_t orc_splitmix_next(uint64_t* state);

/* model/ppo.h:575-626 forward over rows; head [rows][act+1] */
void orc_forward(const orc_dims* d, const float* params, const float* obs, uint32_t rows, float* head, int threads);

/* model/sample.metal:18-47 / model/gaussian.metal:42-71 */
void orc_sample(const orc_dims* d, const float* params, const float* head, uint32_t rows, uint32_t* rng,
                void* actions, float* logp, float* value);

/* model/gae.metal:14-36 */
void orc_gae(const float* reward, const uint8_t* done, const float* value, const float* head, uint32_t head_dim,
             uint32_t act_dim, uint32_t n, uint32_t horizon, float gamma, float lambda, float* adv, float* ret);

/* model/ppo.h:716-751 plus GAE. teacher_actions ([T][n], nullable): when given,
 * each env steps with the teacher's action instead of its own sample (the sample
 * is still drawn, so RNG streams stay aligned); sampled_actions ([T][n],
 * nullable) receives the oracle's own sampled actions. */
void orc_collect(int env, const orc_dims* d, const float* params, uint32_t n, uint32_t horizon, int first,
                 float gamma, float lambda, void* state, uint32_t* rng, uint8_t* done, float* obs_slots,
                 void* action_slots, float* logp_slots, float* value_slots, float* reward_slots,
                 uint8_t* done_slots, float* adv_slots, float* ret_slots, float* head_out,
                 const void* teacher_actions, void* sampled_actions, int threads);

/* One minibatch: forward, model/gae.metal:42-77 normalisation, loss
 * (model/policy.metal:14-69 or model/gaussian.metal:76-135), backward
 * (model/ppo.h:793-865), global grad norm and Adam (model/optimizer.metal:23-60).
 * Updates params, m, v in place; writes the gradient (pre-clip) to grad if not NULL. */
void orc_train_minibatch(const orc_dims* d, const orc_hparams* hp, float* params, float* m, float* v,
                         uint32_t step, uint32_t rows, const float* obs, const void* actions, const float* adv,
                         const float* ret, const float* old_logp, float* grad, orc_stats* stats, float* head_out,
                         int threads);

/* orc_train_minibatch with the forward's ReLU decisions given: relu_mask
 * ([rows][layers][hidden], 1 = the unit passes its pre-activation, nullable)
 * replaces the test z > 0 in the forward and in the backward's mask, so the
 * oracle evaluates the same piecewise-linear function as a run whose
 * summation order put a pre-activation within rounding of 0 on the other side.
 * preact_out ([rows][layers][hidden], nullable) receives the pre-activations. */
void orc_train_minibatch_masked(const orc_dims* d, const orc_hparams* hp, float* params, float* m, float* v,
                                uint32_t step, uint32_t rows, const float* obs, const void* actions, const float* adv,
                                const float* ret, const float* old_logp, float* grad, orc_stats* stats,
                                float* head_out, const uint8_t* relu_mask, float* preact_out, int threads);

/* This build's minibatch order (the reference has no random-access minibatch
 * order of its own at n > 4096): per epoch a Fisher-Yates shuffle of the
 * block ids driven by the model's SplitMix64 shuffle stream. */
void orc_shuffle_state_init(uint32_t seed, uint64_t* state);
void orc_shuffle_blocks(uint64_t* state, uint32_t* order, uint32_t count);

/* model/ppo.h:918-923: epochs over the slots; per-minibatch stats in stats_out
 * (epochs * blocks entries). order_inout is the model's persistent block order
 * (slotOrder, model/ppo.h:347-348), shuffled in place at each epoch. */
void orc_train(const orc_dims* d, const orc_hparams* hp, float* params, float* m, float* v, uint32_t* step,
               uint64_t* shuffle_state, uint32_t n, uint32_t horizon, uint32_t minibatch, uint32_t epochs,
               const float* obs_slots, const void* action_slots, const float* adv_slots, const float* ret_slots,
               const float* logp_slots, orc_stats* stats_out, uint32_t* order_inout, int threads);

#ifdef __cplusplus
}
#endif
#endif
