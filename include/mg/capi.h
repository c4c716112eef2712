/*
 * metalgym_amd C ABI: the drop-in boundary for MetalGym's rollout-and-policy
 * hot path on one AMD Instinct MI355X (gfx950).
 *
 * Every entry point takes plain pointers, sizes and POD structs and returns an
 * int status (MG_OK == 0, negative on error; mg_last_error() has the message).
 * Device pointers are HIP device allocations. Nothing here exits the process:
 * the reference prints to stderr and calls std::exit(1) on a bad configuration
 * (gym.h:65-69; model/ppo.h:290-298); the C++ layer (mg/gym.h, mg/ppo.h) keeps
 * that visible behaviour on top of these status codes.
 *
 * Calls are not thread-safe, as in the reference. Work is enqueued on the
 * gym's HIP stream; functions documented as blocking wait for it, matching the
 * reference, where every public call waits for its command buffer
 * (model/ppo.h:507-515, 749, 914; gym.h:115-116).
 */
#ifndef MG_CAPI_H
#define MG_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MG_ABI_VERSION 4
#define MG_MAX_LAYERS 8
#define MG_EMBED 128 /* the reference's N_EMBED_CFG (model/config.h:7) */

enum {
    MG_OK = 0,
    MG_ERR_INVALID = -1,   /* bad argument or configuration */
    MG_ERR_NOT_FOUND = -2, /* unknown env kernel name */
    MG_ERR_HIP = -3,       /* a HIP runtime call failed */
    MG_ERR_OOM = -4,       /* device allocation failed */
    MG_ERR_STATE = -5      /* call not valid in the object's current state */
};

/* Message of the last failing call on this thread ("" if none). */
const char* mg_last_error(void);
int mg_abi_version(void);

/* ---------------------------------------------------------------------------
 * Memory helpers. The reference keeps every buffer in Apple shared memory
 * (gym.h:46-51; model/ppo.h:493-495); on a discrete GPU the C++ layer mirrors
 * host-visible buffers explicitly with these copies.
 * ------------------------------------------------------------------------- */
int mg_device_count(int* count);
int mg_malloc(void** ptr, size_t bytes);
int mg_free(void* ptr);
int mg_host_alloc(void** ptr, size_t bytes); /* pinned host memory */
int mg_host_free(void* ptr);
int mg_memcpy_h2d(void* dst, const void* src, size_t bytes);
int mg_memcpy_d2h(void* dst, const void* src, size_t bytes);
int mg_memcpy_d2d(void* dst, const void* src, size_t bytes);
int mg_memset(void* dst, int value, size_t bytes);
int mg_synchronize(void);

/* ---------------------------------------------------------------------------
 * Environment registry. Replaces the reference's kernel lookup by name
 * (gym.h:43-44: newDefaultLibrary()->newFunction(Env::KERNEL)). Each env's
 * kernels are instantiated by MG_DEFINE_ENV (mg/device/env_kernels.h), which
 * registers this table under Env::KERNEL. The built-in envs are
 * "rollout_cartpole", "rollout_cartpole_continuous",
 * "rollout_cartpole_continuous_clamp", "rollout_voxelnav" (the reference's
 * heightmap env) and "rollout_voxelnav16".
 * ------------------------------------------------------------------------- */

enum { MG_ACTIONS_GIVEN = 0, MG_ACTIONS_RANDOM = 1 };

/* Launch arguments of an env's rollout kernel: `steps` env steps of every env,
 * one lane per env (rollout.h:31-54). In MG_ACTIONS_GIVEN mode step t reads
 * actions_in[t * n + i]; in MG_ACTIONS_RANDOM mode each env draws its own action
 * from its RNG before the reset-if-done (rngInt(rng, ACT_DIM), or uniform in
 * [-1, 1) per dimension for a float action) and records it in actions_out.
 * Slot outputs are [steps][n]; any of them may be NULL. */
typedef struct mg_rollout_args {
    void* stream;
    uint32_t n;
    uint32_t steps;
    uint32_t mode;
    uint32_t reserved;
    void* state;            /* [n] Env::State */
    uint32_t* rng;          /* [n] */
    uint8_t* done;          /* [n] live done flags */
    const void* actions_in; /* [steps][n] Env::Action (GIVEN) */
    void* actions_out;      /* [steps][n] Env::Action (RANDOM), nullable */
    float* obs_out;         /* [steps][n] Env::Obs, nullable */
    float* reward_out;      /* [steps][n], nullable */
    uint8_t* done_out;      /* [steps][n], nullable */
} mg_rollout_args;

/* Device view of a policy's parameters: one flat fp32 arena plus element
 * offsets. Layout (same grouping as model/ppo.h:412-423, each entry padded to
 * a multiple of 128 elements): in_w [obs x 128], in_b [128], per block
 * ln_gamma/ln_beta [128], final ln_gamma/ln_beta [128], log_std [act]
 * (Gaussian head only); then per block up [128 x hidden] and down [hidden x 128]
 * (row-major, x @ W), then head [128 x head_dim], head_dim = act + 1
 * (columns < act: logits or means, column act: value).
 * frag_fwd32, frag_fwd16 and frag_bwd16 hold the block matrices again, at
 * the same offsets, in the operand order of MT x MT matrix instructions: a
 * matrix read as rows n of contraction length K is cut into MT x 128 tiles,
 * and element (n, k) sits at (n / MT) MT K + (k / 128) MT 128 +
 * (k % 128 / KG) 256 + (k % KG / 4) 4 MT + (n % MT) 4 + k % 4 from the
 * matrix's offset (MT = 32, KG = 8 for 32x32x2; MT = 16, KG = 16 for 16x16x4).
 * frag_fwd32 and frag_fwd16 hold up^T and down^T (the forward's operands),
 * frag_bwd16 up and down as stored (the backward's). With precision
 * MG_PRECISION_BF16, frag_fwd32_bf and frag_fwd16_bf hold up^T and down^T and
 * frag_bwd16_bf up and down, rounded to bfloat16 (16-bit patterns), in the
 * operand order of the bf16 instructions (32x32x16 and 16x16x32: k-groups of
 * 16 and 32, each lane 8 consecutive k); otherwise they are NULL. The fused kernels read the
 * matrices from them. The library derives all of them from params at creation and in
 * mg_ppo_set_params / mg_ppo_params_updated. A train step (mg_ppo_train, mg_ppo_train_block,
 * mg_ppo_train_block_noalloc) rewrites only the copies its own kernels read next (frag_fwd16
 * and frag_bwd16; in bf16 mode their bf16 versions) and leaves the others (frag_fwd32, and in
 * bf16 mode the fp32 copies and frag_fwd32_bf) behind params until the next mg_ppo_policy,
 * mg_ppo_collect or mg_ppo_forward re-derives them. The pointers never change, so a view stays
 * valid for the model's life, but its copies are current only after one of those calls: a
 * caller that launches kernels with a view after training (an env's mg_env_desc.collect, say)
 * calls mg_ppo_policy first. */
enum { MG_PRECISION_FP32 = 0, MG_PRECISION_BF16 = 1 };
typedef struct mg_policy_view {
    float* params;
    float* frag_fwd32;
    float* frag_fwd16;
    float* frag_bwd16;
    uint16_t* frag_fwd32_bf;
    uint16_t* frag_fwd16_bf;
    uint16_t* frag_bwd16_bf;
    uint32_t obs_dim;
    uint32_t act_dim;
    uint32_t embed;
    uint32_t hidden;
    uint32_t layers;
    uint32_t head_dim;
    uint32_t continuous;
    uint32_t precision; /* MG_PRECISION_*: the policy forward's matrix operands */
    uint32_t count;     /* arena length in floats */
    uint32_t off_in_w;
    uint32_t off_in_b;
    uint32_t off_ln_gamma[MG_MAX_LAYERS + 1]; /* index `layers` = final LN */
    uint32_t off_ln_beta[MG_MAX_LAYERS + 1];
    uint32_t off_up[MG_MAX_LAYERS];
    uint32_t off_down[MG_MAX_LAYERS];
    uint32_t off_head;
    uint32_t off_log_std; /* Gaussian head only */
    uint32_t float_group; /* elements in the vector-parameter group */
} mg_policy_view;

/* Launch arguments of an env's fused collect kernel (model/ppo.h:716-751 minus
 * GAE): for each env, `horizon` steps of policy forward, sampling from the
 * env's RNG, reset-if-done and Env::step, with state and RNG in registers,
 * then the bootstrap forward on the last obs. */
typedef struct mg_collect_args {
    void* stream;
    mg_policy_view policy;
    uint32_t n;
    uint32_t horizon;
    uint32_t first; /* 1: run the reference's extra first step with action 0 (model/ppo.h:720-722) */
    uint32_t reserved;
    void* state;
    uint32_t* rng;
    uint8_t* done;
    float* obs_slots;    /* [horizon + 1][n] Env::Obs */
    void* action_slots;  /* [horizon][n] Env::Action */
    float* logp_slots;   /* [horizon][n] */
    float* value_slots;  /* [horizon][n] */
    float* reward_slots; /* [horizon][n] */
    uint8_t* done_slots; /* [horizon][n] */
    float* head_out;     /* [n][head_dim]: head of the bootstrap forward */
} mg_collect_args;

typedef struct mg_env_desc {
    uint32_t abi_version;
    uint32_t state_bytes;
    uint32_t action_bytes;
    uint32_t obs_dim;
    uint32_t act_dim;
    uint32_t continuous;
    uint32_t state_in_registers;
    uint32_t reserved;
    const char* kernel; /* Env::KERNEL */
    int (*rollout)(const mg_rollout_args* args);
    int (*collect)(const mg_collect_args* args);
} mg_env_desc;

/* Register an env; the table must outlive the library (MG_DEFINE_ENV uses a static). */
int mg_env_register(const mg_env_desc* desc);
/* gym.h:43-44: find an env's kernels by Env::KERNEL. */
int mg_env_lookup(const char* kernel, const mg_env_desc** out);
int mg_env_count(void);
const char* mg_env_name(int index);

/* ---------------------------------------------------------------------------
 * Gym: the env runtime (gym.h:15-122).
 * ------------------------------------------------------------------------- */
typedef struct mg_gym mg_gym;

typedef struct mg_gym_buffers {
    void* stream;
    const mg_env_desc* env;
    uint32_t n;
    uint32_t seed;
    void* state;    /* [n] Env::State */
    void* actions;  /* [n] Env::Action, read by mg_gym_run (gym.h:86) */
    float* obs;     /* [n] Env::Obs, written by mg_gym_run (gym.h:88) */
    float* reward;  /* [n] */
    uint8_t* done;  /* [n] (gym.h:87) */
    uint32_t* rng;  /* [n] */
} mg_gym_buffers;

/* gym.h:36-61: allocate the six env buffers for n envs, done = 1, actions = 0,
 * rng[i] = env_seed(seed, i) (seed 0 gives the reference's i * 2654435761 + 1). */
int mg_gym_create(const char* kernel, uint32_t n, uint32_t seed, mg_gym** out);
/* gym.h:73-85 */
int mg_gym_destroy(mg_gym* gym);
int mg_gym_buffers_get(mg_gym* gym, mg_gym_buffers* out);
/* gym.h:94-108 (encodeStep): one env step reading actions from actions_in and
 * writing obs/reward to the given device buffers; the gym's own state, done and
 * rng are updated. Asynchronous on the gym's stream. */
int mg_gym_step_into(mg_gym* gym, const void* actions_in, float* obs_out, float* reward_out);
/* gym.h:110-121 (run): one step from the gym's action buffer into its obs and
 * reward buffers. Asynchronous; mg_gym_sync waits. */
int mg_gym_run(mg_gym* gym);
/* A random-policy rollout of `steps` steps with [steps][n] slot outputs
 * (each nullable). Asynchronous. */
int mg_gym_rollout_random(mg_gym* gym, uint32_t steps, void* actions_out, float* obs_out, float* reward_out,
                          uint8_t* done_out);
/* A given-action rollout: step t reads actions_in[t * n + i]. Asynchronous. */
int mg_gym_rollout_given(mg_gym* gym, uint32_t steps, const void* actions_in, float* obs_out, float* reward_out,
                         uint8_t* done_out);
int mg_gym_sync(mg_gym* gym);

/* ---------------------------------------------------------------------------
 * PPO model: PPOModel<Env> (model/ppo.h:106-1009).
 * ------------------------------------------------------------------------- */
typedef struct mg_ppo mg_ppo;

/* Constructor arguments (model/ppo.h:274): embed (must be 128), hidden scale,
 * layers, learning rate, horizon T and seed; plus the minibatch row count
 * (multiple of 64 that divides n; 0 = min(n, 4096)). */
typedef struct mg_ppo_config {
    uint32_t embed;
    uint32_t scale;
    uint32_t layers;
    uint32_t horizon;
    uint32_t minibatch;
    uint32_t seed;
    float lr;
    /* MG_PRECISION_FP32 (default), or MG_PRECISION_BF16: the block matmuls of
     * the forward, the backward and the weight gradients multiply bfloat16
     * operands (weights, LN outputs, hidden activations and their gradients)
     * with fp32 accumulation, as the reference's matmuls do; master weights,
     * Adam, LN, head and embed stay fp32 (no reference counterpart as a switch:
     * the reference is bf16-only, README.md:174-175). */
    uint32_t precision;
} mg_ppo_config;

/* Public hyperparameter fields (model/ppo.h:186-191), read on every call. */
typedef struct mg_ppo_hparams {
    float clip;
    float value_coef;
    float entropy_coef;
    float max_grad_norm; /* 0 disables clipping */
    float gamma;
    float lambda;
} mg_ppo_hparams;

/* LossStats (model/ppo.h:97-104): means over one minibatch's rows; grad_norm is
 * the global L2 norm before clipping. */
typedef struct mg_loss_stats {
    float policy;
    float value;
    float entropy;
    float approx_kl;
    float clip_frac;
    float grad_norm;
} mg_loss_stats;

/* Device pointers of the rollout slots (model/ppo.h:336-345, 470-476), all
 * [horizon][n] except obs ([horizon + 1][n]). */
typedef struct mg_ppo_slots {
    float* obs;
    void* actions;
    float* logp;
    float* value;
    float* reward;
    uint8_t* done;
    float* advantage;
    float* ret;
    uint32_t n;
    uint32_t horizon;
} mg_ppo_slots;

/* model/ppo.h:290-298: the constructor's validation alone, for env `kernel` and
 * n envs; no device work, so configuration errors are testable without a GPU. */
int mg_ppo_check_config(const char* kernel, uint32_t n, const mg_ppo_config* config);
/* model/ppo.h:274-446: validate, allocate, initialise parameters from seed. The
 * model borrows the gym (its stream, state, rng and done) and must be destroyed
 * before it. */
int mg_ppo_create(mg_gym* gym, const mg_ppo_config* config, mg_ppo** out);
int mg_ppo_destroy(mg_ppo* model);
/* The effective configuration (minibatch resolved from 0 to its default). */
int mg_ppo_config_get(mg_ppo* model, mg_ppo_config* out);
int mg_ppo_set_hparams(mg_ppo* model, const mg_ppo_hparams* hp);
int mg_ppo_get_hparams(mg_ppo* model, mg_ppo_hparams* hp);
/* model/ppo.h:716-751: one rollout of T steps plus GAE. Blocking. */
int mg_ppo_collect(mg_ppo* model);
/* model/ppo.h:918-923: `epochs` shuffled passes over the rollout, one Adam step
 * per minibatch. Blocking. */
int mg_ppo_train(mg_ppo* model, uint32_t epochs);
/* model/ppo.h:906-916 (trainSlot) generalised to a minibatch block id
 * (block b covers rows (b % (n / minibatch)) * minibatch ... of slot b / (n / minibatch)).
 * Blocking. */
int mg_ppo_train_block(mg_ppo* model, uint32_t block);
/* No reference counterpart: mg_ppo_train_block for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). The minibatch's workspace lives in a
 * static device array of 64 MiB per device (held from library load to process
 * exit), so the call makes no allocation; a policy whose workspace for one
 * minibatch exceeds it (64 MiB minus 256 bytes; 60 MB for the 2-block, hidden
 * 512 policy at 4096 rows) is rejected with MG_ERR_INVALID. The LossStats
 * (6 floats, mg_loss_stats order) go to stats_out, a device pointer, or to
 * the array when it is NULL. Asynchronous on the gym's stream; the Adam step
 * count and its bias corrections are taken at call time. Every call on one
 * device shares the array: calls that overlap on one device (two streams, two
 * threads) race. mg_ppo_last_stats, mg_ppo_train_stats, mg_ppo_last_order
 * and mg_ppo_train_capture are not updated (the captures of a no-alloc call
 * live in the array; mg_ppo_train_capture keeps returning those of the last
 * mg_ppo_train or mg_ppo_train_block, or MG_ERR_STATE if there was none). */
int mg_ppo_train_block_noalloc(mg_ppo* model, uint32_t block, float* stats_out);
/* model/ppo.h:628-634: policy forward on `rows` obs rows (device pointer) into
 * the model's head buffer. Blocking. */
int mg_ppo_forward(mg_ppo* model, const float* obs, uint32_t rows);
/* model/ppo.h:925-943 */
int mg_ppo_last_stats(mg_ppo* model, mg_loss_stats* out);
/* LossStats of every minibatch of the last mg_ppo_train call, in order. */
int mg_ppo_train_stats(mg_ppo* model, mg_loss_stats* out, uint32_t capacity, uint32_t* count);
int mg_ppo_slots_get(mg_ppo* model, mg_ppo_slots* out);
/* model/ppo.h:450-452: device pointer of the head of the last forward,
 * [rows][head_dim] (the bootstrap forward after collect, the last minibatch
 * after train). */
int mg_ppo_head(mg_ppo* model, const float** head, uint32_t* rows, uint32_t* head_dim);
int mg_ppo_policy(mg_ppo* model, mg_policy_view* out);
/* Replaces all parameters (count = mg_policy_view.count floats from host
 * memory) and re-derives the fragment-tiled copies. No reference counterpart: the reference's
 * weights are shared CPU/GPU memory that tests write in place. */
int mg_ppo_set_params(mg_ppo* model, const float* host, uint32_t count);
/* Re-derives the fragment-tiled copies after the caller wrote params through
 * the device view. */
int mg_ppo_params_updated(mg_ppo* model);
/* Activation captures of the last minibatch of mg_ppo_train or
 * mg_ppo_train_block (the row pass writes them for the weight gradients;
 * mg_ppo_train_block_noalloc leaves them unchanged), for tests and debugging; no reference
 * counterpart (the reference keeps its activations in internal buffers,
 * model/ppo.h:355-372). which = MG_CAPTURE_*: the LN outputs entering each
 * block ([layers][B][128]), the relu'd hidden activations ([layers][B][hidden]),
 * the gradients at the block outputs ([layers][B][128]) and the masked hidden
 * gradients ([layers][B][hidden]). MG_PRECISION_FP32: fp32, row-major.
 * MG_PRECISION_BF16: bfloat16 bit patterns, row-group-packed (element (r, c)
 * of a C-column capture at ((r / 8) C + c) 8 + r % 8). *ptr is a device
 * pointer valid until the next train call; MG_ERR_STATE before the first. */
enum { MG_CAPTURE_LN_OUT = 0, MG_CAPTURE_HIDDEN = 1, MG_CAPTURE_DH = 2, MG_CAPTURE_DV = 3 };
int mg_ppo_train_capture(mg_ppo* model, uint32_t which, const void** ptr, uint32_t* rows, uint32_t* cols,
                         uint32_t* layers);
/* Adam state: first and second moments, same layout as the parameters. */
int mg_ppo_adam_state(mg_ppo* model, float** m, float** v, uint32_t* step);
/* model/ppo.h:460-469 (Gaussian head only). */
int mg_ppo_set_log_std(mg_ppo* model, float value);
/* Minibatch order of the last train call: block ids, epochs * blocks_per_epoch. */
int mg_ppo_last_order(mg_ppo* model, uint32_t* out, uint32_t capacity, uint32_t* count);

/* Stage entry points used by parity tests (teacher forcing) and by act():
 * sample one action per row from a head (model/sample.metal:18-47 or
 * model/gaussian.metal:42-71), advancing the given RNG states. */
int mg_ppo_sample(mg_ppo* model, const float* head, uint32_t rows, uint32_t* rng, void* actions, float* logp,
                  float* value);
/* model/gae.metal:14-36 over [horizon][n] slots; the bootstrap value is column
 * act_dim of head ([n][head_dim]). */
int mg_gae(void* stream, const float* reward, const uint8_t* done, const float* value, const float* head,
           uint32_t head_dim, uint32_t act_dim, uint32_t n, uint32_t horizon, float gamma, float lambda,
           float* advantage, float* ret);

/* ---------------------------------------------------------------------------
 * Kernel timing for measurement: when enabled, the library records HIP events
 * around each launch on the stream it uses and accumulates durations.
 * ------------------------------------------------------------------------- */
enum {
    MG_K_ROLLOUT = 0,
    MG_K_COLLECT = 1,
    MG_K_GAE = 2,
    MG_K_ADV_STATS = 3,
    MG_K_TRAIN_ROWS = 4,
    MG_K_TRAIN_DW = 5,
    MG_K_GRAD_REDUCE = 6,
    MG_K_ADAM = 7,
    MG_K_FORWARD = 8,
    MG_K_COPY = 9, /* mg_memcpy_d2d: the size floor of a kernel's HBM traffic */
    MG_K_COUNT = 10
};
typedef struct mg_kernel_times {
    double total_ms[MG_K_COUNT];
    uint64_t launches[MG_K_COUNT];
} mg_kernel_times;
int mg_timing_enable(int on);
int mg_timing_get(mg_kernel_times* out);
int mg_timing_reset(void);

#ifdef __cplusplus
}
#endif
#endif /* MG_CAPI_H */
