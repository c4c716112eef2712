// PPOModel (model/ppo.h:106-1009) behind the C ABI: validation, parameter
// layout and seeded initialisation, rollout slots, and the collect/train
// orchestration on the gym's stream.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "kernels.h"

struct mg_ppo {
    mg_gym* gym = nullptr;
    const mg_env_desc* env = nullptr;
    mg_ppo_config cfg{};
    mg_ppo_hparams hp{};
    uint32_t n = 0, T = 0, B = 0, blocks = 0;
    mg_policy_view pv{};
    float* m = nullptr;
    float* v = nullptr;
    uint32_t step = 0;
    uint64_t shuffle_state = 0;
    std::vector<uint32_t> order;       // persistent block order (slotOrder, model/ppo.h:347-348)
    std::vector<uint32_t> last_order;  // block sequence of the last train call
    float* obs_slots = nullptr;
    void* action_slots = nullptr;
    float* logp = nullptr;
    float* value = nullptr;
    float* reward = nullptr;
    uint8_t* done_slots = nullptr;
    float* adv = nullptr;
    float* ret = nullptr;
    float* head = nullptr;
    uint32_t head_rows = 0, head_cap = 0;
    float* adv_stats = nullptr;
    bool rollout_started = false;
    bool collected = false;
    bool tiles_stale = false;  // a train call left the copies that only collect and forward read behind params
    void* ws_base = nullptr;
    mg::TrainWs ws{};
    float* mb_stats = nullptr;
    uint32_t mb_cap = 0;
    std::vector<float> mb_host;
};

namespace mg {
namespace {

uint32_t pad128(uint32_t x) { return (x + 127u) / 128u * 128u; }

// model/ppo.h:412-423: vector parameters first, then matrices, each padded to
// 128 elements; the head is act + 1 columns wide.
void make_layout(mg_policy_view& pv) {
    const uint32_t E = pv.embed, H = pv.hidden, O = pv.obs_dim, A = pv.act_dim, L = pv.layers;
    uint32_t off = 0;
    pv.head_dim = A + 1;
    pv.off_in_w = off, off += pad128(O * E);
    pv.off_in_b = off, off += pad128(E);
    for (uint32_t l = 0; l <= L; ++l) {
        pv.off_ln_gamma[l] = off, off += pad128(E);
        pv.off_ln_beta[l] = off, off += pad128(E);
    }
    pv.off_log_std = 0;
    if (pv.continuous) pv.off_log_std = off, off += pad128(A);
    pv.float_group = off;
    for (uint32_t l = 0; l < L; ++l) {
        pv.off_up[l] = off, off += pad128(E * H);
        pv.off_down[l] = off, off += pad128(H * E);
    }
    pv.off_head = off, off += pad128(E * pv.head_dim);
    pv.count = off;
}

// SplitMix64 (Steele, Lea & Flood 2014): the build's host-side generator for
// initial weights and minibatch order (the reference uses std::mt19937,
// model/ppo.h:349, 375).
uint64_t splitmix(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
constexpr uint64_t kInitStream = 0x4D47494E49540000ull;     // "MGINIT"
constexpr uint64_t kShuffleStream = 0x4D47534855460000ull;  // "MGSHUF"

float uniform_pm(uint64_t& s, float bound) {
    const float u = (float)(splitmix(s) >> 40) * (1.0f / 16777216.0f);
    return bound * (2.0f * u - 1.0f);
}

// model/ppo.h:375-410 with uniform draws of the same per-layer standard
// deviation (bound = sqrt(3) std), in the reference's parameter order.
void init_params(const mg_policy_view& pv, uint32_t seed, std::vector<float>& P) {
    P.assign(pv.count, 0.0f);
    uint64_t s = kInitStream ^ (uint64_t)seed;
    const uint32_t E = pv.embed, H = pv.hidden, O = pv.obs_dim, A = pv.act_dim, HD = pv.head_dim;
    const float bIn = sqrtf(3.0f / (float)O);
    for (uint32_t i = 0; i < O * E; ++i) P[pv.off_in_w + i] = uniform_pm(s, bIn);
    for (uint32_t l = 0; l < pv.layers; ++l) {
        for (uint32_t c = 0; c < E; ++c) P[pv.off_ln_gamma[l] + c] = 1.0f;
        const float bUp = sqrtf(6.0f / (float)E);
        for (uint32_t i = 0; i < E * H; ++i) P[pv.off_up[l] + i] = uniform_pm(s, bUp);
        const float bDn = sqrtf(3.0f / (float)H) / sqrtf((float)pv.layers);
        for (uint32_t i = 0; i < H * E; ++i) P[pv.off_down[l] + i] = uniform_pm(s, bDn);
    }
    for (uint32_t c = 0; c < E; ++c) P[pv.off_ln_gamma[pv.layers] + c] = 1.0f;
    const float bPol = 0.01f * sqrtf(3.0f), bVal = sqrtf(3.0f / (float)E);
    for (uint32_t k = 0; k < E; ++k)
        for (uint32_t j = 0; j < HD; ++j) P[pv.off_head + k * HD + j] = uniform_pm(s, j < A ? bPol : bVal);
}

// Fisher-Yates over the current order, in place (std::shuffle's role at model/ppo.h:920).
void shuffle_blocks(uint64_t& s, std::vector<uint32_t>& order) {
    for (uint32_t i = (uint32_t)order.size(); i > 1; --i) {
        const uint32_t j = (uint32_t)(splitmix(s) % (uint64_t)i);
        std::swap(order[i - 1], order[j]);
    }
}

int ensure_head(mg_ppo* p, uint32_t rows) {
    if (rows <= p->head_cap) return MG_OK;
    (void)hipFree(p->head);
    p->head = nullptr;
    p->head_cap = 0;
    int rc = device_alloc((void**)&p->head, (size_t)rows * p->pv.head_dim * sizeof(float), "PPOModel head");
    if (rc) return rc;
    p->head_cap = rows;
    return MG_OK;
}

int ensure_train_ws(mg_ppo* p, uint32_t minibatches) {
    if (!p->ws_base) {
        size_t bytes = 0;
        train_ws_bytes(p->pv, p->B, &bytes);
        int rc = device_alloc(&p->ws_base, bytes, "PPOModel train workspace");
        if (rc) return rc;
        // every element the kernels read is written first (the only padding,
        // after log_std, gets explicit zeros), so this clear only makes a fresh
        // workspace deterministic to inspect through mg_ppo_train_capture
        MG_HIP(hipMemsetAsync(p->ws_base, 0, bytes, p->gym->stream), "train workspace clear");
        train_ws_bind(p->pv, p->B, p->ws_base, &p->ws);
    }
    if (minibatches > p->mb_cap) {
        (void)hipFree(p->mb_stats);
        p->mb_stats = nullptr;
        p->mb_cap = 0;
        int rc = device_alloc((void**)&p->mb_stats, (size_t)minibatches * 6 * sizeof(float), "PPOModel stats");
        if (rc) return rc;
        p->mb_cap = minibatches;
    }
    return MG_OK;
}

// One minibatch update on the stream (no host wait), with workspace ws; the
// minibatch's LossStats go to stats (6 floats, device).
int enqueue_minibatch(mg_ppo* p, uint32_t block, uint32_t mb_index, const TrainWs& ws, float* stats) {
    p->tiles_stale = true;
    const uint32_t perSlot = p->n / p->B;
    const uint32_t t = block / perSlot, r0 = (block % perSlot) * p->B;
    p->step += 1;
    // model/ppo.h:874-880: float step counter, float powers
    const float stepF = (float)p->step;
    TrainStep ts;
    ts.row0 = t * p->n + r0;
    ts.block = block;
    ts.rows = p->B;
    ts.mb_index = mb_index;
    ts.beta1_pow = powf(0.9f, stepF);
    ts.beta2_pow = powf(0.999f, stepF);
    return launch_train_step(p->gym->stream, p->pv, p->hp, p->cfg.lr, ws, ts, p->obs_slots, p->action_slots,
                             p->adv, p->ret, p->logp, p->adv_stats, p->m, p->v, p->head, stats);
}

// The fragment-tiled copies that the train kernels do not keep current
// (launch_train_step), derived from params on the model's stream before a
// kernel that reads them.
int sync_tiles(mg_ppo* p) {
    if (!p->tiles_stale) return MG_OK;
    int rc = launch_derive_blocks(p->gym->stream, p->pv);
    if (rc) return rc;
    p->tiles_stale = false;
    return MG_OK;
}

int enqueue_minibatch(mg_ppo* p, uint32_t block, uint32_t mb_index) {
    return enqueue_minibatch(p, block, mb_index, p->ws, p->mb_stats + (size_t)mb_index * 6);
}

// ---- device memory of mg_ppo_train_block_noalloc -------------------------------
// The train workspace of one minibatch and its LossStats in a file-scope
// device array (below), which the HIP runtime places on every device that
// loads the library and keeps until the process ends. Host code never uses
// the array's name as an address: scratch_address() asks the runtime for the
// array's address on the stream's device, once per device.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr size_t kNoAllocStatsBytes = 256;  // LossStats, at the array's start
constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices];

}  // namespace
}  // namespace mg

static __device__ __align__(256) unsigned char scratch[mg::kNoAllocScratchBytes];

namespace mg {
namespace {

int scratch_address(hipStream_t st, unsigned char** out) {
    hipDevice_t dev = 0;
    MG_HIP(hipStreamGetDevice(st, &dev), "train_block_noalloc: stream device");
    MG_CHECK(dev >= 0 && dev < kMaxDevices, MG_ERR_INVALID, "train_block_noalloc: device %d out of range", (int)dev);
    if (!g_scratch[dev]) {
        int cur = 0;
        MG_HIP(hipGetDevice(&cur), "train_block_noalloc: current device");
        if (cur != dev) MG_HIP(hipSetDevice(dev), "train_block_noalloc: select the stream's device");
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur != dev) MG_HIP(hipSetDevice(cur), "train_block_noalloc: restore the current device");
        MG_HIP(e, "train_block_noalloc: scratch address");
        MG_CHECK(ptr, MG_ERR_HIP, "train_block_noalloc: no scratch address");
        g_scratch[dev] = ptr;
    }
    *out = static_cast<unsigned char*>(g_scratch[dev]);
    return MG_OK;
}

int download_stats(mg_ppo* p, uint32_t count) {
    p->mb_host.resize((size_t)count * 6);
    if (count)
        MG_HIP(hipMemcpyAsync(p->mb_host.data(), p->mb_stats, (size_t)count * 6 * sizeof(float),
                              hipMemcpyDeviceToHost, p->gym->stream),
               "stats download");
    MG_HIP(hipStreamSynchronize(p->gym->stream), "train synchronize");
    return MG_OK;
}

}  // namespace
}  // namespace mg

using namespace mg;

namespace mg {
namespace {
// model/ppo.h:290-298 plus this build's limits; *B_out receives the minibatch.
int validate_config(const mg_env_desc* env, uint32_t n, const mg_ppo_config* c, uint32_t* B_out) {
    MG_CHECK(env && c, MG_ERR_INVALID, "PPOModel: null argument");
    MG_CHECK(n > 0 && n % 64 == 0, MG_ERR_INVALID, "PPOModel: the env count %u must be a positive multiple of 64", n);
    MG_CHECK(c->embed == MG_EMBED, MG_ERR_INVALID, "PPOModel: embedDim %u != %d (compile-time embed width)", c->embed,
             MG_EMBED);
    MG_CHECK(c->scale >= 1 && c->scale <= 8, MG_ERR_INVALID, "PPOModel: hidden scale %u must be in [1, 8]", c->scale);
    MG_CHECK(c->layers >= 1 && c->layers <= MG_MAX_LAYERS, MG_ERR_INVALID, "PPOModel: layers %u must be in [1, %d]",
             c->layers, MG_MAX_LAYERS);
    MG_CHECK(c->horizon >= 1, MG_ERR_INVALID, "PPOModel: horizon must be >= 1");
    MG_CHECK(c->precision == MG_PRECISION_FP32 || c->precision == MG_PRECISION_BF16, MG_ERR_INVALID,
             "PPOModel: precision %u must be MG_PRECISION_FP32 or MG_PRECISION_BF16", c->precision);
    MG_CHECK(env->obs_dim >= 1 && env->obs_dim <= 64, MG_ERR_INVALID, "PPOModel: OBS_DIM %u must be in [1, 64]",
             env->obs_dim);
    MG_CHECK(env->act_dim >= 1 && env->act_dim + 1 <= 64, MG_ERR_INVALID,
             "PPOModel: ACT_DIM + value must fit a 64-wide head");
    MG_CHECK(env->collect, MG_ERR_INVALID, "PPOModel: env '%s' has no collect kernel", env->kernel);
    const uint32_t B = c->minibatch ? c->minibatch : std::min<uint32_t>(n, 4096u);
    MG_CHECK(B % 64 == 0 && n % B == 0, MG_ERR_INVALID, "PPOModel: minibatch %u must be a multiple of 64 that divides %u",
             B, n);
    MG_CHECK((uint64_t)n * (c->horizon + 1) < (1ull << 31), MG_ERR_INVALID, "PPOModel: n * (horizon + 1) too large");
    // the weight-gradient kernels address a capture of B rows with 32-bit
    // byte offsets (buffer loads): B * max(hidden, 128) * 4 must stay below 2^31
    const uint64_t widest = std::max<uint64_t>((uint64_t)c->embed * c->scale, MG_EMBED);
    MG_CHECK((uint64_t)B * widest * 4 < (1ull << 31), MG_ERR_INVALID,
             "PPOModel: minibatch %u x hidden %u is too large (the captures' byte offsets must fit 31 bits)", B,
             c->embed * c->scale);
    if (B_out) *B_out = B;
    return MG_OK;
}
}  // namespace
}  // namespace mg

extern "C" {

int mg_ppo_check_config(const char* kernel, uint32_t n, const mg_ppo_config* c) {
    const mg_env_desc* env = nullptr;
    int rc = mg_env_lookup(kernel, &env);
    if (rc) return rc;
    return validate_config(env, n, c, nullptr);
}

int mg_ppo_create(mg_gym* gym, const mg_ppo_config* c, mg_ppo** out) {
    MG_CHECK(gym && c && out, MG_ERR_INVALID, "PPOModel: null argument");
    *out = nullptr;
    const mg_env_desc* env = gym->env;
    uint32_t B = 0;
    int vrc = validate_config(env, gym->n, c, &B);
    if (vrc) return vrc;
    mg_ppo* p = new mg_ppo();
    p->gym = gym;
    p->env = env;
    p->cfg = *c;
    p->cfg.minibatch = B;
    p->hp = mg_ppo_hparams{0.2f, 0.5f, 0.01f, 0.5f, 0.99f, 0.95f};  // model/ppo.h:186-191
    p->n = gym->n;
    p->T = c->horizon;
    p->B = B;
    p->blocks = p->T * (p->n / B);
    mg_policy_view& pv = p->pv;
    pv.obs_dim = env->obs_dim;
    pv.act_dim = env->act_dim;
    pv.embed = c->embed;
    pv.hidden = c->embed * c->scale;
    pv.layers = c->layers;
    pv.continuous = env->continuous;
    pv.precision = c->precision;
    make_layout(pv);
    auto fail = [&](int code) {
        mg_ppo_destroy(p);
        return code;
    };
    const size_t n = p->n, T = p->T;
    const size_t slot = T * n;
    int rc;
    if ((rc = check_matrix_layout(pv))) return fail(rc);
    if ((rc = device_alloc((void**)&pv.params, (size_t)pv.count * 4, "PPOModel params")) ||
        (rc = device_alloc((void**)&pv.frag_fwd32, (size_t)pv.count * 4, "PPOModel forward matrix tiles")) ||
        (rc = device_alloc((void**)&pv.frag_fwd16, (size_t)pv.count * 4, "PPOModel forward matrix tiles")) ||
        (rc = device_alloc((void**)&pv.frag_bwd16, (size_t)pv.count * 4, "PPOModel backward matrix tiles")) ||
        (pv.precision == MG_PRECISION_BF16 &&
         ((rc = device_alloc((void**)&pv.frag_fwd32_bf, (size_t)pv.count * 2, "PPOModel bf16 matrix tiles")) ||
          (rc = device_alloc((void**)&pv.frag_fwd16_bf, (size_t)pv.count * 2, "PPOModel bf16 matrix tiles")) ||
          (rc = device_alloc((void**)&pv.frag_bwd16_bf, (size_t)pv.count * 2, "PPOModel bf16 matrix tiles")))) ||
        (rc = device_alloc((void**)&p->m, (size_t)pv.count * 4, "PPOModel adam m")) ||
        (rc = device_alloc((void**)&p->v, (size_t)pv.count * 4, "PPOModel adam v")) ||
        (rc = device_alloc((void**)&p->obs_slots, (T + 1) * n * env->obs_dim * 4, "obs slots")) ||
        (rc = device_alloc(&p->action_slots, slot * env->action_bytes, "action slots")) ||
        (rc = device_alloc((void**)&p->logp, slot * 4, "logp slots")) ||
        (rc = device_alloc((void**)&p->value, slot * 4, "value slots")) ||
        (rc = device_alloc((void**)&p->reward, slot * 4, "reward slots")) ||
        (rc = device_alloc((void**)&p->done_slots, slot, "done slots")) ||
        (rc = device_alloc((void**)&p->adv, slot * 4, "advantage slots")) ||
        (rc = device_alloc((void**)&p->ret, slot * 4, "return slots")) ||
        (rc = device_alloc((void**)&p->adv_stats, (size_t)p->blocks * 2 * 4, "advantage stats")) ||
        (rc = ensure_head(p, std::max(p->n, p->B))))
        return fail(rc);
    std::vector<float> P;
    init_params(pv, c->seed, P);
    hipStream_t st = gym->stream;
    if (hipMemcpyAsync(pv.params, P.data(), (size_t)pv.count * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemsetAsync(p->m, 0, (size_t)pv.count * 4, st) != hipSuccess ||
        hipMemsetAsync(p->v, 0, (size_t)pv.count * 4, st) != hipSuccess ||
        hipMemsetAsync(p->obs_slots, 0, (T + 1) * n * env->obs_dim * 4, st) != hipSuccess ||
        hipMemsetAsync(p->action_slots, 0, slot * env->action_bytes, st) != hipSuccess ||
        hipMemsetAsync(p->logp, 0, slot * 4, st) != hipSuccess ||
        hipMemsetAsync(p->value, 0, slot * 4, st) != hipSuccess ||
        hipMemsetAsync(p->reward, 0, slot * 4, st) != hipSuccess ||
        hipMemsetAsync(p->done_slots, 0, slot, st) != hipSuccess ||
        hipMemsetAsync(p->adv, 0, slot * 4, st) != hipSuccess ||
        hipMemsetAsync(p->ret, 0, slot * 4, st) != hipSuccess ||
        hipMemsetAsync(p->head, 0, (size_t)p->head_cap * pv.head_dim * 4, st) != hipSuccess ||
        hipMemsetAsync(pv.frag_fwd32, 0, (size_t)pv.count * 4, st) != hipSuccess ||
        hipMemsetAsync(pv.frag_fwd16, 0, (size_t)pv.count * 4, st) != hipSuccess ||
        hipMemsetAsync(pv.frag_bwd16, 0, (size_t)pv.count * 4, st) != hipSuccess ||
        (pv.frag_fwd32_bf && hipMemsetAsync(pv.frag_fwd32_bf, 0, (size_t)pv.count * 2, st) != hipSuccess) ||
        (pv.frag_fwd16_bf && hipMemsetAsync(pv.frag_fwd16_bf, 0, (size_t)pv.count * 2, st) != hipSuccess) ||
        (pv.frag_bwd16_bf && hipMemsetAsync(pv.frag_bwd16_bf, 0, (size_t)pv.count * 2, st) != hipSuccess))
        return fail(set_error(MG_ERR_HIP, "PPOModel: initialisation upload failed"));
    if ((rc = launch_derive_blocks(st, pv))) return fail(rc);
    if (hipStreamSynchronize(st) != hipSuccess)
        return fail(set_error(MG_ERR_HIP, "PPOModel: initialisation upload failed"));
    p->order.resize(p->blocks);
    for (uint32_t b = 0; b < p->blocks; ++b) p->order[b] = b;
    p->shuffle_state = kShuffleStream ^ (uint64_t)c->seed;
    *out = p;
    return MG_OK;
}

int mg_ppo_destroy(mg_ppo* p) {
    if (!p) return MG_OK;
    if (p->gym && p->gym->stream) (void)hipStreamSynchronize(p->gym->stream);
    (void)hipFree(p->pv.params);
    (void)hipFree(p->pv.frag_fwd32);
    (void)hipFree(p->pv.frag_fwd16);
    (void)hipFree(p->pv.frag_bwd16);
    (void)hipFree(p->pv.frag_fwd32_bf);
    (void)hipFree(p->pv.frag_fwd16_bf);
    (void)hipFree(p->pv.frag_bwd16_bf);
    (void)hipFree(p->m);
    (void)hipFree(p->v);
    (void)hipFree(p->obs_slots);
    (void)hipFree(p->action_slots);
    (void)hipFree(p->logp);
    (void)hipFree(p->value);
    (void)hipFree(p->reward);
    (void)hipFree(p->done_slots);
    (void)hipFree(p->adv);
    (void)hipFree(p->ret);
    (void)hipFree(p->head);
    (void)hipFree(p->adv_stats);
    (void)hipFree(p->ws_base);
    (void)hipFree(p->mb_stats);
    delete p;
    return MG_OK;
}

int mg_ppo_config_get(mg_ppo* p, mg_ppo_config* out) {
    MG_CHECK(p && out, MG_ERR_INVALID, "config_get: null argument");
    *out = p->cfg;
    return MG_OK;
}

int mg_ppo_set_hparams(mg_ppo* p, const mg_ppo_hparams* hp) {
    MG_CHECK(p && hp, MG_ERR_INVALID, "mg_ppo_set_hparams: null argument");
    p->hp = *hp;
    return MG_OK;
}

int mg_ppo_get_hparams(mg_ppo* p, mg_ppo_hparams* hp) {
    MG_CHECK(p && hp, MG_ERR_INVALID, "mg_ppo_get_hparams: null argument");
    *hp = p->hp;
    return MG_OK;
}

int mg_ppo_collect(mg_ppo* p) {
    MG_CHECK(p, MG_ERR_INVALID, "collect: null model");
    hipStream_t st = p->gym->stream;
    if (int rc = sync_tiles(p)) return rc;
    mg_collect_args a{};
    a.stream = st;
    a.policy = p->pv;
    a.n = p->n;
    a.horizon = p->T;
    a.first = p->rollout_started ? 0u : 1u;
    a.state = p->gym->state;
    a.rng = p->gym->rng;
    a.done = p->gym->done;
    a.obs_slots = p->obs_slots;
    a.action_slots = p->action_slots;
    a.logp_slots = p->logp;
    a.value_slots = p->value;
    a.reward_slots = p->reward;
    a.done_slots = p->done_slots;
    a.head_out = p->head;
    {
        TimedLaunch tl(MG_K_COLLECT, st);
        int rc = launcher_status(p->env->collect(&a), "collect");
        if (rc) return rc;
    }
    p->rollout_started = true;
    p->head_rows = p->n;
    {
        TimedLaunch tl(MG_K_GAE, st);
        int rc = launch_gae(st, p->reward, p->done_slots, p->value, p->head, p->pv.head_dim, p->pv.act_dim, p->n, p->T,
                            p->hp.gamma, p->hp.lambda, p->adv, p->ret);
        if (rc) return rc;
    }
    {
        TimedLaunch tl(MG_K_ADV_STATS, st);
        int rc = launch_adv_stats(st, p->adv, p->n, p->T, p->B, p->adv_stats);
        if (rc) return rc;
    }
    p->collected = true;
    MG_HIP(hipStreamSynchronize(st), "collect synchronize");
    return MG_OK;
}

int mg_ppo_train(mg_ppo* p, uint32_t epochs) {
    MG_CHECK(p, MG_ERR_INVALID, "train: null model");
    MG_CHECK(p->collected, MG_ERR_STATE, "train: call collect() first");
    const uint32_t total = epochs * p->blocks;
    int rc = ensure_train_ws(p, total ? total : 1);
    if (rc) return rc;
    p->last_order.clear();
    uint32_t mb = 0;
    for (uint32_t e = 0; e < epochs; ++e) {
        shuffle_blocks(p->shuffle_state, p->order);
        for (uint32_t b : p->order) {
            p->last_order.push_back(b);
            if ((rc = enqueue_minibatch(p, b, mb++))) return rc;
        }
    }
    if (total) p->head_rows = p->B;
    return download_stats(p, total);
}

int mg_ppo_train_block(mg_ppo* p, uint32_t block) {
    MG_CHECK(p, MG_ERR_INVALID, "train_block: null model");
    MG_CHECK(p->collected, MG_ERR_STATE, "train_block: call collect() first");
    MG_CHECK(block < p->blocks, MG_ERR_INVALID, "train_block: block %u out of range (%u blocks)", block, p->blocks);
    int rc = ensure_train_ws(p, 1);
    if (rc) return rc;
    p->last_order.assign(1, block);
    if ((rc = enqueue_minibatch(p, block, 0))) return rc;
    p->head_rows = p->B;
    return download_stats(p, 1);
}

int mg_ppo_train_block_noalloc(mg_ppo* p, uint32_t block, float* stats_out) {
    MG_CHECK(p, MG_ERR_INVALID, "train_block_noalloc: null model");
    MG_CHECK(p->collected, MG_ERR_STATE, "train_block_noalloc: call collect() first");
    MG_CHECK(block < p->blocks, MG_ERR_INVALID, "train_block_noalloc: block %u out of range (%u blocks)", block,
             p->blocks);
    size_t need = 0;
    train_ws_bytes(p->pv, p->B, &need);
    MG_CHECK(need <= kNoAllocScratchBytes - kNoAllocStatsBytes, MG_ERR_INVALID,
             "train_block_noalloc: a %u-row minibatch of this policy needs %zu bytes of workspace, more than the "
             "%zu-byte static scratch (use mg_ppo_train_block)",
             p->B, need, kNoAllocScratchBytes - kNoAllocStatsBytes);
    unsigned char* base = nullptr;
    int rc = scratch_address(p->gym->stream, &base);
    if (rc) return rc;
    TrainWs ws{};
    train_ws_bind(p->pv, p->B, base + kNoAllocStatsBytes, &ws);
    if ((rc = enqueue_minibatch(p, block, 0, ws, stats_out ? stats_out : reinterpret_cast<float*>(base)))) return rc;
    p->head_rows = p->B;
    return MG_OK;
}

int mg_ppo_forward(mg_ppo* p, const float* obs, uint32_t rows) {
    MG_CHECK(p && (obs || rows == 0), MG_ERR_INVALID, "forward: null argument");
    int rc = ensure_head(p, rows);
    if (rc) return rc;
    if ((rc = sync_tiles(p))) return rc;
    {
        TimedLaunch tl(MG_K_FORWARD, p->gym->stream);
        if ((rc = launch_forward(p->gym->stream, p->pv, obs, rows, p->head))) return rc;
    }
    p->head_rows = rows;
    MG_HIP(hipStreamSynchronize(p->gym->stream), "forward synchronize");
    return MG_OK;
}

int mg_ppo_last_stats(mg_ppo* p, mg_loss_stats* out) {
    MG_CHECK(p && out, MG_ERR_INVALID, "last_stats: null argument");
    memset(out, 0, sizeof(*out));
    if (p->mb_host.size() >= 6) memcpy(out, p->mb_host.data() + p->mb_host.size() - 6, sizeof(*out));
    return MG_OK;
}

int mg_ppo_train_stats(mg_ppo* p, mg_loss_stats* out, uint32_t capacity, uint32_t* count) {
    MG_CHECK(p && count, MG_ERR_INVALID, "train_stats: null argument");
    const uint32_t n = (uint32_t)(p->mb_host.size() / 6);
    *count = n;
    if (out) memcpy(out, p->mb_host.data(), (size_t)std::min(n, capacity) * sizeof(mg_loss_stats));
    return MG_OK;
}

int mg_ppo_slots_get(mg_ppo* p, mg_ppo_slots* out) {
    MG_CHECK(p && out, MG_ERR_INVALID, "slots: null argument");
    out->obs = p->obs_slots;
    out->actions = p->action_slots;
    out->logp = p->logp;
    out->value = p->value;
    out->reward = p->reward;
    out->done = p->done_slots;
    out->advantage = p->adv;
    out->ret = p->ret;
    out->n = p->n;
    out->horizon = p->T;
    return MG_OK;
}

int mg_ppo_head(mg_ppo* p, const float** head, uint32_t* rows, uint32_t* head_dim) {
    MG_CHECK(p && head && rows && head_dim, MG_ERR_INVALID, "head: null argument");
    *head = p->head;
    *rows = p->head_rows;
    *head_dim = p->pv.head_dim;
    return MG_OK;
}

int mg_ppo_policy(mg_ppo* p, mg_policy_view* out) {
    MG_CHECK(p && out, MG_ERR_INVALID, "policy: null argument");
    if (p->tiles_stale) {  // the view's copies are current when it is handed out
        if (int rc = sync_tiles(p)) return rc;
        MG_HIP(hipStreamSynchronize(p->gym->stream), "policy synchronize");
    }
    *out = p->pv;
    return MG_OK;
}

int mg_ppo_set_params(mg_ppo* p, const float* host, uint32_t count) {
    MG_CHECK(p && host, MG_ERR_INVALID, "set_params: null argument");
    MG_CHECK(count == p->pv.count, MG_ERR_INVALID, "set_params: %u floats given, the arena holds %u", count,
             p->pv.count);
    MG_HIP(hipMemcpyAsync(p->pv.params, host, (size_t)count * 4, hipMemcpyHostToDevice, p->gym->stream),
           "set_params upload");
    return mg_ppo_params_updated(p);
}

int mg_ppo_params_updated(mg_ppo* p) {
    MG_CHECK(p, MG_ERR_INVALID, "params_updated: null model");
    int rc = launch_derive_blocks(p->gym->stream, p->pv);
    if (rc) return rc;
    p->tiles_stale = false;
    MG_HIP(hipStreamSynchronize(p->gym->stream), "params_updated synchronize");
    return MG_OK;
}

int mg_ppo_train_capture(mg_ppo* p, uint32_t which, const void** ptr, uint32_t* rows, uint32_t* cols,
                         uint32_t* layers) {
    MG_CHECK(p && ptr && rows && cols && layers, MG_ERR_INVALID, "train_capture: null argument");
    MG_CHECK(p->ws_base, MG_ERR_STATE, "train_capture: no train call yet");
    const float* bufs[4] = {p->ws.x, p->ws.v, p->ws.dhb, p->ws.dvb};
    MG_CHECK(which < 4, MG_ERR_INVALID, "train_capture: unknown capture %u", which);
    *ptr = bufs[which];
    *rows = p->B;
    *cols = (which & 1) ? p->pv.hidden : MG_EMBED;
    *layers = p->pv.layers;
    return MG_OK;
}

int mg_ppo_adam_state(mg_ppo* p, float** m, float** v, uint32_t* step) {
    MG_CHECK(p, MG_ERR_INVALID, "adam_state: null model");
    if (m) *m = p->m;
    if (v) *v = p->v;
    if (step) *step = p->step;
    return MG_OK;
}

int mg_ppo_set_log_std(mg_ppo* p, float value) {
    MG_CHECK(p, MG_ERR_INVALID, "set_log_std: null model");
    MG_CHECK(p->pv.continuous, MG_ERR_STATE, "setLogStd needs a continuous Env::Action");
    std::vector<float> v(p->pv.act_dim, value);
    MG_HIP(hipMemcpyAsync(p->pv.params + p->pv.off_log_std, v.data(), v.size() * 4, hipMemcpyHostToDevice,
                          p->gym->stream),
           "set_log_std upload");
    MG_HIP(hipStreamSynchronize(p->gym->stream), "set_log_std synchronize");
    return MG_OK;
}

int mg_ppo_last_order(mg_ppo* p, uint32_t* out, uint32_t capacity, uint32_t* count) {
    MG_CHECK(p && count, MG_ERR_INVALID, "last_order: null argument");
    *count = (uint32_t)p->last_order.size();
    if (out) memcpy(out, p->last_order.data(), std::min<size_t>(capacity, p->last_order.size()) * 4);
    return MG_OK;
}

int mg_ppo_sample(mg_ppo* p, const float* head, uint32_t rows, uint32_t* rng, void* actions, float* logp,
                  float* value) {
    MG_CHECK(p && head && rng && actions && logp && value, MG_ERR_INVALID, "sample: null argument");
    int rc = launch_sample(p->gym->stream, p->pv, head, rows, rng, actions, logp, value);
    if (rc) return rc;
    MG_HIP(hipStreamSynchronize(p->gym->stream), "sample synchronize");
    return MG_OK;
}

int mg_gae(void* stream, const float* reward, const uint8_t* done, const float* value, const float* head,
           uint32_t head_dim, uint32_t act_dim, uint32_t n, uint32_t horizon, float gamma, float lambda,
           float* advantage, float* ret) {
    MG_CHECK(reward && done && value && head && advantage && ret, MG_ERR_INVALID, "gae: null argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    int rc;
    {
        TimedLaunch tl(MG_K_GAE, st);
        rc = launch_gae(st, reward, done, value, head, head_dim, act_dim, n, horizon, gamma, lambda, advantage, ret);
    }
    if (rc) return rc;
    MG_HIP(hipStreamSynchronize(st), "gae synchronize");
    return MG_OK;
}

}  // extern "C"
