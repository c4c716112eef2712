// Library runtime: errors, memory helpers, the env registry, kernel timing and
// the Gym object (gym.h:15-122).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "internal.h"
#include "mg/env.h"

namespace mg {

static thread_local std::string g_error;

int set_error(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

void clear_error() { g_error.clear(); }

int launcher_status(int rc, const char* what) {
    if (rc == 0) return MG_OK;
    if (rc > 0) return set_error(MG_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString((hipError_t)rc));
    return set_error(rc, "%s: invalid launch arguments", what);
}

int device_alloc(void** p, size_t bytes, const char* what) {
    *p = nullptr;
    if (bytes == 0) return MG_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        return set_error(e == hipErrorOutOfMemory ? MG_ERR_OOM : MG_ERR_HIP, "%s: hipMalloc(%zu): %s", what, bytes,
                         hipGetErrorString(e));
    }
    return MG_OK;
}

// ---- kernel timing ----------------------------------------------------------
namespace {
struct Pending {
    int kernel;
    hipEvent_t start, stop;
};
struct Timing {
    std::mutex mu;
    bool on = false;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;
    mg_kernel_times acc{};
    hipEvent_t get() {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
    void resolve() {
        for (auto& p : pending) {
            if (hipEventSynchronize(p.stop) == hipSuccess) {
                float ms = 0.0f;
                if (hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
                    acc.total_ms[p.kernel] += ms;
                    acc.launches[p.kernel] += 1;
                }
            }
            pool.push_back(p.start);
            pool.push_back(p.stop);
        }
        pending.clear();
    }
};
Timing& timing() {
    static Timing t;
    return t;
}
}  // namespace

TimedLaunch::TimedLaunch(int kernel, hipStream_t stream) : kernel_(kernel), stream_(stream), start_(nullptr) {
    Timing& t = timing();
    if (!t.on) return;
    std::lock_guard<std::mutex> lk(t.mu);
    hipEvent_t e = t.get();
    if (e && hipEventRecord(e, stream) == hipSuccess) start_ = e;
}

TimedLaunch::~TimedLaunch() {
    if (!start_) return;
    Timing& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    hipEvent_t e = t.get();
    if (e && hipEventRecord(e, stream_) == hipSuccess) {
        t.pending.push_back({kernel_, (hipEvent_t)start_, e});
        if (t.pending.size() > 4096) t.resolve();
    }
}

// ---- env registry -------------------------------------------------------------
namespace {
std::vector<const mg_env_desc*>& registry() {
    static std::vector<const mg_env_desc*> r;
    return r;
}
std::mutex& registry_mu() {
    static std::mutex m;
    return m;
}
}  // namespace

}  // namespace mg

using namespace mg;

extern "C" {

const char* mg_last_error(void) { return g_error.c_str(); }
int mg_abi_version(void) { return MG_ABI_VERSION; }

int mg_device_count(int* count) {
    MG_CHECK(count, MG_ERR_INVALID, "mg_device_count: null output");
    MG_HIP(hipGetDeviceCount(count), "hipGetDeviceCount");
    return MG_OK;
}
int mg_malloc(void** ptr, size_t bytes) {
    MG_CHECK(ptr, MG_ERR_INVALID, "mg_malloc: null output");
    return device_alloc(ptr, bytes, "mg_malloc");
}
int mg_free(void* ptr) {
    if (ptr) MG_HIP(hipFree(ptr), "hipFree");
    return MG_OK;
}
int mg_host_alloc(void** ptr, size_t bytes) {
    MG_CHECK(ptr, MG_ERR_INVALID, "mg_host_alloc: null output");
    MG_HIP(hipHostMalloc(ptr, bytes, hipHostMallocDefault), "hipHostMalloc");
    return MG_OK;
}
int mg_host_free(void* ptr) {
    if (ptr) MG_HIP(hipHostFree(ptr), "hipHostFree");
    return MG_OK;
}
int mg_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    MG_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return MG_OK;
}
int mg_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    MG_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return MG_OK;
}
int mg_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    {
        TimedLaunch tl(MG_K_COPY, nullptr);
        MG_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, nullptr), "hipMemcpyAsync D2D");
    }
    MG_HIP(hipStreamSynchronize(nullptr), "hipMemcpy D2D synchronize");
    return MG_OK;
}
int mg_memset(void* dst, int value, size_t bytes) {
    MG_HIP(hipMemset(dst, value, bytes), "hipMemset");
    return MG_OK;
}
int mg_synchronize(void) {
    MG_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return MG_OK;
}

int mg_env_register(const mg_env_desc* desc) {
    MG_CHECK(desc && desc->kernel && desc->rollout, MG_ERR_INVALID, "mg_env_register: incomplete descriptor");
    MG_CHECK(desc->abi_version == MG_ABI_VERSION, MG_ERR_INVALID, "mg_env_register(%s): ABI version %u, library %d",
             desc->kernel, desc->abi_version, MG_ABI_VERSION);
    std::lock_guard<std::mutex> lk(registry_mu());
    for (auto& d : registry()) {
        if (strcmp(d->kernel, desc->kernel) == 0) {
            d = desc;  // a later registration replaces an earlier one
            return MG_OK;
        }
    }
    registry().push_back(desc);
    return MG_OK;
}

int mg_env_lookup(const char* kernel, const mg_env_desc** out) {
    MG_CHECK(kernel && out, MG_ERR_INVALID, "mg_env_lookup: null argument");
    std::lock_guard<std::mutex> lk(registry_mu());
    for (auto* d : registry()) {
        if (strcmp(d->kernel, kernel) == 0) {
            *out = d;
            return MG_OK;
        }
    }
    *out = nullptr;
    return set_error(MG_ERR_NOT_FOUND, "env kernel '%s' is not registered (missing MG_DEFINE_ENV?)", kernel);
}

int mg_env_count(void) {
    std::lock_guard<std::mutex> lk(registry_mu());
    return (int)registry().size();
}

const char* mg_env_name(int index) {
    std::lock_guard<std::mutex> lk(registry_mu());
    if (index < 0 || index >= (int)registry().size()) return nullptr;
    return registry()[index]->kernel;
}

int mg_timing_enable(int on) {
    Timing& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    t.on = on != 0;
    return MG_OK;
}
int mg_timing_get(mg_kernel_times* out) {
    MG_CHECK(out, MG_ERR_INVALID, "mg_timing_get: null output");
    Timing& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    t.resolve();
    *out = t.acc;
    return MG_OK;
}
int mg_timing_reset(void) {
    Timing& t = timing();
    std::lock_guard<std::mutex> lk(t.mu);
    t.resolve();
    t.acc = mg_kernel_times{};
    return MG_OK;
}

// ---- Gym (gym.h:15-122) --------------------------------------------------------

int mg_gym_create(const char* kernel, uint32_t n, uint32_t seed, mg_gym** out) {
    MG_CHECK(out, MG_ERR_INVALID, "mg_gym_create: null output");
    *out = nullptr;
    MG_CHECK(n > 0, MG_ERR_INVALID, "Gym: the env count must be positive");
    const mg_env_desc* env = nullptr;
    int rc = mg_env_lookup(kernel, &env);
    if (rc) return rc;
    mg_gym* g = new mg_gym{};
    g->env = env;
    g->n = n;
    g->seed = seed;
    auto fail = [&](int code) {
        mg_gym_destroy(g);
        return code;
    };
    // A blocking stream: the synchronous mg_memcpy_* helpers (null stream) then
    // order after the gym's queued work.
    if (hipStreamCreate(&g->stream) != hipSuccess)
        return fail(set_error(MG_ERR_HIP, "Gym: hipStreamCreate failed"));
    const size_t N = n;
    if ((rc = device_alloc(&g->state, N * env->state_bytes, "Gym state")) ||
        (rc = device_alloc(&g->actions, N * env->action_bytes, "Gym actions")) ||
        (rc = device_alloc((void**)&g->obs, N * env->obs_dim * sizeof(float), "Gym obs")) ||
        (rc = device_alloc((void**)&g->reward, N * sizeof(float), "Gym reward")) ||
        (rc = device_alloc((void**)&g->done, N, "Gym done")) ||
        (rc = device_alloc((void**)&g->rng, N * sizeof(uint32_t), "Gym rng")))
        return fail(rc);
    // gym.h:54-61: done = 1 so the first step resets every env; actions = 0;
    // one nonzero xorshift seed per env.
    std::vector<uint32_t> seeds(n);
    for (uint32_t i = 0; i < n; ++i) seeds[i] = env_seed(seed, i);
    if (hipMemsetAsync(g->state, 0, N * env->state_bytes, g->stream) != hipSuccess ||
        hipMemsetAsync(g->actions, 0, N * env->action_bytes, g->stream) != hipSuccess ||
        hipMemsetAsync(g->obs, 0, N * env->obs_dim * sizeof(float), g->stream) != hipSuccess ||
        hipMemsetAsync(g->reward, 0, N * sizeof(float), g->stream) != hipSuccess ||
        hipMemsetAsync(g->done, 1, N, g->stream) != hipSuccess ||
        hipMemcpyAsync(g->rng, seeds.data(), N * sizeof(uint32_t), hipMemcpyHostToDevice, g->stream) != hipSuccess ||
        hipStreamSynchronize(g->stream) != hipSuccess)
        return fail(set_error(MG_ERR_HIP, "Gym: buffer initialisation failed"));
    *out = g;
    return MG_OK;
}

int mg_gym_destroy(mg_gym* g) {
    if (!g) return MG_OK;
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    (void)hipFree(g->state);
    (void)hipFree(g->actions);
    (void)hipFree(g->obs);
    (void)hipFree(g->reward);
    (void)hipFree(g->done);
    (void)hipFree(g->rng);
    if (g->stream) (void)hipStreamDestroy(g->stream);
    delete g;
    return MG_OK;
}

int mg_gym_buffers_get(mg_gym* g, mg_gym_buffers* out) {
    MG_CHECK(g && out, MG_ERR_INVALID, "mg_gym_buffers_get: null argument");
    out->stream = g->stream;
    out->env = g->env;
    out->n = g->n;
    out->seed = g->seed;
    out->state = g->state;
    out->actions = g->actions;
    out->obs = g->obs;
    out->reward = g->reward;
    out->done = g->done;
    out->rng = g->rng;
    return MG_OK;
}

static int gym_rollout(mg_gym* g, uint32_t steps, uint32_t mode, const void* actions_in, void* actions_out,
                       float* obs_out, float* reward_out, uint8_t* done_out) {
    MG_CHECK(g, MG_ERR_INVALID, "gym rollout: null gym");
    MG_CHECK(mode == MG_ACTIONS_RANDOM || actions_in, MG_ERR_INVALID, "gym rollout: null actions");
    mg_rollout_args a{};
    a.stream = g->stream;
    a.n = g->n;
    a.steps = steps;
    a.mode = mode;
    a.state = g->state;
    a.rng = g->rng;
    a.done = g->done;
    a.actions_in = actions_in;
    a.actions_out = actions_out;
    a.obs_out = obs_out;
    a.reward_out = reward_out;
    a.done_out = done_out;
    TimedLaunch tl(MG_K_ROLLOUT, g->stream);
    return launcher_status(g->env->rollout(&a), g->env->kernel);
}

int mg_gym_step_into(mg_gym* g, const void* actions_in, float* obs_out, float* reward_out) {
    return gym_rollout(g, 1, MG_ACTIONS_GIVEN, actions_in, nullptr, obs_out, reward_out, nullptr);
}

int mg_gym_run(mg_gym* g) {
    MG_CHECK(g, MG_ERR_INVALID, "mg_gym_run: null gym");
    return gym_rollout(g, 1, MG_ACTIONS_GIVEN, g->actions, nullptr, g->obs, g->reward, nullptr);
}

int mg_gym_rollout_random(mg_gym* g, uint32_t steps, void* actions_out, float* obs_out, float* reward_out,
                          uint8_t* done_out) {
    return gym_rollout(g, steps, MG_ACTIONS_RANDOM, nullptr, actions_out, obs_out, reward_out, done_out);
}

int mg_gym_rollout_given(mg_gym* g, uint32_t steps, const void* actions_in, float* obs_out, float* reward_out,
                         uint8_t* done_out) {
    return gym_rollout(g, steps, MG_ACTIONS_GIVEN, actions_in, nullptr, obs_out, reward_out, done_out);
}

int mg_gym_sync(mg_gym* g) {
    MG_CHECK(g, MG_ERR_INVALID, "mg_gym_sync: null gym");
    MG_HIP(hipStreamSynchronize(g->stream), "Gym: stream synchronize");
    return MG_OK;
}

}  // extern "C"
