// Env-agnostic policy kernels: forward over arbitrary obs rows (forward()),
// per-row sampling (act() and teacher-forced parity), GAE and the per-block
// advantage statistics used by the PPO loss.
#include "kernels.h"
#include "mg/device/policy_bf16.h"
#include "mg/device/sample.h"

namespace mg {
namespace dev {

constexpr int kMaxObs = 64;   // OBS_DIM limit of the staged forward
constexpr int kMaxHead = 64;  // ACT_DIM + 1 limit (model/ppo.h:117)

// model/ppo.h:575-626 on `rows` obs rows; rows past the end compute on zeros
// and are not stored.
template <int M, bool BF16>
__global__ void __launch_bounds__(256) forward_kernel(const mg_policy_view pv, const float* __restrict__ obs,
                                                      uint32_t rows, float* __restrict__ head) {
    __shared__ typename std::conditional<BF16, FwdSmemB<M>, FwdSmem<M>>::type sm;
    __shared__ float obsL[M * kMaxObs];
    __shared__ float headL[M * kMaxHead];
    FwdRegs<M> R;
    const int O = (int)pv.obs_dim, HD = (int)pv.head_dim;
    const uint32_t row0 = blockIdx.x * M;
    for (int idx = threadIdx.x; idx < M * O; idx += 256) {
        const uint32_t r = row0 + idx / O;
        obsL[idx] = r < rows ? obs[(size_t)row0 * O + idx] : 0.0f;
    }
    __syncthreads();
    if constexpr (BF16)
        policy_forward_b<M>(pv, small_params(pv), sm, R, obsL, O, headL, HD);
    else
        policy_forward<M>(pv, small_params(pv), sm, R, obsL, O, headL, HD);
    for (int idx = threadIdx.x; idx < M * HD; idx += 256) {
        const uint32_t r = row0 + idx / HD;
        if (r < rows) head[(size_t)row0 * HD + idx] = headL[idx];
    }
}

// model/sample.metal:18-47 / model/gaussian.metal:42-71, one thread per row.
__global__ void __launch_bounds__(256) sample_kernel(const mg_policy_view pv, const float* __restrict__ head,
                                                     uint32_t rows, uint32_t* __restrict__ rng, void* actions,
                                                     float* __restrict__ logp, float* __restrict__ value) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const int A = (int)pv.act_dim, HD = (int)pv.head_dim;
    const float* h = head + (size_t)r * HD;
    uint32_t s = rng[r];
    float lp;
    if (pv.continuous) {
        sample_gaussian(h, pv.params + pv.off_log_std, A, s, static_cast<float*>(actions) + (size_t)r * A, lp);
    } else {
        static_cast<int*>(actions)[r] = sample_categorical(h, A, s, lp);
    }
    rng[r] = s;
    logp[r] = lp;
    value[r] = h[A];
}

// model/gae.metal:14-36: one thread per env, reverse scan over the horizon.
// The [t][n] loads of a lane are independent of the scan, so they are issued
// in batches of 8 ahead of the dependent arithmetic.
__global__ void __launch_bounds__(256) gae_kernel(const float* __restrict__ reward, const uint8_t* __restrict__ done,
                                                  const float* __restrict__ value, const float* __restrict__ head,
                                                  uint32_t head_dim, uint32_t act_dim, uint32_t n, uint32_t horizon,
                                                  float gamma, float lambda, float* __restrict__ adv,
                                                  float* __restrict__ ret) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float lastAdv = 0.0f;
    float nextValue = head[(size_t)i * head_dim + act_dim];
    int t = (int)horizon - 1;
    for (; t >= 7; t -= 8) {
        float r[8], v[8];
        uint8_t d[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const size_t k = (size_t)(t - u) * n + i;
            r[u] = reward[k];
            v[u] = value[k];
            d[u] = done[k];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const size_t k = (size_t)(t - u) * n + i;
            const float nonTerminal = d[u] ? 0.0f : 1.0f;
            const float delta = r[u] + gamma * nextValue * nonTerminal - v[u];
            lastAdv = delta + gamma * lambda * nonTerminal * lastAdv;
            adv[k] = lastAdv;
            ret[k] = lastAdv + v[u];
            nextValue = v[u];
        }
    }
    for (; t >= 0; --t) {
        const size_t k = (size_t)t * n + i;
        const float nonTerminal = done[k] ? 0.0f : 1.0f;
        const float delta = reward[k] + gamma * nextValue * nonTerminal - value[k];
        lastAdv = delta + gamma * lambda * nonTerminal * lastAdv;
        adv[k] = lastAdv;
        ret[k] = lastAdv + value[k];
        nextValue = value[k];
    }
}

// model/gae.metal:42-77 for every minibatch block at once: one workgroup per
// block, two passes (mean, then population variance), deterministic tree sums.
__global__ void __launch_bounds__(256) adv_stats_kernel(const float* __restrict__ adv, uint32_t n,
                                                        uint32_t minibatch, float* __restrict__ stats) {
    __shared__ float red[256];
    const uint32_t b = blockIdx.x, perSlot = n / minibatch;
    const float* a = adv + (size_t)(b / perSlot) * n + (size_t)(b % perSlot) * minibatch;
    float s = 0.0f;
    for (uint32_t r = threadIdx.x; r < minibatch; r += 256) s += a[r];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const float mean = red[0] / (float)minibatch;
    __syncthreads();
    float q = 0.0f;
    for (uint32_t r = threadIdx.x; r < minibatch; r += 256) {
        const float d = a[r] - mean;
        q += d * d;
    }
    red[threadIdx.x] = q;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float var = red[0] / (float)minibatch;
        stats[2 * b] = mean;
        stats[2 * b + 1] = 1.0f / (sqrtf(var) + 1e-8f);
    }
}

}  // namespace dev

int launch_forward(hipStream_t st, const mg_policy_view& pv, const float* obs, uint32_t rows, float* head) {
    MG_CHECK(pv.obs_dim <= (uint32_t)dev::kMaxObs && pv.head_dim <= (uint32_t)dev::kMaxHead, MG_ERR_INVALID,
             "forward: OBS_DIM must be <= %d and ACT_DIM + 1 <= %d", dev::kMaxObs, dev::kMaxHead);
    if (rows == 0) return MG_OK;
    if (pv.precision == MG_PRECISION_BF16)
        hipLaunchKernelGGL((dev::forward_kernel<32, true>), dim3((rows + 31) / 32), dim3(256), 0, st, pv, obs, rows,
                           head);
    else
        hipLaunchKernelGGL((dev::forward_kernel<32, false>), dim3((rows + 31) / 32), dim3(256), 0, st, pv, obs, rows,
                           head);
    MG_HIP(hipGetLastError(), "forward launch");
    return MG_OK;
}

int launch_sample(hipStream_t st, const mg_policy_view& pv, const float* head, uint32_t rows, uint32_t* rng,
                  void* actions, float* logp, float* value) {
    if (rows == 0) return MG_OK;
    hipLaunchKernelGGL(dev::sample_kernel, dim3((rows + 255) / 256), dim3(256), 0, st, pv, head, rows, rng, actions,
                       logp, value);
    MG_HIP(hipGetLastError(), "sample launch");
    return MG_OK;
}

int launch_gae(hipStream_t st, const float* reward, const uint8_t* done, const float* value, const float* head,
               uint32_t head_dim, uint32_t act_dim, uint32_t n, uint32_t horizon, float gamma, float lambda,
               float* adv, float* ret) {
    MG_CHECK(act_dim < head_dim, MG_ERR_INVALID, "gae: value column %u outside head width %u", act_dim, head_dim);
    if (n == 0 || horizon == 0) return MG_OK;
    hipLaunchKernelGGL(dev::gae_kernel, dim3((n + 255) / 256), dim3(256), 0, st, reward, done, value, head, head_dim,
                       act_dim, n, horizon, gamma, lambda, adv, ret);
    MG_HIP(hipGetLastError(), "gae launch");
    return MG_OK;
}

int launch_adv_stats(hipStream_t st, const float* adv, uint32_t n, uint32_t horizon, uint32_t minibatch,
                     float* stats) {
    MG_CHECK(minibatch > 0 && n % minibatch == 0, MG_ERR_INVALID, "adv stats: minibatch must divide n");
    const uint32_t blocks = horizon * (n / minibatch);
    hipLaunchKernelGGL(dev::adv_stats_kernel, dim3(blocks), dim3(256), 0, st, adv, n, minibatch, stats);
    MG_HIP(hipGetLastError(), "adv stats launch");
    return MG_OK;
}

}  // namespace mg
