// One PPO minibatch update (model/ppo.h:906-916) as four launches:
//
//  1. train_rows: per 32-row tile, the forward recompute with activation
//     capture (model/ppo.h:909), the loss and head gradient
//     (model/policy.metal:14-69 / model/gaussian.metal:76-135) and the whole
//     backward dX chain (model/ppo.h:793-865) on fp32 MFMA, writing the
//     activations and gradients the weight gradients need.
//  2. train_dw: every weight gradient as a sum over rows, split into kSplits
//     row ranges: 64x64 MFMA tiles of X^T dY for the block matrices, column
//     sums for the vector parameters, the head and log_std.
//  3. grad_reduce: sums the splits in fixed order, the global squared norm
//     (last-workgroup pattern, fixed order) and the minibatch's LossStats.
//  4. adam: clip scale and Adam (model/optimizer.metal:36-60).
//
// Every reduction has a fixed order, so a rerun gives the same bits (the
// reference uses float atomics for several of these).
#include <string.h>

#include "kernels.h"
#include "mg/device/policy.h"
#include "mg/device/sample.h"

namespace mg {
namespace dev {

constexpr int kTR = 32;  // rows per train_rows workgroup
constexpr int kMaxHeadT = 64;
constexpr int kMaxObsT = 64;

struct RowsArgs {
    mg_policy_view pv;
    TrainWs ws;
    TrainStep step;
    mg_ppo_hparams hp;
    const float* obs_slots;
    const void* action_slots;
    const float* adv_slots;
    const float* ret_slots;
    const float* logp_slots;
    const float* adv_stats;
    float* head_out;
};

// Gradient at the final LN output: dX = dZ W_head^T (model/linear.metal:40-60).
template <int M>
__device__ __forceinline__ void bwd_head(const mg_policy_view& pv, const float* dheadL, int HD, FwdRegs<M>& G) {
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, col = 32 * w + (lane & 31);
    const float* Wh = pv.params + pv.off_head + col * HD;
#pragma unroll
    for (int rt = 0; rt < FwdRegs<M>::RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) G.h[rt][r] = 0.0f;
    for (int j = 0; j < HD; ++j) {
        const float wj = Wh[j];
#pragma unroll
        for (int rt = 0; rt < FwdRegs<M>::RT; ++rt)
#pragma unroll
            for (int r = 0; r < 16; ++r) G.h[rt][r] += dheadL[(32 * rt + c32_row(r, lane)) * HD + j] * wj;
    }
}

// model/layernorm.metal:74-127 on a register tile: G holds the gradient at the
// LN output on entry (also stored to dx_store, [M][128]) and the gradient at
// the LN input on exit. xn/sd are the tile's forward captures.
template <int M>
__device__ __forceinline__ void bwd_layernorm(FwdSmem<M>& sm, FwdRegs<M>& G, const float* xn, const float* sd,
                                              const float* gamma, float* dx_store) {
    constexpr int TPR = 256 / M, CPT = kEmbed / TPR;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, col = 32 * w + (lane & 31);
#pragma unroll
    for (int rt = 0; rt < FwdRegs<M>::RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 32 * rt + c32_row(r, lane);
            sm.xs[row * kLds + col] = G.h[rt][r];
            dx_store[row * kEmbed + col] = G.h[rt][r];
        }
    __syncthreads();
    const int row = tid / TPR, part = tid % TPR, c0 = part * CPT;
    float* zr = sm.xs + row * kLds + c0;
    const float* xr = xn + row * kEmbed + c0;
    float dxn[CPT], xv[CPT];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        xv[c] = xr[c];
        dxn[c] = zr[c] * gamma[c0 + c];
        s1 += dxn[c];
        s2 += dxn[c] * xv[c];
    }
    s1 = group_sum<TPR>(s1);
    s2 = group_sum<TPR>(s2);
    const float r1 = s1 / (float)kEmbed, r2 = s2 / (float)kEmbed, rd = 1.0f / sd[row];
#pragma unroll
    for (int c = 0; c < CPT; ++c) zr[c] = rd * (dxn[c] - r1 - xv[c] * r2);
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < FwdRegs<M>::RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) G.h[rt][r] = sm.xs[(32 * rt + c32_row(r, lane)) * kLds + col];
    __syncthreads();
}

// Backward of block l (model/mlp.metal:88-153 + model/ppo.h:851-852). D holds
// the gradient at the block output (dStream) and is updated in place to the
// gradient at the block input. Chunked like the forward: dV_c = (dh Down_c^T)
// masked by relu, then dx += dV_c Up_c^T; both weight reads are contiguous
// float4s along the contraction.
template <int M>
__device__ __forceinline__ void bwd_block(const mg_policy_view& pv, int l, FwdSmem<M>& sm, FwdRegs<M>& D,
                                          const float* v_tile, float* dv_store, float* dh_store, const float* xn_tile,
                                          const float* sd_tile, float* dx_store) {
    constexpr int RT = FwdRegs<M>::RT;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, n = lane & 31, hh = lane >> 5;
    const int H = (int)pv.hidden;
    const float* Up = pv.params + pv.off_up[l];
    const float* Dn = pv.params + pv.off_down[l];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 32 * rt + c32_row(r, lane);
            sm.xs[row * kLds + 32 * w + n] = D.h[rt][r];
            dh_store[row * kEmbed + 32 * w + n] = D.h[rt][r];
        }
    __syncthreads();
    FwdRegs<M> G;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) G.h[rt] = f32x16{};
    for (int c = 0; c < H / kChunk; ++c) {
        f32x16 v[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) v[rt] = f32x16{};
        const float* bp = Dn + (size_t)(kChunk * c + 32 * w + n) * kEmbed + 4 * hh;
        const float* ap = sm.xs + n * kLds + 4 * hh;
#pragma unroll
        for (int g = 0; g < kEmbed / 8; ++g) {
            const f32x4 b = *reinterpret_cast<const f32x4*>(bp + 8 * g);
            f32x4 a[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) a[rt] = *reinterpret_cast<const f32x4*>(ap + 32 * rt * kLds + 8 * g);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) v[rt] = mfma32x32x2(a[rt][j], b[j], v[rt]);
        }
        __syncthreads();
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 32 * rt + c32_row(r, lane);
                const int hid = kChunk * c + 32 * w + n;
                const float x = v_tile[(size_t)row * H + hid] > 0.0f ? v[rt][r] : 0.0f;
                sm.vs[row * kLds + 32 * w + n] = x;
                dv_store[(size_t)row * H + hid] = x;
            }
        __syncthreads();
        const float* bp2 = Up + (size_t)(32 * w + n) * H + kChunk * c + 4 * hh;
        const float* ap2 = sm.vs + n * kLds + 4 * hh;
#pragma unroll
        for (int g = 0; g < kChunk / 8; ++g) {
            const f32x4 b = *reinterpret_cast<const f32x4*>(bp2 + 8 * g);
            f32x4 a[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) a[rt] = *reinterpret_cast<const f32x4*>(ap2 + 32 * rt * kLds + 8 * g);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) G.h[rt] = mfma32x32x2(a[rt][j], b[j], G.h[rt]);
        }
    }
    __syncthreads();
    bwd_layernorm<M>(sm, G, xn_tile, sd_tile, pv.params + pv.off_ln_gamma[l], dx_store);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) D.h[rt] = G.h[rt] + D.h[rt];  // residualAdd(dBranch, dStream)
}

template <int M>
__global__ void __launch_bounds__(256) train_rows_kernel(const RowsArgs a) {
    __shared__ FwdSmem<M> sm;
    __shared__ float obsL[M * kMaxObsT];
    __shared__ float headL[M * kMaxHeadT];
    __shared__ float dheadL[M * kMaxHeadT];
    FwdRegs<M> R;
    const mg_policy_view& pv = a.pv;
    const TrainWs& ws = a.ws;
    const int O = (int)pv.obs_dim, A = (int)pv.act_dim, HD = (int)pv.head_dim, H = (int)pv.hidden;
    const int NL = (int)pv.layers;
    const uint32_t B = a.step.rows;
    const uint32_t r0 = blockIdx.x * M;           // row within the minibatch
    const size_t g0 = (size_t)a.step.row0 + r0;   // row within the slot arrays
    const int tid = threadIdx.x;

    for (int idx = tid; idx < M * O; idx += 256) obsL[idx] = a.obs_slots[g0 * O + idx];
    __syncthreads();

    // ---- forward with capture ----
    fwd_embed<M>(pv, obsL, O, R);
    for (int l = 0; l < NL; ++l) {
        fwd_layernorm<M>(sm, R, pv.params + pv.off_ln_gamma[l], pv.params + pv.off_ln_beta[l],
                         ws.xn + ((size_t)l * B + r0) * kEmbed, ws.sd + (size_t)l * B + r0,
                         ws.x + ((size_t)l * B + r0) * kEmbed);
        fwd_block<M>(pv, l, sm, R, ws.v + ((size_t)l * B + r0) * H);
    }
    fwd_layernorm<M>(sm, R, pv.params + pv.off_ln_gamma[NL], pv.params + pv.off_ln_beta[NL],
                     ws.xn + ((size_t)NL * B + r0) * kEmbed, ws.sd + (size_t)NL * B + r0,
                     ws.x + ((size_t)NL * B + r0) * kEmbed);
    fwd_head<M>(pv, sm, headL, HD);

    // ---- loss and head gradient, one lane per row ----
    if (tid < M) {
        const float* h = headL + tid * HD;
        float* dz = dheadL + tid * HD;
        const size_t gr = g0 + tid;
        const float mean = a.adv_stats[2 * a.step.block], inv = a.adv_stats[2 * a.step.block + 1];
        const float an = (a.adv_slots[gr] - mean) * inv;
        const float oldLp = a.logp_slots[gr];
        const float scale = 1.0f / (float)B;
        const float clip = a.hp.clip, ec = a.hp.entropy_coef;
        float entropy = 0.0f, logpA, ratio, gLogp, policyLoss;
        if (!pv.continuous) {  // model/policy.metal:14-69
            float rowMax = -__builtin_huge_valf();
            for (int j = 0; j < A; ++j) rowMax = rowMax < h[j] ? h[j] : rowMax;
            float s = 0.0f;
            for (int j = 0; j < A; ++j) s += mg::expf(h[j] - rowMax);
            const float lse = rowMax + mg::logf(s);
            for (int j = 0; j < A; ++j) {
                const float lp = h[j] - lse;
                entropy -= mg::expf(lp) * lp;
            }
            const int act = static_cast<const int*>(a.action_slots)[gr];
            logpA = h[act] - lse;
            ratio = mg::expf(logpA - oldLp);
            const float surr1 = ratio * an;
            const float cr = fminf(fmaxf(ratio, 1.0f - clip), 1.0f + clip);
            const float surr2 = cr * an;
            policyLoss = -(surr1 < surr2 ? surr1 : surr2);
            gLogp = (surr1 <= surr2) ? -an * ratio : 0.0f;
            for (int j = 0; j < A; ++j) {
                const float lp = h[j] - lse;
                const float prob = mg::expf(lp);
                const float g = gLogp * ((j == act ? 1.0f : 0.0f) - prob) + ec * prob * (lp + entropy);
                dz[j] = g * scale;
            }
        } else {  // model/gaussian.metal:76-135
            const float* act = static_cast<const float*>(a.action_slots) + gr * A;
            const float* logStd = pv.params + pv.off_log_std;
            float logp = 0.0f;
            for (int k = 0; k < A; ++k) {
                const float ls = logStd[k];
                const float d = (act[k] - h[k]) * mg::expf(-ls);
                logp += -0.5f * d * d - ls - kLogSqrt2Pi;
                entropy += ls + kLogSqrt2Pi + 0.5f;
            }
            logpA = logp;
            ratio = mg::expf(logp - oldLp);
            const float surr1 = ratio * an;
            const float cr = fminf(fmaxf(ratio, 1.0f - clip), 1.0f + clip);
            const float surr2 = cr * an;
            policyLoss = -(surr1 < surr2 ? surr1 : surr2);
            gLogp = (surr1 <= surr2) ? -an * ratio : 0.0f;
            for (int k = 0; k < A; ++k) {
                const float ls = logStd[k];
                const float invStd = mg::expf(-ls);
                const float d = (act[k] - h[k]) * invStd;
                dz[k] = gLogp * d * invStd * scale;
                ws.dls[(r0 + tid) * A + k] = (gLogp * (d * d - 1.0f) - ec) * scale;
            }
        }
        const float vErr = h[A] - a.ret_slots[gr];
        dz[A] = a.hp.value_coef * vErr * scale;
        float* st = ws.rowstats + (size_t)(r0 + tid) * 5;
        st[0] = policyLoss;
        st[1] = 0.5f * a.hp.value_coef * vErr * vErr;
        st[2] = entropy;
        st[3] = oldLp - logpA;
        st[4] = (fabsf(ratio - 1.0f) > clip) ? 1.0f : 0.0f;
        for (int j = 0; j < HD; ++j) {
            ws.dhead[(size_t)(r0 + tid) * HD + j] = dz[j];
            if (a.head_out) a.head_out[(size_t)(r0 + tid) * HD + j] = h[j];
        }
    }
    __syncthreads();

    // ---- backward ----
    FwdRegs<M> D;
    bwd_head<M>(pv, dheadL, HD, D);
    bwd_layernorm<M>(sm, D, ws.xn + ((size_t)NL * B + r0) * kEmbed, ws.sd + (size_t)NL * B + r0,
                     pv.params + pv.off_ln_gamma[NL], ws.dxl + ((size_t)NL * B + r0) * kEmbed);
    for (int l = NL - 1; l >= 0; --l) {
        bwd_block<M>(pv, l, sm, D, ws.v + ((size_t)l * B + r0) * H, ws.dvb + ((size_t)l * B + r0) * H,
                     ws.dhb + ((size_t)l * B + r0) * kEmbed, ws.xn + ((size_t)l * B + r0) * kEmbed,
                     ws.sd + (size_t)l * B + r0, ws.dxl + ((size_t)l * B + r0) * kEmbed);
    }
    {
        const int w = tid >> 6, lane = tid & 63, col = 32 * w + (lane & 31);
#pragma unroll
        for (int rt = 0; rt < FwdRegs<M>::RT; ++rt)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                ws.dh0[(size_t)(r0 + 32 * rt + c32_row(r, lane)) * kEmbed + col] = D.h[rt][r];
    }
}

// ---- weight gradients ---------------------------------------------------------

// A column-sum segment: out[o] = sum over rows of a[r * lda + ia(o)] * b[r * ldb + ib(o)]
// (b == nullptr: sum of the a term alone), for o < count, written at param offset `off`.
struct Seg {
    const float* a;
    const float* b;
    uint32_t lda, ldb;
    uint32_t count;
    uint32_t off;
    uint32_t ncol;  // o = k * ncol + j: a index k (outer), b index j (inner); ncol = 0: both index o
    uint32_t pad;
};
constexpr int kMaxSegs = 24;

// A big tile job: C[m][n] = sum_r X[r][m] Y[r][n] for a 128 x H (or H x 128) matrix.
struct BigMat {
    const float* x;
    const float* y;
    uint32_t ldx, ldy;  // row strides
    uint32_t mdim, ndim;
    uint32_t off;
    uint32_t pad;
};
constexpr int kMaxBig = 2 * MG_MAX_LAYERS;

struct DwArgs {
    BigMat big[kMaxBig];
    Seg seg[kMaxSegs];
    uint32_t nbig, nseg;
    uint32_t tiles_per_big[kMaxBig];
    uint32_t big_tiles;   // total 64x64 tiles over all big matrices
    uint32_t small_count; // total small outputs
    uint32_t rows;        // B
    uint32_t splits;      // row splits (gridDim.y)
    uint32_t count;       // arena length
    float* partial;
};

__global__ void __launch_bounds__(256) train_dw_kernel(const DwArgs a) {
    const uint32_t split = blockIdx.y;
    const uint32_t rowsPer = a.rows / a.splits;
    const uint32_t rb = split * rowsPer;
    float* out = a.partial + (size_t)split * a.count;
    if (blockIdx.x < a.big_tiles) {
        // locate the matrix and tile
        uint32_t t = blockIdx.x, m = 0;
        while (t >= a.tiles_per_big[m]) t -= a.tiles_per_big[m], ++m;
        const BigMat& bm = a.big[m];
        const uint32_t ntn = bm.ndim / 64;
        const uint32_t tm = t / ntn, tn = t % ntn;
        const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, nn = lane & 31, hh = lane >> 5;
        const uint32_t m0 = tm * 64 + 32 * (w >> 1), n0 = tn * 64 + 32 * (w & 1);
        const float* xp = bm.x + (size_t)(rb + 4 * hh) * bm.ldx + m0 + nn;
        const float* yp = bm.y + (size_t)(rb + 4 * hh) * bm.ldy + n0 + nn;
        f32x16 acc = f32x16{};
        for (uint32_t g = 0; g < rowsPer / 8; ++g) {
            float av[4], bv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                av[j] = xp[(size_t)(8 * g + j) * bm.ldx];
                bv[j] = yp[(size_t)(8 * g + j) * bm.ldy];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = mfma32x32x2(av[j], bv[j], acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = m0 + c32_row(r, lane);
            out[bm.off + (size_t)row * bm.ndim + n0 + nn] = acc[r];
        }
        return;
    }
    const uint32_t o = (blockIdx.x - a.big_tiles) * 256 + threadIdx.x;
    if (o >= a.small_count) return;
    uint32_t s = 0, oo = o;
    while (oo >= a.seg[s].count) oo -= a.seg[s].count, ++s;
    const Seg& sg = a.seg[s];
    const uint32_t ia = sg.ncol ? oo / sg.ncol : oo;
    const uint32_t ib = sg.ncol ? oo % sg.ncol : oo;
    float acc = 0.0f;
    if (sg.b) {
        for (uint32_t r = rb; r < rb + rowsPer; ++r) acc += sg.a[(size_t)r * sg.lda + ia] * sg.b[(size_t)r * sg.ldb + ib];
    } else {
        for (uint32_t r = rb; r < rb + rowsPer; ++r) acc += sg.a[(size_t)r * sg.lda + ia];
    }
    out[sg.off + oo] = acc;
}

// Sum of the splits per parameter, then the squared norm; the last workgroup
// to finish adds the per-workgroup norms in order and the row stats.
__global__ void __launch_bounds__(256) grad_reduce_kernel(const float* __restrict__ partial, uint32_t splits,
                                                          uint32_t count,
                                                          float* __restrict__ grad, float* __restrict__ normpart,
                                                          float* __restrict__ normsq, unsigned* __restrict__ counter,
                                                          const float* __restrict__ rowstats, uint32_t rows,
                                                          float* __restrict__ mb_stats) {
    __shared__ float red[256 * 5];
    __shared__ bool last;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    float g = 0.0f;
    if (i < count) {
        for (uint32_t s = 0; s < splits; ++s) g += partial[(size_t)s * count + i];
        grad[i] = g;
    }
    red[threadIdx.x] = g * g;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        normpart[blockIdx.x] = red[0];
        __threadfence();
        last = atomicAdd(counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    // normsq = sum of the workgroup norms, fixed tree order
    float s = 0.0f;
    for (uint32_t b = threadIdx.x; b < gridDim.x; b += 256) s += normpart[b];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const float nsq = red[0];
    __syncthreads();
    // model/ppo.h:925-943: LossStats means over the minibatch rows
    float st[5] = {0, 0, 0, 0, 0};
    for (uint32_t r = threadIdx.x; r < rows; r += 256)
#pragma unroll
        for (int q = 0; q < 5; ++q) st[q] += rowstats[(size_t)r * 5 + q];
#pragma unroll
    for (int q = 0; q < 5; ++q) red[q * 256 + threadIdx.x] = st[q];
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o)
#pragma unroll
            for (int q = 0; q < 5; ++q) red[q * 256 + threadIdx.x] += red[q * 256 + threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        normsq[0] = nsq;
        const float inv = 1.0f / (float)rows;
#pragma unroll
        for (int q = 0; q < 5; ++q) mb_stats[q] = red[q * 256] * inv;
        mb_stats[5] = sqrtf(nsq);
        *counter = 0u;
    }
}

// model/optimizer.metal:36-60
__global__ void __launch_bounds__(256) adam_kernel(float* __restrict__ param, const float* __restrict__ grad,
                                                   float* __restrict__ mom, float* __restrict__ var,
                                                   const float* __restrict__ normsq, uint32_t count, float lr,
                                                   float beta1_pow, float beta2_pow, float max_grad_norm) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    const float beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f;
    const float norm = sqrtf(normsq[0]);
    const float scale = (max_grad_norm > 0.0f && norm > max_grad_norm) ? max_grad_norm / (norm + 1e-6f) : 1.0f;
    const float g = grad[i] * scale;
    const float m = beta1 * mom[i] + (1.0f - beta1) * g;
    const float v = beta2 * var[i] + (1.0f - beta2) * g * g;
    mom[i] = m;
    var[i] = v;
    const float mHat = m / (1.0f - beta1_pow);
    const float vHat = v / (1.0f - beta2_pow);
    param[i] = param[i] - lr * mHat / (sqrtf(vHat) + eps);
}

}  // namespace dev

namespace {
size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct WsPlan {
    size_t off[16];
    size_t total;
};

WsPlan plan(const mg_policy_view& pv, uint32_t B) {
    const size_t E = MG_EMBED, L = pv.layers, H = pv.hidden, HD = pv.head_dim, A = pv.act_dim;
    const size_t sizes[16] = {
        (L + 1) * B * E * 4,               // xn
        (L + 1) * B * E * 4,               // x
        (L + 1) * B * 4,                   // sd
        L * B * H * 4,                     // v
        (L + 1) * B * E * 4,               // dxl
        L * B * E * 4,                     // dhb
        L * B * H * 4,                     // dvb
        B * E * 4,                         // dh0
        B * HD * 4,                        // dhead
        B * 5 * 4,                         // rowstats
        B * (A ? A : 1) * 4,               // dls
        (size_t)kSplits * pv.count * 4,  // partial
        (size_t)pv.count * 4,              // grad
        (((size_t)pv.count + 255) / 256) * 4,  // normpart
        4,                                 // normsq
        4,                                 // counter
    };
    WsPlan p;
    size_t o = 0;
    for (int k = 0; k < 16; ++k) {
        p.off[k] = o;
        o += align256(sizes[k]);
    }
    p.total = o;
    return p;
}
}  // namespace

int train_ws_bytes(const mg_policy_view& pv, uint32_t rows, size_t* bytes) {
    *bytes = plan(pv, rows).total;
    return MG_OK;
}

int train_ws_bind(const mg_policy_view& pv, uint32_t rows, void* base, TrainWs* ws) {
    WsPlan p = plan(pv, rows);
    char* b = static_cast<char*>(base);
    ws->xn = (float*)(b + p.off[0]);
    ws->x = (float*)(b + p.off[1]);
    ws->sd = (float*)(b + p.off[2]);
    ws->v = (float*)(b + p.off[3]);
    ws->dxl = (float*)(b + p.off[4]);
    ws->dhb = (float*)(b + p.off[5]);
    ws->dvb = (float*)(b + p.off[6]);
    ws->dh0 = (float*)(b + p.off[7]);
    ws->dhead = (float*)(b + p.off[8]);
    ws->rowstats = (float*)(b + p.off[9]);
    ws->dls = (float*)(b + p.off[10]);
    ws->partial = (float*)(b + p.off[11]);
    ws->grad = (float*)(b + p.off[12]);
    ws->normpart = (float*)(b + p.off[13]);
    ws->normsq = (float*)(b + p.off[14]);
    ws->counter = (unsigned*)(b + p.off[15]);
    return MG_OK;
}

int launch_train_step(hipStream_t st, const mg_policy_view& pv, const mg_ppo_hparams& hp, float lr,
                      const TrainWs& ws, const TrainStep& step, const float* obs_slots, const void* action_slots,
                      const float* adv_slots, const float* ret_slots, const float* logp_slots,
                      const float* adv_stats, float* m, float* v, float* head_out, float* mb_stats) {
    const uint32_t B = step.rows;
    MG_CHECK(B % 64 == 0, MG_ERR_INVALID, "train: minibatch %u must be a multiple of 64", B);
    // row splits of the weight-gradient sums: each split covers a multiple of 8 rows
    const uint32_t splits = (B % (8 * kSplits) == 0) ? (uint32_t)kSplits : (uint32_t)kSplits / 2;
    MG_CHECK(pv.obs_dim <= (uint32_t)dev::kMaxObsT && pv.head_dim <= (uint32_t)dev::kMaxHeadT, MG_ERR_INVALID,
             "train: OBS_DIM <= 64 and ACT_DIM + 1 <= 64 required");
    const uint32_t E = MG_EMBED, L = pv.layers, H = pv.hidden, HD = pv.head_dim, A = pv.act_dim, O = pv.obs_dim;

    {  // 1. rows
        TimedLaunch tl(MG_K_TRAIN_ROWS, st);
        dev::RowsArgs ra;
        ra.pv = pv;
        ra.ws = ws;
        ra.step = step;
        ra.hp = hp;
        ra.obs_slots = obs_slots;
        ra.action_slots = action_slots;
        ra.adv_slots = adv_slots;
        ra.ret_slots = ret_slots;
        ra.logp_slots = logp_slots;
        ra.adv_stats = adv_stats;
        ra.head_out = head_out;
        hipLaunchKernelGGL((dev::train_rows_kernel<dev::kTR>), dim3(B / dev::kTR), dim3(256), 0, st, ra);
        MG_HIP(hipGetLastError(), "train rows launch");
    }
    {  // 2. weight gradients
        TimedLaunch tl(MG_K_TRAIN_DW, st);
        dev::DwArgs da;
        memset(&da, 0, sizeof(da));
        da.rows = B;
        da.splits = splits;
        da.count = pv.count;
        da.partial = ws.partial;
        uint32_t nb = 0, tiles = 0;
        for (uint32_t l = 0; l < L; ++l) {
            // dUp_l[k][j] = sum_r x_l[r][k] dV_l[r][j]  (model/mlp.metal:201-203)
            da.big[nb] = {ws.x + (size_t)l * B * E, ws.dvb + (size_t)l * B * H, E, H, E, H, pv.off_up[l], 0};
            da.tiles_per_big[nb] = (E / 64) * (H / 64);
            tiles += da.tiles_per_big[nb++];
            // dDown_l[j][c] = sum_r V_l[r][j] dh_l[r][c]  (model/mlp.metal:205-207)
            da.big[nb] = {ws.v + (size_t)l * B * H, ws.dhb + (size_t)l * B * E, H, E, H, E, pv.off_down[l], 0};
            da.tiles_per_big[nb] = (H / 64) * (E / 64);
            tiles += da.tiles_per_big[nb++];
        }
        da.nbig = nb;
        da.big_tiles = tiles;
        uint32_t ns = 0, small = 0;
        auto seg = [&](const float* a, const float* b, uint32_t lda, uint32_t ldb, uint32_t count, uint32_t off,
                       uint32_t ncol) {
            da.seg[ns++] = {a, b, lda, ldb, count, off, ncol, 0};
            small += count;
        };
        // model/input.metal:38-60: dW_in[k][c] = sum_r obs[r][k] dh0[r][c]; db_in = sum_r dh0
        seg(obs_slots + (size_t)step.row0 * O, ws.dh0, O, E, O * E, pv.off_in_w, E);
        seg(ws.dh0, nullptr, E, 0, E, pv.off_in_b, 0);
        for (uint32_t l = 0; l <= L; ++l) {  // model/layernorm.metal:80-81
            seg(ws.xn + (size_t)l * B * E, ws.dxl + (size_t)l * B * E, E, E, E, pv.off_ln_gamma[l], 0);
            seg(ws.dxl + (size_t)l * B * E, nullptr, E, 0, E, pv.off_ln_beta[l], 0);
        }
        // model/linear.metal:71-93: dW_head[k][j] = sum_r x_f[r][k] dhead[r][j]
        seg(ws.x + (size_t)L * B * E, ws.dhead, E, HD, E * HD, pv.off_head, HD);
        if (pv.continuous) seg(ws.dls, nullptr, A, 0, A, pv.off_log_std, 0);
        da.nseg = ns;
        da.small_count = small;
        dim3 grid(tiles + (small + 255) / 256, splits);
        hipLaunchKernelGGL(dev::train_dw_kernel, grid, dim3(256), 0, st, da);
        MG_HIP(hipGetLastError(), "train dW launch");
    }
    const uint32_t rblocks = (pv.count + 255) / 256;
    {  // 3. reduce + norm + stats
        TimedLaunch tl(MG_K_GRAD_REDUCE, st);
        hipLaunchKernelGGL(dev::grad_reduce_kernel, dim3(rblocks), dim3(256), 0, st, ws.partial, splits, pv.count, ws.grad,
                           ws.normpart, ws.normsq, ws.counter, ws.rowstats, B, mb_stats);
        MG_HIP(hipGetLastError(), "grad reduce launch");
    }
    {  // 4. Adam
        TimedLaunch tl(MG_K_ADAM, st);
        hipLaunchKernelGGL(dev::adam_kernel, dim3(rblocks), dim3(256), 0, st, pv.params, ws.grad, m, v, ws.normsq,
                           pv.count, lr, step.beta1_pow, step.beta2_pow, hp.max_grad_norm);
        MG_HIP(hipGetLastError(), "adam launch");
    }
    return MG_OK;
}

}  // namespace mg
