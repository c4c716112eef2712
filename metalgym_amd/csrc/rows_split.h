// The fp32 row pass of a PPO minibatch (the work of train_rows_kernel<false>:
// forward recompute with capture, loss, backward dX chain, tile partials) in
// the hidden-unit split layout of include/mg/device/policy_split.h, so that no
// chunk GEMM waits on a barrier. Included by train_kernels.hip. The loss
// reduces over the same TPR lanes as LayerNorm. The captures for the weight
// gradients have the row-major layouts of train_rows_kernel<false>.
#pragma once
#include "mg/device/policy_split.h"

namespace mg {
namespace dev {

static_assert(kTR == kSplitRows, "a row-pass tile is a split tile");

template <int W>
struct SkShape {
    static_assert(W == 4 || W == 8, "4 or 8 waves");
    static constexpr int NT = 64 * W;         // threads
    static constexpr int S = 8 / W;           // 16-unit strips per wave and chunk
    static constexpr int TPR = NT / kTR;      // threads per row outside the GEMMs
    static constexpr int CPT = kEmbed / TPR;  // columns per thread
    static constexpr int NV = CPT / 4;        // float4s per thread and row
    // limits of the static LDS; larger shapes use train_rows_kernel<false>
    static constexpr int LAYERS = W == 4 ? MG_MAX_LAYERS : 4;
    static constexpr int HEAD = 16;
    static constexpr int OBS = 48;
};

// LDS of one workgroup.
template <int W>
struct alignas(16) SkSmem {
    using Sh = SkShape<W>;
    float xs[kTR * kLds];        // block input broadcast (X or dh); x_f for dW_head; dh0 for dW_in
    float red[W][kTR * kLds];    // the waves' partials of a block output; W_in / b_in at start-up
    float part[kTR][2][kEmbed];  // per row: xn dZ and dZ of the last LN backward (dgamma, dbeta terms)
    float xn[(Sh::LAYERS + 1) * kTR * kEmbed];  // LN captures for the backward
    float rstd[(Sh::LAYERS + 1) * kTR];  // 1 / sigma of every LN
    float ln[(Sh::LAYERS + 1) * 2 * kEmbed];  // gamma, beta of every LN
    float wh[kEmbed * Sh::HEAD];              // W_head, HC columns (zero past HD), at sk_wh_index
    float obs[kTR * Sh::OBS];
    float acts[kTR * Sh::HEAD];  // the tile's float actions (Gaussian head)
    float lstd[Sh::HEAD];        // log_std (Gaussian head)
    float dhead[kTR * Sh::HEAD];
    float dls[kTR * Sh::HEAD];
    float stat[kTR * 5];
    static_assert((Sh::OBS + 1) * kEmbed <= W * kTR * kLds, "W_in and b_in fit the partial buffer");
};

// The block output: this wave's partial to LDS, a barrier, then the thread's
// row and columns summed over the waves in order.
template <int W>
__device__ __forceinline__ RowVec<SkShape<W>::NV> sk_reduce(SkSmem<W>& L, const f32x4 (&hp)[8], int wave, int row,
                                                            int c0) {
    return sk_reduce_buf<W, SkShape<W>::NV>(&L.red[0][0], hp, wave, row, c0);
}

// model/layernorm.metal:74-127 on a row: g is the gradient at the LN output,
// the result the gradient at its input. The row's terms of the dgamma and
// dbeta sums (xn g and g) go to part.
template <int W>
__device__ __forceinline__ RowVec<SkShape<W>::NV> sk_layernorm_bwd(SkSmem<W>& L, const RowVec<SkShape<W>::NV>& g,
                                                                   int lnIdx, int row, int c0) {
    constexpr int NV = SkShape<W>::NV, CPT = SkShape<W>::CPT, TPR = SkShape<W>::TPR;
    const RowVec<NV> xv = rv_load<NV>(L.xn + (lnIdx * kTR + row) * kEmbed + c0);
    const RowVec<NV> gm = rv_load<NV>(L.ln + lnIdx * 2 * kEmbed + c0);
    RowVec<NV> dxn, prod;
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        dxn[c] = g[c] * gm[c];
        s1 += dxn[c];
        s2 += dxn[c] * xv[c];
        prod[c] = xv[c] * g[c];
    }
    rv_store(&L.part[row][0][c0], prod);
    rv_store(&L.part[row][1][c0], g);
    s1 = group_sum<TPR>(s1);
    s2 = group_sum<TPR>(s2);
    const float r1 = s1 / (float)kEmbed, r2 = s2 / (float)kEmbed, rd = L.rstd[lnIdx * kTR + row];
    RowVec<NV> o;
#pragma unroll
    for (int c = 0; c < CPT; ++c) o[c] = rd * (dxn[c] - r1 - xv[c] * r2);
    return o;
}

// model/layernorm.metal:10-71 on a row held by TPR lanes, returning 1 / sigma
// (one v_rsq_f32, about 1 ulp) for the backward instead of sigma.
template <int TPR, int NV>
__device__ __forceinline__ void sk_layernorm_r(const RowVec<NV>& h, const float* gamma, const float* beta, int c0,
                                               RowVec<NV>& x, RowVec<NV>& xn, float& rstd) {
    constexpr int CPT = 4 * NV;
    float s = h[0];
#pragma unroll
    for (int c = 1; c < CPT; ++c) s += h[c];
    s = group_sum<TPR>(s);
    const float mean = s * (1.0f / (float)kEmbed);
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const float d = h[c] - mean;
        q += d * d;
    }
    q = group_sum<TPR>(q);
    rstd = __builtin_amdgcn_rsqf(q * (1.0f / (float)kEmbed) + 1e-5f);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        xn[c] = (h[c] - mean) * rstd;
        x[c] = gamma[c0 + c] * xn[c] + beta[c0 + c];
    }
}

// The tile's dgamma and dbeta (rows summed in order) from part; after a
// barrier that follows the LN backward. Threads 0 .. 255.
template <int W>
__device__ __forceinline__ void sk_ln_sums(const SkSmem<W>& L, float* tp_gamma, float* tp_beta) {
    const int t = threadIdx.x;
    if (t < 2 * kEmbed) {
        const int c = t & (kEmbed - 1), which = t >> 7;
        float s = 0.0f;
#pragma unroll
        for (int r = 0; r < kTR; ++r) s += L.part[r][which][c];
        (which ? tp_beta : tp_gamma)[c] = s;
    }
}

// W_head (element (k, j): embed row k, head column j < HC) in LDS, laid out
// for the row layout's reads: thread t of a row's TPR holds embed rows
// k = CPT t + c and reads float4 q (columns 4 q .. 4 q + 3) of each, and run
// (c, q) of the TPR threads is contiguous, 16 bytes a thread, so one float4
// read of a wave touches consecutive banks. (Rows of HC floats in k order put
// consecutive threads 4 HC floats apart, several of them on one bank for every
// read: the head took 0.8 K cycles for CartPole and 2.7 K for VoxelNav16.)
template <int TPR, int CPT, int HC>
__device__ __forceinline__ int sk_wh_index(int k, int j) {
    return (((k % CPT) * (HC / 4) + j / 4) * TPR + k / CPT) * 4 + j % 4;
}

// model/linear.metal:17-37 for one row held by TPR lanes: hv[j] = x_f[row] .
// W_head[:, j] (0 for HD <= j < HC), the HC column sums reduced together, so
// every lane of the row holds the whole head. wh: W_head in LDS at
// sk_wh_index, zero past HD, read as float4s.
template <int TPR, int HC, int NV>
__device__ __forceinline__ void sk_head(const RowVec<NV>& x, const float* wh, int c0, float (&hv)[HC]) {
    static_assert(HC % 4 == 0, "float4 rows");
    constexpr int CPT = 4 * NV;
#pragma unroll
    for (int j = 0; j < HC; ++j) hv[j] = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
#pragma unroll
        for (int q = 0; q < HC / 4; ++q) {
            const f32x4 w = *reinterpret_cast<const f32x4*>(wh + sk_wh_index<TPR, CPT, HC>(c0 + c, 4 * q));
#pragma unroll
            for (int i = 0; i < 4; ++i) hv[4 * q + i] += x[c] * w[i];
        }
    }
    group_sum_n<TPR, HC>(hv);
}

// model/policy.metal:14-69 / model/gaussian.metal:76-135 for one row from its
// whole head hv (A actions, HD = A + 1 <= HC columns), computed by every lane
// of the row alike: the head gradient dz[j] (0 from HD on), the Gaussian
// head's log_std gradients dls[j] (j < A) and the row's LossStats terms st.
// Sums over the head columns run in column order. lstd: log_std, actRow: the
// row's A float actions (both LDS, Gaussian head only); act: the discrete
// action.
template <int HC>
__device__ __forceinline__ void sk_loss_row(const RowsArgs& a, const float (&hv)[HC], int A, bool cont,
                                            const float* lstd, const float* actRow, float an, float oldLp, float ret,
                                            int act, float (&dz)[HC], float (&dls)[HC], float (&st)[5]) {
    const float scale = 1.0f / (float)a.step.rows;
    const float clip = a.hp.clip, ec = a.hp.entropy_coef;
    float entropy = 0.0f, logpA = 0.0f, value = 0.0f;
    float pr[HC], lp[HC], is[HC], dd[HC];
#pragma unroll
    for (int j = 0; j < HC; ++j) {
        pr[j] = lp[j] = is[j] = dd[j] = 0.0f;
        value = j == A ? hv[j] : value;
    }
    if (!cont) {  // model/policy.metal:14-69
        float zmax = -__builtin_huge_valf();
#pragma unroll
        for (int j = 0; j < HC; ++j) zmax = j < A ? fmaxf(zmax, hv[j]) : zmax;
        float e = 0.0f;
#pragma unroll
        for (int j = 0; j < HC; ++j)
            if (j < A) e += fast_exp(hv[j] - zmax);
        const float lse = zmax + fast_log(e);
        float za = 0.0f;
#pragma unroll
        for (int j = 0; j < HC; ++j) {
            if (j < A) {
                lp[j] = hv[j] - lse;
                pr[j] = fast_exp(lp[j]);
                entropy -= pr[j] * lp[j];
            }
            za = j == act ? hv[j] : za;
        }
        logpA = za - lse;
    } else {  // model/gaussian.metal:76-135
#pragma unroll
        for (int j = 0; j < HC; ++j) {
            if (j < A) {
                const float ls = lstd[j];
                is[j] = fast_exp(-ls);
                dd[j] = (actRow[j] - hv[j]) * is[j];
                logpA += -0.5f * dd[j] * dd[j] - ls - kLogSqrt2Pi;
                entropy += ls + kLogSqrt2Pi + 0.5f;
            }
        }
    }
    const float ratio = fast_exp(logpA - oldLp);
    const float surr1 = ratio * an;
    const float cr = fminf(fmaxf(ratio, 1.0f - clip), 1.0f + clip);
    const float surr2 = cr * an;
    const float gLogp = (surr1 <= surr2) ? -an * ratio : 0.0f;
    const float vErr = value - ret;
#pragma unroll
    for (int j = 0; j < HC; ++j) {
        float d = 0.0f, l = 0.0f;
        if (j < A) {
            if (!cont) {
                d = (gLogp * ((j == act ? 1.0f : 0.0f) - pr[j]) + ec * pr[j] * (lp[j] + entropy)) * scale;
            } else {
                d = gLogp * dd[j] * is[j] * scale;
                l = (gLogp * (dd[j] * dd[j] - 1.0f) - ec) * scale;
            }
        }
        dz[j] = j == A ? a.hp.value_coef * vErr * scale : d;
        dls[j] = l;
    }
    st[0] = -(surr1 < surr2 ? surr1 : surr2);
    st[1] = 0.5f * a.hp.value_coef * vErr * vErr;
    st[2] = entropy;
    st[3] = oldLp - logpA;
    st[4] = (fabsf(ratio - 1.0f) > clip) ? 1.0f : 0.0f;
}

// HC: a compile-time bound on the head width (4, 8 or 16), for the head and
// loss in registers.
template <int W, int HC>
__global__ void __launch_bounds__(64 * W) train_rows_split_kernel(const RowsArgs a) {
    using Sh = SkShape<W>;
    constexpr int M = kTR, NT = Sh::NT, S = Sh::S, TPR = Sh::TPR, CPT = Sh::CPT, NV = Sh::NV;
    static_assert(NT >= 2 * kEmbed, "sk_ln_sums takes one thread per output");
    __shared__ SkSmem<W> L;
    const mg_policy_view& pv = a.pv;
    const TrainWs& ws = a.ws;
    const int O = (int)pv.obs_dim, HD = (int)pv.head_dim, H = (int)pv.hidden, NL = (int)pv.layers;
    const int NC = H / kChunk;
    const uint32_t B = a.step.rows;
    const uint32_t r0 = blockIdx.x * M;          // row within the minibatch
    const size_t g0 = (size_t)a.step.row0 + r0;  // row within the slot arrays
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = tid / TPR, lk = tid % TPR, c0 = CPT * lk;  // this thread's row and columns outside the GEMMs
    const int n16 = lane & 15, q4 = 4 * (lane >> 4);
    float* tp = ws.tp + (size_t)blockIdx.x * ws.tp_count;

    // start-up: every small array's first element per thread is loaded
    // first (branch-free: out-of-range threads load an element in range and
    // drop it), then the weight stream's first loads; the staging stores
    // then wait for the small loads alone (vector memory loads complete in
    // order), so the embed and LN0 overlap the arrival of the first weights
    const int rot = (wave + (int)(blockIdx.x >> 3)) % NC;
    const SkSeq<S> seq{pv.frag_fwd16 + pv.float_group, pv.frag_bwd16 + pv.float_group, NL, NC, wave, rot,
                       (uint32_t)kEmbed * (uint32_t)H};
    SkPos pos{0, 0, 0};
    SkStream<S> wst;
    float* const winL = &L.red[0][0];  // the partial buffer is unused until the first block's reduction
    float* const binL = winL + Sh::OBS * kEmbed;
    const float* lnp = pv.params + pv.off_ln_gamma[0];
    const int n_obs = M * O, n_win = O * kEmbed, n_ln = (NL + 1) * 2 * kEmbed;
    const int A = (int)pv.act_dim;
    float an, oldLp, ret;
    int act = 0;
    {
        // W_in as float4s, all of a thread's issued with the other first loads
        // (VoxelNav16's 3840 floats four loads at a time took two memory round
        // trips of the start-up)
        constexpr int NW4 = (Sh::OBS * kEmbed / 4 + NT - 1) / NT;
        const int n_win4 = n_win / 4;  // O x 128 floats
        float o0 = a.obs_slots[g0 * O + (tid < n_obs ? tid : n_obs - 1)];
        // W_head, HC columns a row, zero past HD
        constexpr int NWH = (kEmbed * HC + NT - 1) / NT;
        float hw[NWH];
#pragma unroll
        for (int u = 0; u < NWH; ++u) {
            const int idx = tid + u * NT, k = idx / HC, j = idx % HC;
            const bool in = idx < kEmbed * HC && j < HD;
            hw[u] = pv.params[pv.off_head + (in ? k * HD + j : 0)];
        }
        f32x4 wv[NW4];
#pragma unroll
        for (int u = 0; u < NW4; ++u) {
            const int i4 = tid + u * NT;
            wv[u] = *reinterpret_cast<const f32x4*>(pv.params + pv.off_in_w + 4 * (i4 < n_win4 ? i4 : n_win4 - 1));
        }
        const float b0 = pv.params[pv.off_in_b + (tid < kEmbed ? tid : 0)];
        const float l0 = lnp[tid < n_ln ? tid : 0];
        const float l1 = lnp[tid + NT < n_ln ? tid + NT : 0];
        float av = 0.0f, ls = 0.0f;
        if (pv.continuous) {  // the Gaussian head's inputs of the loss
            av = static_cast<const float*>(a.action_slots)[g0 * A + (tid < M * A ? tid : 0)];
            ls = pv.params[pv.off_log_std + (tid < A ? tid : 0)];
        }
        {
            const size_t gr = g0 + row;
            const float mean = a.adv_stats[2 * a.step.block], inv = a.adv_stats[2 * a.step.block + 1];
            an = (a.adv_slots[gr] - mean) * inv;
            oldLp = a.logp_slots[gr];
            ret = a.ret_slots[gr];
            if (!pv.continuous) act = static_cast<const int*>(a.action_slots)[gr];
        }
        wst.start(seq, pos);
        if (tid < n_obs) L.obs[tid] = o0;
#pragma unroll
        for (int u = 0; u < NWH; ++u) {
            const int idx = tid + u * NT;
            if (idx < kEmbed * HC) L.wh[sk_wh_index<TPR, CPT, HC>(idx / HC, idx % HC)] = idx % HC < HD ? hw[u] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < NW4; ++u)
            if (tid + u * NT < n_win4) *reinterpret_cast<f32x4*>(winL + 4 * (tid + u * NT)) = wv[u];
        if (tid < kEmbed) binL[tid] = b0;
        if (tid < n_ln) L.ln[tid] = l0;
        if (tid + NT < n_ln) L.ln[tid + NT] = l1;
        if (pv.continuous) {
            if (tid < M * A) L.acts[tid] = av;
            if (tid < A) L.lstd[tid] = ls;
        }
    }
    // the rest, four elements' loads ahead of their stores (CartPole's arrays
    // need no second element)
#pragma unroll 4
    for (int idx = tid + NT; idx < n_obs; idx += NT) L.obs[idx] = a.obs_slots[g0 * O + idx];
#pragma unroll 4
    for (int idx = tid + 2 * NT; idx < n_ln; idx += NT) L.ln[idx] = lnp[idx];
    __syncthreads();

    float* const cx = ws.x;
    float* const cv = ws.v;
    float* const cdh = ws.dhb;
    float* const cdv = ws.dvb;

    // ---- forward with capture: model/input.metal:11-27, then the blocks ----
    RowVec<NV> h;
#pragma unroll
    for (int c = 0; c < CPT; ++c) h[c] = binL[c0 + c];
#pragma unroll 4  // the LDS reads of four observations issued together
    for (int k = 0; k < O; ++k) {
        const float ok = L.obs[row * O + k];
#pragma unroll
        for (int c = 0; c < CPT; ++c) h[c] += ok * winL[k * kEmbed + c0 + c];
    }
    for (int l = 0; l < NL; ++l) {
        RowVec<NV> x, xn;
        float sd;  // 1 / sigma
        sk_layernorm_r<TPR>(h, L.ln + l * 2 * kEmbed, L.ln + l * 2 * kEmbed + kEmbed, c0, x, xn, sd);
        rv_store(L.xn + (l * M + row) * kEmbed + c0, xn);
        if (lk == 0) L.rstd[l * M + row] = sd;
        rv_store(cx + ((size_t)l * B + r0 + row) * kEmbed + c0, x);
        rv_store(L.xs + row * kLds + c0, x);
        __syncthreads();  // X complete; every wave is past its reads of red (and of W_in)
        f32x4 xb[8];
        sk_load_input(L.xs, xb);
        f32x4 hp[8];
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) hp[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float* vrow = cv + ((size_t)l * B + r0 + n16) * H + 16 * S * wave + q4;
        for (int k = 0; k < NC; ++k) {  // model/mlp.metal:18-86 for this wave's units of a chunk
            const SkPos nx = seq.next(pos);
            f32x4 v[S];
#pragma unroll
            for (int s = 0; s < S; ++s) v[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            wst.gemm0(v, xb, seq.role0(nx));
            const int c = seq.chunk(pos);
#pragma unroll
            for (int s = 0; s < S; ++s) {
#pragma unroll
                for (int r = 0; r < 4; ++r) v[s][r] = v[s][r] > 0.0f ? v[s][r] : 0.0f;
                *reinterpret_cast<f32x4*>(vrow + kChunk * c + 16 * s) = v[s];
            }
            wst.gemm1(hp, v, seq.role1(nx), seq.stride1());
            pos = nx;
        }
        h = rv_add(h, sk_reduce<W>(L, hp, wave, row, c0));  // model/elementwise.metal:4-13
    }
    // ---- final LN, head, loss and the head's backward, each row in its lanes'
    // registers (model/ppo.h:616-625, then model/ppo.h:793-806) ----
    RowVec<NV> D;
    {
        RowVec<NV> x, xn;
        float sd;  // 1 / sigma
        sk_layernorm_r<TPR>(h, L.ln + NL * 2 * kEmbed, L.ln + NL * 2 * kEmbed + kEmbed, c0, x, xn, sd);
        rv_store(L.xn + (NL * M + row) * kEmbed + c0, xn);
        if (lk == 0) L.rstd[NL * M + row] = sd;
        rv_store(L.xs + row * kLds + c0, x);  // x_f for dW_head
        float hv[HC], dz[HC], dls[HC], st[5];
        sk_head<TPR, HC>(x, L.wh, c0, hv);
        sk_loss_row<HC>(a, hv, A, pv.continuous != 0, L.lstd, L.acts + row * A, an, oldLp, ret, act, dz, dls, st);
        // lane lk < HD of the row writes head column lk and its gradient
        float hm = 0.0f, dm = 0.0f, lm = 0.0f;
#pragma unroll
        for (int j = 0; j < HC; ++j) {
            hm = j == lk ? hv[j] : hm;
            dm = j == lk ? dz[j] : dm;
            lm = j == lk ? dls[j] : lm;
        }
        if (lk < HD) {
            L.dhead[row * HD + lk] = dm;
            if (a.head_out) a.head_out[(size_t)(r0 + row) * HD + lk] = hm;
        }
        if (pv.continuous && lk < A) L.dls[row * A + lk] = lm;
        if (lk == 0) {
#pragma unroll
            for (int q = 0; q < 5; ++q) L.stat[row * 5 + q] = st[q];
        }
        // model/linear.metal:40-60: the gradient at the final LN output, then its LN
        RowVec<NV> g = rv_zero<NV>();
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
#pragma unroll
            for (int q = 0; q < HC / 4; ++q) {
                const f32x4 w = *reinterpret_cast<const f32x4*>(L.wh + sk_wh_index<TPR, CPT, HC>(c0 + c, 4 * q));
#pragma unroll
                for (int i = 0; i < 4; ++i) g[c] += dz[4 * q + i] * w[i];
            }
        }
        D = sk_layernorm_bwd<W>(L, g, NL, row, c0);
    }
    __syncthreads();  // dhead, dls, the LossStats terms and the LN's part terms written

    // model/linear.metal:71-93 on this tile: dW_head[k][j] = sum_r x_f[r][k] dhead[r][j]
    // (its outputs start at thread 0; the log_std and LossStats sums go to the
    // last waves, which have the fewest of them)
    tile_outer<M, NT>(L.dhead, HD, HD, L.xs, tp + pv.float_group, 1, HD);
    const int tl = tid - (NT - kEmbed);  // thread index within the last 128
    if (pv.continuous && tl >= 0) {  // model/gaussian.metal:166-168, summed over the tile in row order
        float s = 0.0f;
        if (tl < A)
            for (int r = 0; r < M; ++r) s += L.dls[r * A + tl];
        tp[pv.off_log_std + tl] = s;  // and 0 in the arena padding after log_std (A <= 63 < 128)
    }
    if (tl >= 64 && tl < 64 + 5) {  // the tile's LossStats sums, in row order
        const int qq = tl - 64;
        float s = 0.0f;
        for (int r = 0; r < M; ++r) s += L.stat[r * 5 + qq];
        tp[pv.float_group + kEmbed * HD + qq] = s;
    }
    __syncthreads();  // dW_head's reads of x_f in xs are done before xs takes dh

    int lnDone = NL;  // the LN whose dgamma / dbeta terms are in part
    for (int l = NL - 1; l >= 0; --l) {  // model/mlp.metal:88-153 + model/ppo.h:851-852
        rv_store(cdh + ((size_t)l * B + r0 + row) * kEmbed + c0, D);
        rv_store(L.xs + row * kLds + c0, D);
        __syncthreads();  // dh complete; red read; part holds LN lnDone's terms
        sk_ln_sums<W>(L, tp + pv.off_ln_gamma[lnDone], tp + pv.off_ln_beta[lnDone]);
        f32x4 xb[8];
        sk_load_input(L.xs, xb);
        f32x4 hp[8];
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) hp[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const float* vrow = cv + ((size_t)l * B + r0 + n16) * H + 16 * S * wave + q4;
        float* dvrow = cdv + ((size_t)l * B + r0 + n16) * H + 16 * S * wave + q4;
        for (int k = 0; k < NC; ++k) {
            const SkPos nx = seq.next(pos);
            const int c = seq.chunk(pos);
            // this lane's hidden values of the forward: the relu mask (loaded
            // before the GEMM issues its weight refills)
            f32x4 m[S], dv[S];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                m[s] = *reinterpret_cast<const f32x4*>(vrow + kChunk * c + 16 * s);
                dv[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            wst.gemm0(dv, xb, seq.role0(nx));  // dV^T = Down strip . dh^T
#pragma unroll
            for (int s = 0; s < S; ++s) {
#pragma unroll
                for (int r = 0; r < 4; ++r) dv[s][r] = m[s][r] > 0.0f ? dv[s][r] : 0.0f;
                *reinterpret_cast<f32x4*>(dvrow + kChunk * c + 16 * s) = dv[s];
            }
            wst.gemm1(hp, dv, seq.role1(nx), seq.stride1());  // dx += dV Up^T
            pos = nx;
        }
        const RowVec<NV> dx = sk_reduce<W>(L, hp, wave, row, c0);
        D = rv_add(D, sk_layernorm_bwd<W>(L, dx, l, row, c0));  // residualAdd(dBranch, dStream)
        lnDone = l;
    }
    // model/input.metal:38-60 on this tile: dW_in[k][c] = sum_r obs[r][k] dh0[r][c], db_in = sum_r dh0
    rv_store(L.xs + row * kLds + c0, D);
    __syncthreads();
    // LN0's sums on threads 0 .. 255 and db_in's on the waves past them (on 8
    // waves: 256 .. 383), so no wave adds two of the tail's column sums
    sk_ln_sums<W>(L, tp + pv.off_ln_gamma[0], tp + pv.off_ln_beta[0]);
    tile_colsum2<M>(L.xs, nullptr, tp + pv.off_in_b, nullptr, NT >= 3 * kEmbed ? 2 * kEmbed : 0);
    tile_outer<M, NT>(L.obs, O, O, L.xs, tp + pv.off_in_w, kEmbed, 1);
}

// The split row pass's wave count for a policy: 8 (two waves per SIMD, the
// faster) where that LDS layout holds its LN captures, else 4; 0 where
// neither holds the policy (train_rows_kernel<false> then runs).
template <int W>
inline bool rows_split_fits(const mg_policy_view& pv) {
    using Sh = SkShape<W>;
    return pv.layers <= (uint32_t)Sh::LAYERS && pv.head_dim <= (uint32_t)Sh::HEAD && pv.obs_dim <= (uint32_t)Sh::OBS;
}
inline int rows_split_waves(const mg_policy_view& pv) {
    return rows_split_fits<8>(pv) ? 8 : rows_split_fits<4>(pv) ? 4 : 0;
}

}  // namespace dev
}  // namespace mg
