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
    float sd[(Sh::LAYERS + 1) * kTR];
    float ln[(Sh::LAYERS + 1) * 2 * kEmbed];  // gamma, beta of every LN
    float wh[kEmbed * Sh::HEAD];              // W_head
    float obs[kTR * Sh::OBS];
    float head[kTR * Sh::HEAD];
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
    const float r1 = s1 / (float)kEmbed, r2 = s2 / (float)kEmbed, rd = 1.0f / L.sd[lnIdx * kTR + row];
    RowVec<NV> o;
#pragma unroll
    for (int c = 0; c < CPT; ++c) o[c] = rd * (dxn[c] - r1 - xv[c] * r2);
    return o;
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

template <int W>
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

    // start-up: the weight stream's first loads, then every small array's
    // first element per thread before any is stored, so the staging's one
    // memory round trip overlaps the weights' instead of preceding it
    const int rot = (wave + (int)(blockIdx.x >> 3)) % NC;
    const SkSeq<S> seq{pv.frag_fwd16 + pv.float_group, pv.frag_bwd16 + pv.float_group, NL, NC, wave, rot,
                       (uint32_t)kEmbed * (uint32_t)H};
    SkPos pos{0, 0, 0};
    SkStream<S> wst;
    wst.start(seq, pos);
    float* const winL = &L.red[0][0];  // the partial buffer is unused until the first block's reduction
    float* const binL = winL + Sh::OBS * kEmbed;
    const float* lnp = pv.params + pv.off_ln_gamma[0];
    const int n_obs = M * O, n_wh = kEmbed * HD, n_win = O * kEmbed, n_ln = (NL + 1) * 2 * kEmbed;
    {
        // W_in as float4s, all of a thread's issued with the other first loads
        // (VoxelNav16's 3840 floats four loads at a time took two memory round
        // trips of the start-up)
        constexpr int NW4 = (Sh::OBS * kEmbed / 4 + NT - 1) / NT;
        const int n_win4 = n_win / 4;  // O x 128 floats
        const float o0 = tid < n_obs ? a.obs_slots[g0 * O + tid] : 0.0f;
        const float h0 = tid < n_wh ? pv.params[pv.off_head + tid] : 0.0f;
        f32x4 wv[NW4];
#pragma unroll
        for (int u = 0; u < NW4; ++u) {
            const int i4 = tid + u * NT;
            wv[u] = i4 < n_win4 ? *reinterpret_cast<const f32x4*>(pv.params + pv.off_in_w + 4 * i4)
                                : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        const float b0 = tid < kEmbed ? pv.params[pv.off_in_b + tid] : 0.0f;
        const float l0 = tid < n_ln ? lnp[tid] : 0.0f;
        const float l1 = tid + NT < n_ln ? lnp[tid + NT] : 0.0f;
        if (tid < n_obs) L.obs[tid] = o0;
        if (tid < n_wh) L.wh[tid] = h0;
#pragma unroll
        for (int u = 0; u < NW4; ++u)
            if (tid + u * NT < n_win4) *reinterpret_cast<f32x4*>(winL + 4 * (tid + u * NT)) = wv[u];
        if (tid < kEmbed) binL[tid] = b0;
        if (tid < n_ln) L.ln[tid] = l0;
        if (tid + NT < n_ln) L.ln[tid + NT] = l1;
    }
    // the rest, four elements' loads ahead of their stores (CartPole's arrays
    // need no second element)
#pragma unroll 4
    for (int idx = tid + NT; idx < n_obs; idx += NT) L.obs[idx] = a.obs_slots[g0 * O + idx];
#pragma unroll 4
    for (int idx = tid + NT; idx < n_wh; idx += NT) L.wh[idx] = pv.params[pv.off_head + idx];
#pragma unroll 4
    for (int idx = tid + 2 * NT; idx < n_ln; idx += NT) L.ln[idx] = lnp[idx];
    float an, oldLp, ret;
    int act = 0;
    {
        const size_t gr = g0 + row;
        const float mean = a.adv_stats[2 * a.step.block], inv = a.adv_stats[2 * a.step.block + 1];
        an = (a.adv_slots[gr] - mean) * inv;
        oldLp = a.logp_slots[gr];
        ret = a.ret_slots[gr];
        if (!pv.continuous) act = static_cast<const int*>(a.action_slots)[gr];
    }
    __syncthreads();

    float* const cx = ws.x;
    float* const cv = ws.v;
    float* const cdh = ws.dhb;
    float* const cdv = ws.dvb;

    // ---- forward with capture: model/input.metal:11-27, then the blocks ----
    RowVec<NV> h;
#pragma unroll
    for (int c = 0; c < CPT; ++c) h[c] = binL[c0 + c];
    for (int k = 0; k < O; ++k) {
        const float ok = L.obs[row * O + k];
#pragma unroll
        for (int c = 0; c < CPT; ++c) h[c] += ok * winL[k * kEmbed + c0 + c];
    }
    for (int l = 0; l < NL; ++l) {
        RowVec<NV> x, xn;
        float sd;
        sk_layernorm<TPR>(h, L.ln + l * 2 * kEmbed, L.ln + l * 2 * kEmbed + kEmbed, c0, x, xn, sd);
        rv_store(L.xn + (l * M + row) * kEmbed + c0, xn);
        if (lk == 0) L.sd[l * M + row] = sd;
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
    {  // final LN; x_f also stays in xs for dW_head
        RowVec<NV> x, xn;
        float sd;
        sk_layernorm<TPR>(h, L.ln + NL * 2 * kEmbed, L.ln + NL * 2 * kEmbed + kEmbed, c0, x, xn, sd);
        rv_store(L.xn + (NL * M + row) * kEmbed + c0, xn);
        if (lk == 0) L.sd[NL * M + row] = sd;
        rv_store(L.xs + row * kLds + c0, x);
        // model/linear.metal:17-37: head[row][j] = x_f[row] . W_head[:, j]
        for (int j = 0; j < HD; ++j) {
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < CPT; ++c) acc += x[c] * L.wh[(c0 + c) * HD + j];
            acc = group_sum<TPR>(acc);
            if (lk == 0) L.head[row * HD + j] = acc;
        }
    }
    __syncthreads();

    loss_rows<TPR>(a, LossIo{L.head, L.dhead, L.dls, L.stat}, row, lk, an, oldLp, ret, act, r0, g0);
    __syncthreads();

    // model/linear.metal:71-93 on this tile: dW_head[k][j] = sum_r x_f[r][k] dhead[r][j]
    tile_outer<M, NT>(L.dhead, HD, HD, L.xs, tp + pv.float_group, 1, HD);
    if (pv.continuous && tid < kEmbed) {  // model/gaussian.metal:166-168, summed over the tile in row order
        float s = 0.0f;
        if (tid < (int)pv.act_dim)
            for (int r = 0; r < M; ++r) s += L.dls[r * pv.act_dim + tid];
        tp[pv.off_log_std + tid] = s;  // and 0 in the arena padding after log_std (A <= 63 < 128)
    }
    if (tid >= 64 && tid < 64 + 5) {  // the tile's LossStats sums, in row order
        const int qq = tid - 64;
        float s = 0.0f;
        for (int r = 0; r < M; ++r) s += L.stat[r * 5 + qq];
        tp[pv.float_group + kEmbed * HD + qq] = s;
    }

    // ---- backward (model/ppo.h:793-865) ----
    RowVec<NV> D;
    {  // model/linear.metal:40-60: the gradient at the final LN output, then its LN
        RowVec<NV> g = rv_zero<NV>();
        for (int j = 0; j < HD; ++j) {
            const float dz = L.dhead[row * HD + j];
#pragma unroll
            for (int c = 0; c < CPT; ++c) g[c] += dz * L.wh[(c0 + c) * HD + j];
        }
        D = sk_layernorm_bwd<W>(L, g, NL, row, c0);
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
    sk_ln_sums<W>(L, tp + pv.off_ln_gamma[0], tp + pv.off_ln_beta[0]);
    tile_colsum2<M>(L.xs, nullptr, tp + pv.off_in_b, nullptr);
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
