// One PPO minibatch update (model/ppo.h:906-916) as four launches (three at
// the usual shapes, where 2 and 3 are one kernel):
//
//  1. train_rows: per 16-row tile (256 workgroups for 4096 rows), the forward
//     recompute with activation capture (model/ppo.h:909), the loss and head
//     gradient (model/policy.metal:14-69 / model/gaussian.metal:76-135) and the
//     whole backward dX chain (model/ppo.h:793-865) on MFMA, writing the
//     activations and gradients the weight gradients need.
//     The same workgroup writes its tile's sums of the vector-parameter, head
//     and log_std gradients and of the loss statistics.
//  2. train_dw: the block matrices' gradients X^T dY as MFMA tiles, the rows
//     split into ranges (fp32: 128x64 tiles from LDS-staged slabs; bf16: 64x64
//     tiles, operands loaded straight into registers from row-group-packed
//     captures).
//  3. grad_reduce: sums the tile partials and the row splits in fixed order,
//     writes the minibatch's LossStats (model/ppo.h:925-943) and one partial
//     squared norm per workgroup.
//     (With 128 to 1024 tiles of 32 x 32: train_dw_fused, or
//     train_dw_bf16_fused in bf16 mode, computes the weight gradients without
//     row splits and does this step's tile sums and partial norms in the same
//     launch.)
//  4. adam: every workgroup adds the partial norms in the same fixed order
//     (so no cross-workgroup synchronisation is needed), applies the clip
//     scale and Adam (model/optimizer.metal:23-60).
//
// Every reduction has a fixed order, so a rerun gives the same bits (the
// reference uses float atomics for several of these).
#include <string.h>

#include "kernels.h"
#include "mg/device/policy_bf16.h"
#include "mg/device/sample.h"

namespace mg {
namespace dev {

constexpr int kTR = kTileRows;  // rows per train_rows workgroup
constexpr int kTW = 8;          // waves per train_rows workgroup (two per SIMD)
constexpr int kTNT = 64 * kTW;  // threads per train_rows workgroup
constexpr int kMaxHeadT = 64;
constexpr int kMaxObsT = 64;
using TS = Shape<kTR, kTW>;
using TRegs = FwdRegs<kTR, kTW>;
using TSmem = FwdSmem<kTR, 2>;    // double-buffered hidden chunk
using TSmemB = FwdSmemB<kTR, 2>;  // the same with bf16 GEMM operands

// Per-tile outer-product sums in one pass: out[k * ks + c * cs] =
// sum_r a[r * lda + k] * b[r * kLds + c] for k < K and the 128 columns c, rows
// added in order. a and b are LDS tiles of M = 16 rows. No barrier (the
// caller orders the inputs before and the outputs after).
//  - K < 16: one thread per output. Thread t owns column t % 128 and the
//    k = t / 128 + (NT / 128) j: its column of b is read once into
//    registers, and a wave's reads of a are broadcasts of one address.
//  - K >= 16 (VoxelNav16's 30 x 128 embed gradient, 240 LDS reads per thread
//    one output at a time): 16 x 16 output tiles on v_mfma_f32_16x16x4_f32,
//    one per wave in turn, A = a^T (lane (q, m): a[4 s + q][16 kb + m], 0
//    past K), B = b, four row steps; the same sums in the same order (rows
//    in order, each added with an FMA). For K of 3 or 4 the MFMA tiles were
//    0.5 us slower than one thread per output.
template <int M, int NT>
__device__ __forceinline__ void tile_outer(const float* a, int lda, int K, const float* b, float* out, int ks,
                                           int cs) {
    static_assert(NT % kEmbed == 0, "whole columns per pass");
    static_assert(M == 16, "16-row tiles: four 16x16x4 row steps");
    if (K >= 16) {
        constexpr int NW = NT / 64;
        const int lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
        const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const int tiles = 8 * ((K + 15) / 16);
        for (int t = wave; t < tiles; t += NW) {
            const int kb = t >> 3, c = 16 * (t & 7) + n, k = 16 * kb + n;
            f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int r = 4 * s + q;
                const float av = k < K ? a[r * lda + k] : 0.0f;
                acc = mfma16x16x4(av, b[r * kLds + c], acc);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kk = 16 * kb + 4 * q + i;
                if (kk < K) out[kk * ks + c * cs] = acc[i];
            }
        }
        return;
    }
    const int c = threadIdx.x % kEmbed, k0 = threadIdx.x / kEmbed;
    if (k0 < K) {
        float bv[M];
#pragma unroll
        for (int r = 0; r < M; ++r) bv[r] = b[r * kLds + c];
        for (int k = k0; k < K; k += NT / kEmbed) {
            float s = 0.0f;
#pragma unroll
            for (int r = 0; r < M; ++r) s += a[r * lda + k] * bv[r];
            out[k * ks + c * cs] = s;
        }
    }
}

// Column sums of an LDS tile of M rows (sum_r b[r * kLds + c]) and, if a is
// given, of its products with another tile (sum_r a[r * kEmbed + c] b[...]),
// rows in order; threads t0 .. t0 + 127 one column each. No barrier.
template <int M>
__device__ __forceinline__ void tile_colsum2(const float* b, const float* a, float* out_sum, float* out_prod,
                                             int t0 = 0) {
    const int c = (int)threadIdx.x - t0;
    if (c >= 0 && c < kEmbed) {
        float s = 0.0f, p = 0.0f;
#pragma unroll
        for (int r = 0; r < M; ++r) {
            const float x = b[r * kLds + c];
            s += x;
            if (a) p += a[r * kEmbed + c] * x;
        }
        out_sum[c] = s;
        if (a) out_prod[c] = p;
    }
}

// The loss's transcendentals on the hardware units: e^x = 2^(x log2 e) and
// ln x = log2(x) ln 2 (v_exp_f32 / v_log_f32, about 1 ulp plus the rounding of
// the scaling). The loss and its gradient are compared with the oracle within
// tolerance, not bit for bit, so they do not need the bit-reproducible
// software versions the samplers use.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
__device__ __forceinline__ float fast_log(float x) { return __builtin_amdgcn_logf(x) * 0.693147180559945309f; }

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

// LDS arrays of the loss phase: head [16][HD] in; dhead [16][HD], the
// Gaussian head's per-row log_std gradients [16][A] and the rows' LossStats
// terms [16][5] out.
struct LossIo {
    const float* head;
    float* dhead;
    float* dls;
    float* stat;
};

// model/policy.metal:14-69 / model/gaussian.metal:76-135 for the tile's rows:
// TPR threads per row (lrow, lk), thread lk owning head columns lk + TPR u
// (u < 64 / TPR; ACT_DIM + 1 <= 64), the row sums as group reductions. an,
// oldLp, ret, act are the row's normalised advantage, old log-probability,
// return and action. Also writes the recomputed head to a.head_out. No barrier.
template <int TPR>
__device__ __forceinline__ void loss_rows(const RowsArgs& a, const LossIo& io, int lrow, int lk, float an,
                                          float oldLp, float ret, int act, uint32_t r0, size_t g0) {
    constexpr int NJ = 64 / TPR;  // head columns per thread
    const mg_policy_view& pv = a.pv;
    const int A = (int)pv.act_dim, HD = (int)pv.head_dim;
    const uint32_t B = a.step.rows;
    const float* h = io.head + lrow * HD;
    float* dz = io.dhead + lrow * HD;
    const float scale = 1.0f / (float)B;
    const float clip = a.hp.clip, ec = a.hp.entropy_coef;
    float entropy, logpA;
    float dd[NJ], is[NJ], pr[NJ], lp[NJ];
#pragma unroll
    for (int u = 0; u < NJ; ++u) dd[u] = is[u] = pr[u] = lp[u] = 0.0f;
    if (!pv.continuous) {  // model/policy.metal:14-69
        float z[NJ], zmax = -__builtin_huge_valf();
#pragma unroll
        for (int u = 0; u < NJ; ++u) {
            const int j = lk + TPR * u;
            z[u] = j < A ? h[j] : -__builtin_huge_valf();
            zmax = fmaxf(zmax, z[u]);
        }
        const float rowMax = group_max<TPR>(zmax);
        float e = 0.0f;
#pragma unroll
        for (int u = 0; u < NJ; ++u)
            if (lk + TPR * u < A) e += fast_exp(z[u] - rowMax);
        const float lse = rowMax + fast_log(group_sum<TPR>(e));
        float ent = 0.0f;
#pragma unroll
        for (int u = 0; u < NJ; ++u)
            if (lk + TPR * u < A) lp[u] = z[u] - lse, pr[u] = fast_exp(lp[u]), ent -= pr[u] * lp[u];
        entropy = group_sum<TPR>(ent);
        logpA = h[act] - lse;
    } else {  // model/gaussian.metal:76-135
        const float* actg = static_cast<const float*>(a.action_slots) + (g0 + lrow) * A;
        const float* logStd = pv.params + pv.off_log_std;
        float lpa = 0.0f, ent = 0.0f;
#pragma unroll
        for (int u = 0; u < NJ; ++u) {
            const int j = lk + TPR * u;
            if (j < A) {
                const float ls = logStd[j];
                is[u] = fast_exp(-ls);
                dd[u] = (actg[j] - h[j]) * is[u];
                lpa += -0.5f * dd[u] * dd[u] - ls - kLogSqrt2Pi;
                ent += ls + kLogSqrt2Pi + 0.5f;
            }
        }
        logpA = group_sum<TPR>(lpa);
        entropy = group_sum<TPR>(ent);
    }
    const float ratio = fast_exp(logpA - oldLp);
    const float surr1 = ratio * an;
    const float cr = fminf(fmaxf(ratio, 1.0f - clip), 1.0f + clip);
    const float surr2 = cr * an;
    const float gLogp = (surr1 <= surr2) ? -an * ratio : 0.0f;
#pragma unroll
    for (int u = 0; u < NJ; ++u) {
        const int j = lk + TPR * u;
        if (j < A) {
            if (!pv.continuous) {
                dz[j] = (gLogp * ((j == act ? 1.0f : 0.0f) - pr[u]) + ec * pr[u] * (lp[u] + entropy)) * scale;
            } else {
                dz[j] = gLogp * dd[u] * is[u] * scale;
                io.dls[lrow * A + j] = (gLogp * (dd[u] * dd[u] - 1.0f) - ec) * scale;
            }
        }
    }
    if (lk == 0) {
        const float vErr = h[A] - ret;
        dz[A] = a.hp.value_coef * vErr * scale;
        float* st = io.stat + lrow * 5;
        st[0] = -(surr1 < surr2 ? surr1 : surr2);
        st[1] = 0.5f * a.hp.value_coef * vErr * vErr;
        st[2] = entropy;
        st[3] = oldLp - logpA;
        st[4] = (fabsf(ratio - 1.0f) > clip) ? 1.0f : 0.0f;
    }
    if (a.head_out) {
#pragma unroll
        for (int u = 0; u < NJ; ++u) {
            const int j = lk + TPR * u;
            if (j < HD) a.head_out[(size_t)(r0 + lrow) * HD + j] = h[j];
        }
    }
}

// Gradient at the final LN output: dX = dZ W_head^T (model/linear.metal:40-60);
// Wh is W_head staged in LDS.
__device__ __forceinline__ void bwd_head(const float* Wh, const float* dheadL, int HD, TRegs& G) {
    for_each_elem<kTR, kTW>([&](int rt, int ct, int r, int row, int col) { G.h[rt][ct][r] = 0.0f; });
    for (int j = 0; j < HD; ++j) {
        for_each_elem<kTR, kTW>([&](int rt, int ct, int r, int row, int col) {
            G.h[rt][ct][r] += dheadL[row * HD + j] * Wh[col * HD + j];
        });
    }
}

// model/layernorm.metal:74-127 on a register tile: G holds the gradient at the
// LN output on entry and the gradient at the LN input on exit. xn/sd are the
// tile's forward captures (LDS). The tile's sums for dgamma (xn * dZ) and
// dbeta (dZ) go to tp_gamma / tp_beta (the reference adds them with float
// atomics).
template <class Smem>
__device__ __forceinline__ void bwd_layernorm(Smem& sm, TRegs& G, const float* xn, const float* sd,
                                              const float* gamma, float* tp_gamma, float* tp_beta, float* scratch) {
    constexpr int TPR = kTNT / kTR, CPT = kEmbed / TPR;
    const int tid = threadIdx.x;
    store_tile<kTR, kTW>(G.h, sm.xs);
    __syncthreads();
    tile_colsum2<kTR>(sm.xs, xn, tp_beta, tp_gamma);  // reads the tile before the in-place update below
    __syncthreads();
    const int row = tid / TPR, part = tid % TPR, c0 = part * CPT;
    static_assert(CPT == 4, "one float4 per thread");
    // float4 accesses: a thread's 4 columns are 16 contiguous bytes, so the
    // lanes of a wave touch distinct banks (scalar accesses at a 4-dword
    // lane stride would conflict 4 ways)
    f32x4* zr = reinterpret_cast<f32x4*>(sm.xs + row * kLds + c0);
    const f32x4 xv = *reinterpret_cast<const f32x4*>(xn + row * kEmbed + c0);
    const f32x4 gm = *reinterpret_cast<const f32x4*>(gamma + c0);
    const f32x4 z = *zr;
    float dxn[CPT];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        dxn[c] = z[c] * gm[c];
        s1 += dxn[c];
        s2 += dxn[c] * xv[c];
    }
    s1 = group_sum<TPR>(s1);
    s2 = group_sum<TPR>(s2);
    const float r1 = s1 / (float)kEmbed, r2 = s2 / (float)kEmbed, rd = 1.0f / sd[row];
    f32x4 o;
#pragma unroll
    for (int c = 0; c < CPT; ++c) o[c] = rd * (dxn[c] - r1 - xv[c] * r2);
    *zr = o;
    __syncthreads();
    for_each_elem<kTR, kTW>(
        [&](int rt, int ct, int r, int row2, int col) { G.h[rt][ct][r] = sm.xs[row2 * kLds + col]; });
    __syncthreads();
}

// The backward's GEMM sequence, blocks in reverse: for block l and chunk c,
// GEMM 2 ((L - 1 - l) NC + c) is dV_c = dh Down[c, :]^T (weights Down rows c,
// [128 hidden][128]) and the next one is dx += dV_c Up[:, c]^T (weights Up
// columns c, [128][H]), both from the fragment-tiled copies of the matrices as
// stored (frag_bwd16): Down rows c (K = 128) start at tile row 128 c / 16, Up's
// chunk c (K = H) at tile column c.
struct BwdSeq {
    const mg_policy_view* pv;
    int nc;
    __device__ __forceinline__ FragSrc operator()(int s) const {
        const int l = (int)pv->layers - 1 - s / (2 * nc), c = (s >> 1) % nc;
        if ((s & 1) == 0) return {pv->frag_bwd16 + pv->off_down[l] + (size_t)kChunk * c * kEmbed, (uint32_t)kEmbed};
        return {pv->frag_bwd16 + pv->off_up[l] + 16 * kChunk * c, pv->hidden};
    }
};

// The row pass streams one sequence: the forward's 2 L NC GEMMs, then the
// backward's, so the last forward GEMMs already prefetch the backward's first
// weights.
struct TrainSeq {
    const mg_policy_view* pv;
    int nc;
    __device__ __forceinline__ FragSrc operator()(int s) const {
        const int F = 2 * (int)pv->layers * nc;
        return s < F ? FwdSeq<16>{pv, nc}(s) : BwdSeq{pv, nc}(s - F);
    }
};

// The bf16 copies' sequences (see BwdSeq, TrainSeq): the same offsets in
// frag_fwd16_bf and frag_bwd16_bf.
struct BwdSeqB {
    const mg_policy_view* pv;
    int nc;
    __device__ __forceinline__ FragSrcB operator()(int s) const {
        const int l = (int)pv->layers - 1 - s / (2 * nc), c = (s >> 1) % nc;
        if ((s & 1) == 0) return {pv->frag_bwd16_bf + pv->off_down[l] + (size_t)kChunk * c * kEmbed, (uint32_t)kEmbed};
        return {pv->frag_bwd16_bf + pv->off_up[l] + 16 * kChunk * c, pv->hidden};
    }
};
struct TrainSeqB {
    const mg_policy_view* pv;
    int nc;
    __device__ __forceinline__ FragSrcB operator()(int s) const {
        const int F = 2 * (int)pv->layers * nc;
        return s < F ? FwdSeqB<16>{pv, nc}(s) : BwdSeqB{pv, nc}(s - F);
    }
};

// The row pass's types per precision: LDS tile, weight stream, GEMM sequence.
// The captures for the weight gradients (Cap): fp32 row-major, or bf16
// row-group-packed (copy_tile_p8) as the bf16 weight-gradient GEMMs read them.
template <bool BF>
struct RowsTypes {
    using Smem = TSmem;
    using Stream = TStream<kTR, kTW>;
    using Seq = TrainSeq;
    using Cap = float;
};
template <>
struct RowsTypes<true> {
    using Smem = TSmemB;
    using Stream = TStreamB<kTR, kTW>;
    using Seq = TrainSeqB;
    using Cap = uint16_t;
};

// Backward of block l (model/mlp.metal:88-153 + model/ppo.h:851-852). D holds
// the gradient at the block output (dStream) and is updated in place to the
// gradient at the block input. Chunked like the forward: dV_c = (dh Down_c^T)
// masked by relu, then dx += dV_c Up_c^T; ws streams the row pass's TrainSeq.
// With BF the two GEMMs take bf16 operands (dh and dV rounded as they are
// written to LDS; the captures for the weight gradients are the rounded
// values). v_tile, dv_store and dh_store point at the tile's first row.
template <bool BF, class Stream, class Smem, class Cap = typename RowsTypes<BF>::Cap>
__device__ __forceinline__ void bwd_block(const mg_policy_view& pv, int l, Smem& sm, TRegs& D,
                                          Stream& ws, const Cap* v_tile, Cap* dv_store, Cap* dh_store,
                                          const float* xn_tile, const float* sd_tile, const float* gamma,
                                          float* tp, float* scratch) {
    const int H = (int)pv.hidden, NC = H / kChunk, F = 2 * (int)pv.layers * NC;
    const typename RowsTypes<BF>::Seq seq{&pv, NC};
    // The relu mask of chunk c: the lane's four elements of the hidden capture
    // (rows 4 (lane / 16) .. + 3 of one column). bf16: one 8-byte load from the
    // row-group-packed capture, a value is positive iff its bits are non-zero
    // (relu outputs are +0 or positive).
    static_assert(TS::RT == 1 && TS::CT == 1 && TS::MT == 16, "one 16x16 tile per wave");
    using Mask = typename std::conditional<BF, uint2, typename TS::Acc>::type;
    auto load_mask = [&](int c) {
        Mask m;
        if constexpr (BF) {
            const int lane = threadIdx.x & 63, q = lane >> 4, col = 16 * (threadIdx.x >> 6) + (lane & 15);
            m = *reinterpret_cast<const uint2*>(v_tile + ((size_t)(q >> 1) * H + kChunk * c + col) * 8 + 4 * (q & 1));
        } else {
            for_each_elem<kTR, kTW>(
                [&](int rt, int ct, int r, int row, int col) { m[r] = v_tile[(size_t)row * H + kChunk * c + col]; });
        }
        return m;
    };
    auto positive = [](const Mask& m, int r) {
        if constexpr (BF)
            return (((r < 2 ? m.x : m.y) >> (16 * (r & 1))) & 0xFFFFu) != 0;
        else
            return m[r] > 0.0f;
    };
    if constexpr (BF) {
        store_tile_relu_b<kTR, kTW, false>(D.h, sm.xb);
        __syncthreads();
        copy_tile_p8<kTNT>(sm.xb, dh_store, kEmbed, 0);
    } else {
        store_tile_g<kTR, kTW>(D.h, dh_store, kEmbed);
        store_tile<kTR, kTW>(D.h, sm.xs);
        __syncthreads();
    }
    TRegs G;
    zero<kTR, kTW>(G.h);
    for (int c = 0; c < NC; ++c) {
        const int s = F + 2 * (((int)pv.layers - 1 - l) * NC + c);
        // loaded before the GEMM issues its weight refills (vector memory
        // counters complete in order)
        const Mask mask = load_mask(c);
        TS::Acc v[TS::RT][TS::CT];
        zero<kTR, kTW>(v);
        if constexpr (BF) {
            uint16_t* vb = sm.vb[c & 1];  // double-buffered: no barrier before the write
            ws.template gemm<0>(v, sm.xb, s, seq);
            for_each_elem<kTR, kTW>([&](int rt, int ct, int r, int row, int col) {
                vb[row * kLdsB + col] = bf16_rne(positive(mask, r) ? v[rt][ct][r] : 0.0f);
            });
            __syncthreads();
            copy_tile_p8<kTNT>(vb, dv_store, H, kChunk * c);
            ws.template gemm<1>(G.h, vb, s + 1, seq);
        } else {
            float* vs = sm.vs[c & 1];  // double-buffered: no barrier before the write
            ws.template gemm<0>(v, sm.xs, s, seq);
            for_each_elem<kTR, kTW>([&](int rt, int ct, int r, int row, int col) {
                const float g = positive(mask, r) ? v[rt][ct][r] : 0.0f;
                dv_store[(size_t)row * H + kChunk * c + col] = g;
                vs[row * kLds + col] = g;
            });
            __syncthreads();
            ws.template gemm<1>(G.h, vs, s + 1, seq);
        }
    }
    __syncthreads();
    bwd_layernorm(sm, G, xn_tile, sd_tile, gamma, tp + pv.off_ln_gamma[l], tp + pv.off_ln_beta[l], scratch);
#pragma unroll
    for (int rt = 0; rt < TS::RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < TS::CT; ++ct) D.h[rt][ct] = G.h[rt][ct] + D.h[rt][ct];  // residualAdd(dBranch, dStream)
}

// LDS of one train_rows workgroup, sized for every supported shape. The LN
// captures xn / sd are only read by the LN backward, so they never leave the CU.
template <bool BF>
struct RowsSmem {
    typename RowsTypes<BF>::Smem sm;
    float xn[(MG_MAX_LAYERS + 1) * kTR * kEmbed];
    float sd[(MG_MAX_LAYERS + 1) * kTR];
    float ln[(MG_MAX_LAYERS + 1) * 2 * kEmbed];  // gamma, beta of every LN
    float wh[kEmbed * kMaxHeadT];                // W_head
    float obs[kTR * kMaxObsT];
    float head[kTR * kMaxHeadT];
    float dhead[kTR * kMaxHeadT];
    float dls[kTR * kMaxHeadT];
    float stat[kTR * 5];
    float scratch[kTNT];
};

// BF: the block GEMMs take bf16 operands (MG_PRECISION_BF16).
template <bool BF>
__global__ void __launch_bounds__(kTNT) train_rows_kernel(const RowsArgs a) {
    constexpr int M = kTR;
    using Stream = typename RowsTypes<BF>::Stream;
    __shared__ RowsSmem<BF> L;
    auto& sm = L.sm;
    TRegs R;
    const mg_policy_view& pv = a.pv;
    const TrainWs& ws = a.ws;
    const int O = (int)pv.obs_dim, A = (int)pv.act_dim, HD = (int)pv.head_dim, H = (int)pv.hidden;
    const int NL = (int)pv.layers;
    const uint32_t B = a.step.rows;
    const uint32_t r0 = blockIdx.x * M;           // row within the minibatch
    const size_t g0 = (size_t)a.step.row0 + r0;   // row within the slot arrays
    const int tid = threadIdx.x;
    float* tp = ws.tp + (size_t)blockIdx.x * ws.tp_count;  // this tile's vector-parameter partials

    // Everything small is loaded first, so waiting for it does not wait for the
    // weight stream issued after it (vector memory counters complete in order).
    // W_in and b_in for the embed go to the LN capture area (first written by
    // the first LN, after every wave is done with the embed); the LN
    // parameters (gamma, beta of every LN) are one contiguous run. The first
    // element per thread of each array (and two of the LN run: all of it up to
    // 3 LNs) is loaded before any is stored, so their memory latencies overlap;
    // larger shapes finish in loops.
    float* winL = L.xn;
    float* binL = L.xn + kMaxObsT * kEmbed;
    static_assert((kMaxObsT + 1) * kEmbed <= (MG_MAX_LAYERS + 1) * kTR * kEmbed, "embed staging fits");
    const float* lnp = pv.params + pv.off_ln_gamma[0];
    const int n_obs = M * O, n_wh = kEmbed * HD, n_win = O * kEmbed, n_ln = (NL + 1) * 2 * kEmbed;
    // the loss inputs of this thread's row (32 threads per row)
    const int lrow = tid >> 5, lk = tid & 31;
    float an, oldLp, ret;
    int act = 0;
    Stream wst;
    const typename RowsTypes<BF>::Seq seq{&pv, H / kChunk};
    {
        // branch-free: a thread past an array's end loads an element in range
        // and drops it (loads behind a range branch made the compiler wait for
        // every outstanding load at the branch's join)
        const float o0 = a.obs_slots[g0 * O + (tid < n_obs ? tid : n_obs - 1)];
        const float h0 = pv.params[pv.off_head + (tid < n_wh ? tid : 0)];
        const float w0 = pv.params[pv.off_in_w + (tid < n_win ? tid : 0)];
        const float b0 = pv.params[pv.off_in_b + (tid < kEmbed ? tid : 0)];
        const float l0 = lnp[tid < n_ln ? tid : 0];
        const float l1 = lnp[tid + kTNT < n_ln ? tid + kTNT : 0];
        {
            const size_t gr = g0 + lrow;
            const float mean = a.adv_stats[2 * a.step.block], inv = a.adv_stats[2 * a.step.block + 1];
            an = (a.adv_slots[gr] - mean) * inv;
            oldLp = a.logp_slots[gr];
            ret = a.ret_slots[gr];
            if (!pv.continuous) act = static_cast<const int*>(a.action_slots)[gr];
        }
        // the weight stream next: its loads are in flight while the stores
        // below wait for the small loads ahead of them
        wst.start(4 * NL * (H / kChunk), seq);
        if (tid < n_obs) L.obs[tid] = o0;
        if (tid < n_wh) L.wh[tid] = h0;
        if (tid < n_win) winL[tid] = w0;
        if (tid < kEmbed) binL[tid] = b0;
        if (tid < n_ln) L.ln[tid] = l0;
        if (tid + kTNT < n_ln) L.ln[tid + kTNT] = l1;
    }
#pragma unroll 4
    for (int idx = tid + kTNT; idx < n_obs; idx += kTNT) L.obs[idx] = a.obs_slots[g0 * O + idx];
#pragma unroll 4
    for (int idx = tid + kTNT; idx < n_wh; idx += kTNT) L.wh[idx] = pv.params[pv.off_head + idx];
#pragma unroll 4
    for (int idx = tid + kTNT; idx < n_win; idx += kTNT) winL[idx] = pv.params[pv.off_in_w + idx];
#pragma unroll 4
    for (int idx = tid + 2 * kTNT; idx < n_ln; idx += kTNT) L.ln[idx] = lnp[idx];
    __syncthreads();

    // ---- forward with capture ----
    fwd_embed<M, kTW>(winL, binL, L.obs, O, R);
    // the captures of layer l for rows r0 .. r0 + 15: [B][C] per layer; in the
    // bf16 layout these rows start at row group r0 / 8, element r0 C, too
    using Cap = typename RowsTypes<BF>::Cap;
    Cap* const cx = reinterpret_cast<Cap*>(ws.x);
    Cap* const cv = reinterpret_cast<Cap*>(ws.v);
    Cap* const cdh = reinterpret_cast<Cap*>(ws.dhb);
    Cap* const cdv = reinterpret_cast<Cap*>(ws.dvb);
    for (int l = 0; l < NL; ++l) {
        const float* gamma = L.ln + l * 2 * kEmbed;
        if constexpr (BF) {
            fwd_layernorm<M, kTW>(sm, R, gamma, gamma + kEmbed, L.xn + l * M * kEmbed, L.sd + l * M, nullptr, sm.xb);
            copy_tile_p8<kTNT>(sm.xb, cx + ((size_t)l * B + r0) * kEmbed, kEmbed, 0);
            fwd_block_b<M, kTW, true, 2>(pv, l, sm, R, wst, cv + ((size_t)l * B + r0) * H, seq);
        } else {
            fwd_layernorm<M, kTW>(sm, R, gamma, gamma + kEmbed, L.xn + l * M * kEmbed, L.sd + l * M,
                                  cx + ((size_t)l * B + r0) * kEmbed);
            fwd_block<M, kTW, true, 2>(pv, l, sm, R, wst, cv + ((size_t)l * B + r0) * H, seq);
        }
    }
    // the backward's first weights are in flight through the final LN, the head and the loss
    fwd_layernorm<M, kTW>(sm, R, L.ln + NL * 2 * kEmbed, L.ln + NL * 2 * kEmbed + kEmbed, L.xn + NL * M * kEmbed,
                          L.sd + NL * M);
    fwd_head<M, kTW>(L.wh, sm, L.head, HD);

    // ---- loss and head gradient: 32 threads per row, thread k owning head
    // columns k and k + 32 (ACT_DIM <= 63), the row sums as group reductions ----
    static_assert(kTNT == 32 * M && kMaxHeadT <= 64, "32 threads per row, two columns each");
    loss_rows<32>(a, LossIo{L.head, L.dhead, L.dls, L.stat}, lrow, lk, an, oldLp, ret, act, r0, g0);
    __syncthreads();

    // model/linear.metal:71-93 on this tile: dW_head[k][j] = sum_r x_f[r][k] dhead[r][j]
    // (sm.xs still holds the final LN output x_f)
    tile_outer<M, kTNT>(L.dhead, HD, HD, sm.xs, tp + pv.float_group, 1, HD);
    if (pv.continuous && tid < kEmbed) {  // model/gaussian.metal:166-168, summed over the tile in row order
        float s = 0.0f;
        if (tid < A)
            for (int r = 0; r < M; ++r) s += L.dls[r * A + tid];
        tp[pv.off_log_std + tid] = s;  // and 0 in the arena padding after log_std (A <= 63 < 128)
    }
    if (tid >= 64 && tid < 64 + 5) {  // the tile's LossStats sums, in row order
        const int q = tid - 64;
        float s = 0.0f;
        for (int r = 0; r < M; ++r) s += L.stat[r * 5 + q];
        tp[pv.float_group + kEmbed * HD + q] = s;
    }
    __syncthreads();  // every read of x_f in sm.xs is done before the LN backward overwrites it

    // ---- backward ----
    TRegs D;
    bwd_head(L.wh, L.dhead, HD, D);
    bwd_layernorm(sm, D, L.xn + NL * M * kEmbed, L.sd + NL * M, L.ln + NL * 2 * kEmbed, tp + pv.off_ln_gamma[NL],
                  tp + pv.off_ln_beta[NL], L.scratch);
    for (int l = NL - 1; l >= 0; --l) {
        bwd_block<BF>(pv, l, sm, D, wst, cv + ((size_t)l * B + r0) * H, cdv + ((size_t)l * B + r0) * H,
                      cdh + ((size_t)l * B + r0) * kEmbed, L.xn + l * M * kEmbed, L.sd + l * M,
                      L.ln + l * 2 * kEmbed, tp, L.scratch);
    }
    // model/input.metal:38-60 on this tile: dW_in[k][c] = sum_r obs[r][k] dh0[r][c], db_in = sum_r dh0
    store_tile<M, kTW>(D.h, sm.xs);
    __syncthreads();
    tile_colsum2<M>(sm.xs, nullptr, tp + pv.off_in_b, nullptr);
    tile_outer<M, kTNT>(L.obs, O, O, sm.xs, tp + pv.off_in_w, kEmbed, 1);
}

}  // namespace dev
}  // namespace mg

#include "rows_split.h"

namespace mg {
namespace dev {

// ---- weight gradients ---------------------------------------------------------

// A big tile job: C[m][n] = sum_r X[r][m] Y[r][n] for a 128 x H (or H x 128)
// matrix; X and Y are the captures (T = float: row-major; T = uint16_t: bf16,
// row-group-packed), ldx / ldy their column counts.
template <class T>
struct BigMatT {
    const T* x;
    const T* y;
    uint32_t ldx, ldy;
    uint32_t mdim, ndim;
    uint32_t off;
    uint32_t pad;
};
constexpr int kMaxBig = 2 * MG_MAX_LAYERS;

template <class T>
struct DwArgsT {
    BigMatT<T> big[kMaxBig];
    uint32_t nbig;
    uint32_t tiles_per_big[kMaxBig];
    uint32_t big_tiles;    // total 64x64 tiles over all big matrices
    uint32_t rows;         // B
    uint32_t splits;       // row splits
    uint32_t count;        // arena length
    float* partial;
};

// The full gradient from its two sources, summed in fixed order, plus one
// partial squared norm per workgroup:
//  - workgroups [0, small_wgs): 16 tile-partial columns each (vector
//    parameters, the head, then the 5 LossStats sums); 16 thread groups per
//    column each add a range of tiles, and the ranges are added in order;
//  - the rest: the block matrices, the sum of the row splits (grid-stride).
constexpr int kRedCols = 16;  // tile-partial columns per small workgroup
struct ReduceArgs {
    const float* partial;
    const float* tp;
    float* grad;
    float* normpart;
    float* mb_stats;
    uint32_t splits, tiles, tp_count, count;
    uint32_t float_group, off_head, head_count, small_wgs;
    float inv_rows;
};

// Workgroup wg of nwg summing tile-partial columns (kRedCols at a time): NT /
// kRedCols thread groups per column each add a range of tiles, and the ranges
// are added in order. Writes the vector / head gradient and the minibatch
// LossStats; returns this thread's sum of the squared gradient values it
// wrote. NT threads.
template <int NT>
__device__ __forceinline__ float reduce_tile_partials(const ReduceArgs& a, uint32_t wg, uint32_t nwg) {
    constexpr int NG = NT / kRedCols;  // thread groups per column
    __shared__ float part[NG][kRedCols];
    const int t = threadIdx.x;
    float sq = 0.0f;
    const uint32_t grp = t / kRedCols;
    const uint32_t lo = grp * a.tiles / NG, hi = (grp + 1) * a.tiles / NG;
    const uint32_t stat0 = a.float_group + a.head_count;
    for (uint32_t c0 = wg * kRedCols; c0 < stat0 + 5; c0 += nwg * kRedCols) {
        const uint32_t col = c0 + t % kRedCols;
        float s = 0.0f;
        if (col < stat0 + 5) {
            const float* src = a.tp + col;
            // loads issued eight at a time, added in tile order
            for (uint32_t k0 = lo; k0 < hi; k0 += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) x[u] = k0 + u < hi ? src[(size_t)(k0 + u) * a.tp_count] : 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) s += x[u];
            }
        }
        part[grp][t % kRedCols] = s;
        __syncthreads();
        if (t < kRedCols && col < stat0 + 5) {
            float g = 0.0f;
#pragma unroll
            for (int q = 0; q < NG; ++q) g += part[q][t];
            if (col < a.float_group) {
                a.grad[col] = g;
                sq += g * g;
            } else if (col < stat0) {
                a.grad[a.off_head + (col - a.float_group)] = g;
                sq += g * g;
            } else {
                a.mb_stats[col - stat0] = g * a.inv_rows;  // model/ppo.h:925-943 means
            }
        }
        __syncthreads();
    }
    return sq;
}

// The workgroup's sum of sq to *out, in a fixed order (a DPP tree within each
// wave, then the NW waves in order).
template <int NW>
__device__ __forceinline__ void write_norm_part(float sq, float* out) {
    __shared__ float red[NW];
    sq = group_sum<64>(sq);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = red[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += red[w];
        *out = s;
    }
}

constexpr int kDwRows = 64;             // rows staged in LDS per step
constexpr int kDwTileM = 128;           // output tile: 128 x 64
constexpr int kDwTileN = 64;
constexpr int kDwLdX = kDwTileM + 4;    // LDS row strides of the staged slabs
constexpr int kDwLdY = kDwTileN + 4;
constexpr int kDwWaves = 8;             // two per SIMD

// One 128 x 64 tile of a block matrix's gradient C = X^T Y over one row split:
// 8 waves, wave w owning the 32 x 32 sub-tile at (32 (w / 2), 32 (w % 2)) as
// one accumulator (v_mfma_f32_32x32x2_f32: A = X[k][m], B = Y[k][n] straight
// from the staged slab, k = the rows). 64-row slabs of X (32 KB) and Y (16 KB)
// are double-buffered in LDS, and each slab's loads are issued two slabs
// before it is written there (two register sets), so one workgroup per CU
// keeps two slabs of loads in flight; one barrier per slab. The next slab's
// LDS writes and the loads after them are issued between the current slab's
// MFMAs (written after them, the last wave of a SIMD ran them alone before the
// barrier: 23.6 -> 22.1 us at 4096 rows, hidden 512). Workgroup id =
// tile * splits + split: workgroups go to the 8 XCDs round robin, so with 8
// or 16 splits all tiles of one row split run on the same XCD and share its
// rows through that XCD's L2.
__global__ void __launch_bounds__(64 * kDwWaves) train_dw_kernel(const DwArgsT<float> a) {
    __shared__ float xs[2][kDwRows * kDwLdX];
    __shared__ float ys[2][kDwRows * kDwLdY];
    const uint32_t split = blockIdx.x % a.splits, tile = blockIdx.x / a.splits;
    const uint32_t rowsPer = a.rows / a.splits;
    const uint32_t rb = split * rowsPer;
    float* out = a.partial + (size_t)split * a.count;
    const int tid = threadIdx.x;
    uint32_t t = tile, m = 0;  // the grid is big_tiles * splits: every workgroup has a tile
    while (t >= a.tiles_per_big[m]) t -= a.tiles_per_big[m], ++m;
    const BigMatT<float>& bm = a.big[m];
    const uint32_t ntn = bm.ndim / kDwTileN;
    const uint32_t tm = t / ntn, tn = t % ntn;
    const int w = tid >> 6, lane = tid & 63;
    const int wm = 32 * (w >> 1), wn = 32 * (w & 1);
    // staging: X rows t / 32 + 16 i (i < 4) at column 4 (t % 32); Y rows
    // t / 16 + 32 i (i < 2) at column 4 (t % 16)
    const int xr = tid >> 5, xc = 4 * (tid & 31), yr = tid >> 4, yc = 4 * (tid & 15);
    // slab indices past the split's last slab reload the last one, so every
    // step issues the same loads
    f32x4 px[2][4], py[2][2];
    const uint32_t steps = rowsPer / kDwRows;
    // staging item it < 4: X rows xr + 16 it; it >= 4: Y rows yr + 32 (it - 4),
    // of the slab's 64 rows; buffer loads from the matrices' bases with this
    // thread's byte offset in a VGPR and the row offset in an SGPR.
    // With 8 splits, split s takes the rows of the row pass's 16-row tiles
    // s, s + 8, s + 16, ...: the row-pass workgroups that wrote them ran on the
    // same XCD as this split (workgroups go to the XCDs round robin), so part of
    // the slabs still sit in that XCD's L2 (22.2 -> 21.9 us at 4096 rows);
    // otherwise a split's rows are contiguous. Slab row q is then row
    // 16 s + q % 16 + 128 (q / 16) of the minibatch.
    const bool xcd = a.splits == 8;
    const uint32_t xrow = xcd ? 16 * split + xr : rb + xr;
    const uint32_t yrow = xcd ? 16 * split + (yr & 15) + 128 * (yr >> 4) : rb + yr;
    const uint32_t rstep = xcd ? 8 : 1;  // minibatch rows per slab row, in 16-row groups
    const uint32_t xv = 4 * (xrow * bm.ldx + tm * kDwTileM + xc);
    const uint32_t yv = 4 * (yrow * bm.ldy + tn * kDwTileN + yc);
    auto load_item = [&](int set, int it, uint32_t sl) {
        const uint32_t r0 = (sl < steps ? sl : steps - 1) * kDwRows;
        if (it < 4)
            px[set][it] = buffer_load16(bm.x, xv, 4 * rstep * (r0 + 16 * it) * bm.ldx);
        else
            py[set][it - 4] = buffer_load16(bm.y, yv, 4 * rstep * (r0 + 32 * (it - 4)) * bm.ldy);
    };
    auto put_item = [&](int set, int buf, int it) {
        if (it < 4)
            *reinterpret_cast<f32x4*>(&xs[buf][(xr + 16 * it) * kDwLdX + xc]) = px[set][it];
        else
            *reinterpret_cast<f32x4*>(&ys[buf][(yr + 32 * (it - 4)) * kDwLdY + yc]) = py[set][it - 4];
    };
    f32x16 acc = f32x16{};
    // lane (i = l % 32, k = l / 32) supplies X[k][wm + i] and Y[k][wn + i]
    const int ox = (lane >> 5) * kDwLdX + wm + (lane & 31), oy = (lane >> 5) * kDwLdY + wn + (lane & 31);
    // The MFMAs of the slab in LDS buffer buf, with the next slab's staging
    // interleaved: after MFMA 4 it + 3, register set s's item it goes to
    // buffer buf ^ 1 (last read before the previous barrier) and is reloaded
    // with slab nx's item, so the staging runs in the MFMAs' shadow.
    auto slab = [&](int buf, int s, uint32_t nx) {
        const float* xp = xs[buf] + ox;
        const float* yp = ys[buf] + oy;
#pragma unroll
        for (int kk = 0; kk < kDwRows / 2; ++kk) {
            acc = mfma32x32x2(xp[2 * kk * kDwLdX], yp[2 * kk * kDwLdY], acc);
            if (kk % 4 == 3 && kk / 4 < 6) {
                put_item(s, buf ^ 1, kk / 4);
                load_item(s, kk / 4, nx);
            }
        }
    };
    // slab 0 in LDS buffer 0, slab 1 in set 1, slab 2 in set 0
#pragma unroll
    for (int it = 0; it < 6; ++it) load_item(0, it, 0);
#pragma unroll
    for (int it = 0; it < 6; ++it) load_item(1, it, 1);
#pragma unroll
    for (int it = 0; it < 6; ++it) put_item(0, 0, it);
#pragma unroll
    for (int it = 0; it < 6; ++it) load_item(0, it, 2);
    __syncthreads();
    for (uint32_t sl = 0; sl + 1 < steps; sl += 2) {
        slab(0, 1, sl + 3);  // slab sl; stages slab sl + 1, loads slab sl + 3
        __syncthreads();
        slab(1, 0, sl + 4);  // slab sl + 1; stages slab sl + 2, loads slab sl + 4
        __syncthreads();
    }
    if (steps & 1) slab(0, 1, steps);  // the last slab (its staging is not read)
    float* o = out + bm.off + (size_t)(tm * kDwTileM + wm) * bm.ndim + tn * kDwTileN + wn + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) o[(size_t)c32_row(r, lane) * bm.ndim] = acc[r];
}

// The weight gradients with bf16 operands (MG_PRECISION_BF16). X and Y are
// row-group-packed (element (r, c) at ((r / 8) C + c) 8 + r % 8), so the
// operand of lane l of a v_mfma_f32_32x32x16_bf16 contracting over rows (rows
// 8 (l / 32) .. + 7 of column l % 32) is 16 contiguous bytes, and a half-wave
// reads 512 contiguous bytes: operands go from memory straight into
// registers, no LDS staging. A workgroup computes one 64 x 64 tile over its
// row split (workgroup id = tile * splits + split, as in train_dw_kernel);
// each of its NW waves takes every NW-th 16-row step, with the whole tile as
// 2 x 2 MFMAs per step, and the NW partial tiles are added in LDS in wave
// order. U steps are loaded while the previous U run their MFMAs. (Measured at
// 4096 rows, 2 blocks, hidden 512: 4 or 8 waves, U = 2 or 4 and 4 or 8 row
// splits all ran within 3% of each other, about 10 us.)
constexpr int kDwbWaves = 4;
template <int NW, int U>
__global__ void __launch_bounds__(64 * NW) train_dw_bf16_kernel(const DwArgsT<uint16_t> a) {
    __shared__ float red[NW][64 * 64];
    const uint32_t split = blockIdx.x % a.splits, tile = blockIdx.x / a.splits;
    const uint32_t rowsPer = a.rows / a.splits;  // a multiple of 16 NW
    const uint32_t rb = split * rowsPer;
    uint32_t t = tile, m = 0;
    while (t >= a.tiles_per_big[m]) t -= a.tiles_per_big[m], ++m;
    const BigMatT<uint16_t>& bm = a.big[m];
    const uint32_t ntn = bm.ndim / 64;
    const uint32_t tm = t / ntn, tn = t % ntn;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // lane's operands in step s: row group rb / 8 + 2 (NW s + w) + lane / 32,
    // columns tile + lane % 32 and tile + 32 + lane % 32
    const size_t g0 = rb / 8 + 2 * w + (lane >> 5);
    const uint16_t* xp = bm.x + (g0 * bm.ldx + tm * 64 + (lane & 31)) * 8;
    const uint16_t* yp = bm.y + (g0 * bm.ldy + tn * 64 + (lane & 31)) * 8;
    const size_t xstep = (size_t)16 * NW * bm.ldx, ystep = (size_t)16 * NW * bm.ldy;  // 2 NW row groups
    const uint32_t steps = rowsPer / (16 * NW);
    const uint32_t batches = (steps + U - 1) / U;
    // steps past the split's end load zeros (they add nothing)
    auto load = [&](u32x4 (&op)[U][4], uint32_t b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t st = b * U + u;
            if (st < steps) {
                const uint16_t* x = xp + st * xstep;
                const uint16_t* y = yp + st * ystep;
                op[u][0] = *reinterpret_cast<const u32x4*>(x);
                op[u][1] = *reinterpret_cast<const u32x4*>(x + 256);
                op[u][2] = *reinterpret_cast<const u32x4*>(y);
                op[u][3] = *reinterpret_cast<const u32x4*>(y + 256);
            } else {
                op[u][0] = op[u][1] = op[u][2] = op[u][3] = u32x4{0, 0, 0, 0};
            }
        }
    };
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    u32x4 cur[U][4], nxt[U][4];
    load(cur, 0);
    for (uint32_t b = 0; b < batches; ++b) {
        if (b + 1 < batches) load(nxt, b + 1);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = ShapeB<32>::mfma(cur[u][i], cur[u][2 + j], acc[i][j]);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k) cur[u][k] = nxt[u][k];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                red[w][(32 * i + c32_row(r, lane)) * 64 + 32 * j + (lane & 31)] = acc[i][j][r];
    __syncthreads();
    float* out = a.partial + (size_t)split * a.count + bm.off + (size_t)tm * 64 * bm.ndim + tn * 64;
    for (int e = threadIdx.x; e < 64 * 64; e += 64 * NW) {
        float v = red[0][e];
#pragma unroll
        for (int q = 1; q < NW; ++q) v += red[q][e];
        out[(size_t)(e >> 6) * bm.ndim + (e & 63)] = v;
    }
}

__global__ void __launch_bounds__(256) grad_reduce_kernel(const ReduceArgs a) {
    const int t = threadIdx.x;
    float sq = 0.0f;
    if (blockIdx.x < a.small_wgs) {
        sq = reduce_tile_partials<256>(a, blockIdx.x, a.small_wgs);
    } else {
        const uint32_t nw = gridDim.x - a.small_wgs;
        for (uint32_t i = a.float_group + (blockIdx.x - a.small_wgs) * 256 + t; i < a.off_head; i += nw * 256) {
            float x[kSplits];
#pragma unroll
            for (int s = 0; s < kSplits; ++s) x[s] = s < (int)a.splits ? a.partial[(size_t)s * a.count + i] : 0.0f;
            float g = 0.0f;
#pragma unroll
            for (int s = 0; s < kSplits; ++s) g += x[s];
            a.grad[i] = g;
            sq += g * g;
        }
    }
    write_norm_part<4>(sq, a.normpart + blockIdx.x);
}

// bf16 weight gradients, tile partial sums and partial norms in one launch
// (replacing train_dw + grad_reduce when the block matrices have enough 32 x
// 32 tiles to fill the GPU without row splits). Each of the first T
// workgroups computes one tile of the block matrices over all rows, operands
// as in train_dw_bf16_kernel: its NW waves take every NW-th 16-row step and
// add their tiles in LDS in wave order, and the tile goes straight to grad.
// Each wave keeps up to 2 U steps of loads in flight. The workgroups past T
// (or, in a grid of T, the tile workgroups afterwards) share the tile-partial
// columns (reduce_tile_partials). Every
// workgroup writes the squared norm of what it wrote to normpart; the entries
// past the grid are zeroed, so the Adam kernel's fixed-order sum over
// kReduceBlocks entries is the same sum. (At 4096 rows, 2 blocks, hidden 512:
// 16 waves with U = 4 or 2 and 8 waves with U = 4 ran within 3% of each other.
// Against the split kernel plus grad_reduce it saves one launch per
// minibatch.)
template <class T>
struct DwFusedArgs {
    DwArgsT<T> dw;
    ReduceArgs red;
};
template <int NW, int U>
__global__ void __launch_bounds__(64 * NW) train_dw_bf16_fused_kernel(const DwFusedArgs<uint16_t> a) {
    __shared__ float red[NW][32 * 32];
    float sq = 0.0f;
    const uint32_t T = a.dw.big_tiles;  // workgroups [0, T): one 32 x 32 tile each
    if (blockIdx.x >= T) {
        // the tile-partial columns on workgroups of their own, as in train_dw_fused_kernel
        sq = reduce_tile_partials<64 * NW>(a.red, blockIdx.x - T, gridDim.x - T);
    } else {
        // workgroups go to the 8 XCDs round robin, so workgroup b takes tile
        // (b mod 8) T / 8 + b / 8 of the order (matrix, hidden block, embed
        // block): an XCD's tiles are every embed block of a run of hidden
        // blocks of one matrix (T = 256: 8 hidden blocks), so it fetches the
        // matrix's embed-side capture once and half its hidden-side one (at
        // 4096 rows, hidden 512, 2 blocks: 13.2 -> 12.3 us against the order
        // with the hidden block fastest, whose XCDs each fetched the embed-side
        // captures of all four matrices). T is a multiple of 8.
        uint32_t t = (blockIdx.x % 8) * (T / 8) + blockIdx.x / 8, m = 0;
        while (t >= a.dw.tiles_per_big[m]) t -= a.dw.tiles_per_big[m], ++m;
        const BigMatT<uint16_t>& bm = a.dw.big[m];
        const uint32_t ntm = bm.mdim / 32, ntn = bm.ndim / 32;
        const uint32_t tm = bm.mdim > bm.ndim ? t / ntn : t % ntm;
        const uint32_t tn = bm.mdim > bm.ndim ? t % ntn : t / ntm;
        const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
        // lane's operands in step s: row group 2 (NW s + w) + lane / 32, column
        // tile + lane % 32
        const size_t g0 = 2 * w + (lane >> 5);
        const uint16_t* xp = bm.x + (g0 * bm.ldx + tm * 32 + (lane & 31)) * 8;
        const uint16_t* yp = bm.y + (g0 * bm.ldy + tn * 32 + (lane & 31)) * 8;
        const size_t xstep = (size_t)16 * NW * bm.ldx, ystep = (size_t)16 * NW * bm.ldy;  // 2 NW row groups
        const uint32_t steps = a.dw.rows / (16 * NW);  // rows: a multiple of 16 NW
        const uint32_t batches = (steps + U - 1) / U;
        auto load = [&](u32x4 (&op)[U][2], uint32_t b) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t st = b * U + u;
                if (st < steps) {
                    op[u][0] = *reinterpret_cast<const u32x4*>(xp + st * xstep);
                    op[u][1] = *reinterpret_cast<const u32x4*>(yp + st * ystep);
                } else {
                    op[u][0] = op[u][1] = u32x4{0, 0, 0, 0};
                }
            }
        };
        f32x16 acc = f32x16{};
        u32x4 cur[U][2], nxt[U][2];
        load(cur, 0);
        for (uint32_t b = 0; b < batches; ++b) {
            if (b + 1 < batches) load(nxt, b + 1);
#pragma unroll
            for (int u = 0; u < U; ++u) acc = ShapeB<32>::mfma(cur[u][0], cur[u][1], acc);
#pragma unroll
            for (int u = 0; u < U; ++u) cur[u][0] = nxt[u][0], cur[u][1] = nxt[u][1];
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) red[w][c32_row(r, lane) * 32 + (lane & 31)] = acc[r];
        __syncthreads();
        float* out = a.red.grad + bm.off + (size_t)tm * 32 * bm.ndim + tn * 32;
        for (int e = threadIdx.x; e < 32 * 32; e += 64 * NW) {
            float v = red[0][e];
#pragma unroll
            for (int q = 1; q < NW; ++q) v += red[q][e];
            out[(size_t)(e >> 5) * bm.ndim + (e & 31)] = v;
            sq += v * v;
        }
        if (gridDim.x == T) sq += reduce_tile_partials<64 * NW>(a.red, blockIdx.x, gridDim.x);
    }
    write_norm_part<NW>(sq, a.red.normpart + blockIdx.x);
    if (blockIdx.x == 0)
        for (uint32_t i = gridDim.x + threadIdx.x; i < (uint32_t)kReduceBlocks; i += 64 * NW) a.red.normpart[i] = 0.0f;
}
constexpr int kDwfWaves = 8;

// The fp32 counterpart of train_dw_bf16_fused_kernel, reading the row-major
// captures directly: lane (i = l % 32, k = l / 32) of a
// v_mfma_f32_32x32x2_f32 over rows r, r + 1 takes X[r + k][i] and Y[r + k][i]
// of its tile's columns as dword buffer loads (a half-wave reads one row's 128
// contiguous bytes), the row offset in an SGPR. Wave w takes the row pairs
// 2 (NW s + w), s = 0, 1, ..., in batches of U pairs loaded NB - 1 batches
// ahead into a ring of NB register sets (no copies between sets, so each
// MFMA waits only for its own two loads; batches past the end reload the
// last one), and the NW wave tiles are added in LDS in wave order. (A probe
// on the MI355X with two waves per SIMD: two dword loads per MFMA cost 8.6%
// of the MFMA rate, two 16-byte loads per four MFMAs 14%.) Workgroup b runs
// on XCD b % 8 and takes tile (b % 8) (T / 8) + b / 8 of the T tiles, ordered
// (matrix, hidden block, embed block): an XCD's tiles are all embed columns
// of a run of hidden blocks of one matrix, so each capture column strip is
// fetched into as few L2s as can be (4096 rows, 2 blocks, hidden 512: 19.6 us
// against 26.7 us with tile b on workgroup b). The loop is bound by each CU's
// 1 MB of capture reads through L1 misses. Then the tile-partial columns and
// the norm part as in train_dw_bf16_fused_kernel.
template <int NW, int U, int NB>
__global__ void __launch_bounds__(64 * NW) train_dw_fused_kernel(const DwFusedArgs<float> a) {
    __shared__ float red[NW][32 * 32];
    float sq = 0.0f;
    const uint32_t T = a.dw.big_tiles;  // workgroups [0, T): one 32 x 32 tile each
    if (blockIdx.x >= T) {
        // the tile-partial columns on workgroups of their own, which run beside
        // the tile workgroups instead of after some of them
        sq = reduce_tile_partials<64 * NW>(a.red, blockIdx.x - T, gridDim.x - T);
    } else {
        const uint32_t per = a.dw.tiles_per_big[0];  // every matrix has E H / 1024 tiles
        const uint32_t t = (blockIdx.x % 8) * (T / 8) + blockIdx.x / 8;
        const uint32_t mi = t / per, eb = (t % per) % (kEmbed / 32), hb = (t % per) / (kEmbed / 32);
        const BigMatT<float>& bm = a.dw.big[mi];
        const bool up = bm.mdim == (uint32_t)kEmbed;  // up: X is the embed side
        const uint32_t tm = up ? eb : hb, tn = up ? hb : eb;
        const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
        const uint32_t xv = 4 * ((lane >> 5) * bm.ldx + tm * 32 + (lane & 31));
        const uint32_t yv = 4 * ((lane >> 5) * bm.ldy + tn * 32 + (lane & 31));
        const uint32_t batches = a.dw.rows / (2 * NW * U);  // rows: a multiple of 2 NW U NB
        auto load = [&](float (&op)[U][2], uint32_t b) {
            b = b < batches ? b : batches - 1;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t r = 2 * (NW * (b * U + u) + w);
                op[u][0] = buffer_load4(bm.x, xv, 4 * r * bm.ldx);
                op[u][1] = buffer_load4(bm.y, yv, 4 * r * bm.ldy);
            }
        };
        f32x16 acc = f32x16{};
        float op[NB][U][2];
#pragma unroll
        for (int i = 0; i + 1 < NB; ++i) {
            load(op[i], i);
            __builtin_amdgcn_sched_barrier(0);  // batch 0 first, so its MFMAs wait for it alone
        }
        for (uint32_t b = 0; b < batches; b += NB) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                // kept in this order: the loads, then the batch's MFMAs
                load(op[(i + NB - 1) % NB], b + i + NB - 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < U; ++u) acc = mfma32x32x2(op[i][u][0], op[i][u][1], acc);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) red[w][c32_row(r, lane) * 32 + (lane & 31)] = acc[r];
        __syncthreads();
        float* out = a.red.grad + bm.off + (size_t)tm * 32 * bm.ndim + tn * 32;
        for (int e = threadIdx.x; e < 32 * 32; e += 64 * NW) {
            float v = red[0][e];
#pragma unroll
            for (int q = 1; q < NW; ++q) v += red[q][e];
            out[(size_t)(e >> 5) * bm.ndim + (e & 31)] = v;
            sq += v * v;
        }
        if (gridDim.x == T) sq += reduce_tile_partials<64 * NW>(a.red, blockIdx.x, gridDim.x);
    }
    write_norm_part<NW>(sq, a.red.normpart + blockIdx.x);
    if (blockIdx.x == 0)
        for (uint32_t i = gridDim.x + threadIdx.x; i < (uint32_t)kReduceBlocks; i += 64 * NW) a.red.normpart[i] = 0.0f;
}
constexpr int kDwf32Waves = 8, kDwf32U = 8, kDwf32Sets = 2;

// The block matrices are contiguous from float_group: per block up [128 x H]
// then down [H x 128]. Both matrix kinds split into (128 x H) / 1024 tiles of
// 32 x 32; tile t's matrix, its row/column extents and the tile's origin.
constexpr int kTT = 32;  // block-matrix tile edge of the Adam and derive kernels
struct MatTile {
    uint32_t base;  // arena offset of the matrix
    uint32_t rows, cols;
    uint32_t r0, c0;
};
__device__ __forceinline__ MatTile mat_tile(uint32_t t, uint32_t float_group, uint32_t H) {
    const uint32_t per = H * kEmbed / (kTT * kTT);  // tiles per matrix
    const uint32_t mi = t / per, tt = t % per;
    MatTile m;
    m.base = float_group + mi * kEmbed * H;
    m.rows = (mi & 1) ? H : kEmbed;
    m.cols = (mi & 1) ? kEmbed : H;
    m.r0 = (tt / (m.cols / kTT)) * kTT;
    m.c0 = (tt % (m.cols / kTT)) * kTT;
    return m;
}
constexpr int kTileLd = kTT + 1;  // LDS row stride of such a tile

// Packs lds[(k0 + i) * kTileLd + n], i = 0..7, as eight bf16 (16 bytes).
__device__ __forceinline__ u32x4 pack_bf16_column(const float* lds, int k0, int n) {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)bf16_rne(lds[(k0 + 2 * j) * kTileLd + n]) |
               ((uint32_t)bf16_rne(lds[(k0 + 2 * j + 1) * kTileLd + n]) << 16);
    return w;
}

// Packs lds[n * kTileLd + k0 + i], i = 0..7, as eight bf16 (16 bytes).
__device__ __forceinline__ u32x4 pack_bf16_row(const float* lds, int n, int k0) {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)bf16_rne(lds[n * kTileLd + k0 + 2 * j]) |
               ((uint32_t)bf16_rne(lds[n * kTileLd + k0 + 2 * j + 1]) << 16);
    return w;
}

// Writes the tile held in lds ([r][c], stride kTileLd) to the fragment-tiled
// copies: frag_fwd32 and frag_fwd16 read its transpose (rows n = c,
// contraction k = r, K = rows), frag_bwd16 the matrix as stored (n = r, k = c,
// K = cols). Each thread writes one float4 (four consecutive k of one n) to
// each; a wave's 64 float4s form one 1 KB run. The bf16 copies (when given)
// take 8 k per thread: threads 0-127 the transpose's 32-wide strip (two
// k-groups of 16) and the matrix's two 16-wide strips, threads 128-255 the
// transpose's two 16-wide strips (one k-group of 32 each). Starts with a
// barrier.
__device__ __forceinline__ void store_tile_frags(const MatTile& m, const float* lds, float* fwd32, float* fwd16,
                                                 float* bwd16, uint16_t* fwd32b, uint16_t* fwd16b,
                                                 uint16_t* bwd16b) {
    __syncthreads();
    const int t = threadIdx.x;
    if (fwd32) {  // 32-wide strips: the tile is one strip's four k-groups, 4 KB in a row
        const int n = t & 31, k = 8 * (t >> 6) + 4 * ((t >> 5) & 1);
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = lds[(k + j) * kTileLd + n];
        *reinterpret_cast<f32x4*>(fwd32 + m.base + frag_index<32>(m.c0 + n, m.r0 + k, m.rows)) = v;
    }
    if (fwd16 || bwd16) {
        const int n = 16 * (t >> 7) + (t & 15), k = 16 * ((t >> 6) & 1) + 4 * ((t >> 4) & 3);
        f32x4 vb, vf;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            vb[j] = lds[n * kTileLd + k + j];
            vf[j] = lds[(k + j) * kTileLd + n];
        }
        if (bwd16) *reinterpret_cast<f32x4*>(bwd16 + m.base + frag_index<16>(m.r0 + n, m.c0 + k, m.cols)) = vb;
        if (fwd16) *reinterpret_cast<f32x4*>(fwd16 + m.base + frag_index<16>(m.c0 + n, m.r0 + k, m.rows)) = vf;
    }
    if (t < 128) {
        const int ln = t & 63, nb = ln & 31, kb = 16 * (t >> 6) + 8 * (ln >> 5);
        if (fwd32b)
            *reinterpret_cast<u32x4*>(fwd32b + m.base + frag_index_b<32>(m.c0 + nb, m.r0 + kb, m.rows)) =
                pack_bf16_column(lds, kb, nb);
        const int nr = 16 * (t >> 6) + (ln & 15), kr = 8 * (ln >> 4);
        if (bwd16b)
            *reinterpret_cast<u32x4*>(bwd16b + m.base + frag_index_b<16>(m.r0 + nr, m.c0 + kr, m.cols)) =
                pack_bf16_row(lds, nr, kr);
    } else if (fwd16b) {
        const int t2 = t - 128, ln = t2 & 63, nb = 16 * (t2 >> 6) + (ln & 15), kb = 8 * (ln >> 4);
        *reinterpret_cast<u32x4*>(fwd16b + m.base + frag_index_b<16>(m.c0 + nb, m.r0 + kb, m.rows)) =
            pack_bf16_column(lds, kb, nb);
    }
}

// The fragment-tiled copies from params, one tile per workgroup.
__global__ void __launch_bounds__(256) derive_blocks_kernel(const float* __restrict__ param, float* __restrict__ fwd32,
                                                            float* __restrict__ fwd16, float* __restrict__ bwd16,
                                                            uint16_t* fwd32b, uint16_t* fwd16b, uint16_t* bwd16b,
                                                            uint32_t float_group, uint32_t H) {
    __shared__ float lds[kTT * kTileLd];
    const MatTile m = mat_tile(blockIdx.x, float_group, H);
    const int t = threadIdx.x, c = t & (kTT - 1);
#pragma unroll
    for (int e = 0; e < kTT * kTT / 256; ++e) {
        const int r = (256 / kTT) * e + t / kTT;
        lds[r * kTileLd + c] = param[m.base + (size_t)(m.r0 + r) * m.cols + m.c0 + c];
    }
    store_tile_frags(m, lds, fwd32, fwd16, bwd16, fwd32b, fwd16b, bwd16b);
}

struct AdamArgs {
    float* param;
    float* frag_fwd32;
    float* frag_fwd16;
    float* frag_bwd16;
    uint16_t* frag_fwd32_bf;
    uint16_t* frag_fwd16_bf;
    uint16_t* frag_bwd16_bf;
    const float* grad;
    float* mom;
    float* var;
    const float* normpart;
    float* mb_stats;
    uint32_t count, float_group, off_head, hidden, mat_tiles;
    float lr, beta1_pow, beta2_pow, max_grad_norm;
};

// One parameter's Adam inputs, loaded before the global norm is known so the
// two memory latencies overlap.
struct AdamIn {
    float g, m, v, p;
};
__device__ __forceinline__ AdamIn adam_load(const AdamArgs& a, uint32_t i) {
    return AdamIn{a.grad[i], a.mom[i], a.var[i], a.param[i]};
}

// model/optimizer.metal:36-60 for element i with the clip scale applied.
__device__ __forceinline__ float adam_elem(const AdamArgs& a, uint32_t i, const AdamIn& in, float scale) {
    const float beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f;
    const float g = in.g * scale;
    const float m = beta1 * in.m + (1.0f - beta1) * g;
    const float v = beta2 * in.v + (1.0f - beta2) * g * g;
    a.mom[i] = m;
    a.var[i] = v;
    const float mHat = m / (1.0f - a.beta1_pow);
    const float vHat = v / (1.0f - a.beta2_pow);
    const float p = in.p - a.lr * mHat / (sqrtf(vHat) + eps);
    a.param[i] = p;
    return p;
}

// Every wave adds the kReduceBlocks partial norms in the same order, so all
// workgroups see the same norm without synchronising with each other; returns
// the clip scale (model/optimizer.metal:49) and workgroup 0 records the norm.
__device__ __forceinline__ float adam_clip_scale(const AdamArgs& a) {
    const int lane = threadIdx.x & 63;
    float ns = 0.0f;
#pragma unroll
    for (int k = 0; k < kReduceBlocks / 64; ++k) ns += a.normpart[lane + 64 * k];
    const float norm = sqrtf(group_sum<64>(ns));
    if (blockIdx.x == 0 && threadIdx.x == 0) a.mb_stats[5] = norm;
    return (a.max_grad_norm > 0.0f && norm > a.max_grad_norm) ? a.max_grad_norm / (norm + 1e-6f) : 1.0f;
}

// Workgroups [0, mat_tiles) update one 32 x 32 block-matrix tile each and
// write it to the fragment-tiled copies as well; the rest update the vector
// group and the head elementwise. Workgroup 0 also records the pre-clip norm.
__global__ void __launch_bounds__(256) adam_kernel(const AdamArgs a) {
    __shared__ float lds[kTT * kTileLd];
    constexpr int PER = kTT * kTT / 256;  // tile elements per thread
    const int t = threadIdx.x;
    if (blockIdx.x < a.mat_tiles) {
        const MatTile m = mat_tile(blockIdx.x, a.float_group, a.hidden);
        const int c = t & (kTT - 1);
        uint32_t idx[PER];
        AdamIn in[PER];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int r = (256 / kTT) * e + t / kTT;
            idx[e] = m.base + (m.r0 + r) * m.cols + m.c0 + c;
            in[e] = adam_load(a, idx[e]);
        }
        const float scale = adam_clip_scale(a);
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int r = (256 / kTT) * e + t / kTT;
            lds[r * kTileLd + c] = adam_elem(a, idx[e], in[e], scale);
        }
        store_tile_frags(m, lds, a.frag_fwd32, a.frag_fwd16, a.frag_bwd16, a.frag_fwd32_bf, a.frag_fwd16_bf,
                         a.frag_bwd16_bf);
        return;
    }
    const uint32_t j = (blockIdx.x - a.mat_tiles) * 256 + t;
    const uint32_t i = j < a.float_group ? j : a.off_head + (j - a.float_group);
    AdamIn in{};
    if (i < a.count) in = adam_load(a, i);
    const float scale = adam_clip_scale(a);
    if (i < a.count) adam_elem(a, i, in, scale);
}

}  // namespace dev

namespace {
size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// 32 x 32 tiles over all block matrices (each 128 x H or H x 128).
uint32_t mat_tiles(const mg_policy_view& pv) { return 2 * pv.layers * (pv.hidden * MG_EMBED / 1024); }

struct WsPlan {
    size_t off[8];
    size_t total;
    uint32_t tp_count;
};

WsPlan plan(const mg_policy_view& pv, uint32_t B) {
    const size_t E = MG_EMBED, L = pv.layers, H = pv.hidden, HD = pv.head_dim;
    WsPlan p;
    p.tp_count = (uint32_t)align256(pv.float_group + E * HD + 5);
    const size_t sizes[8] = {
        L * B * E * 4,                             // x
        L * B * H * 4,                             // v
        L * B * E * 4,                             // dhb
        L * B * H * 4,                             // dvb
        (size_t)(B / kTileRows) * p.tp_count * 4,  // tp
        (size_t)kSplits * pv.count * 4,            // partial
        (size_t)pv.count * 4,                      // grad
        (size_t)kReduceBlocks * 4,                 // normpart
    };
    size_t o = 0;
    for (int k = 0; k < 8; ++k) {
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
    ws->x = (float*)(b + p.off[0]);
    ws->v = (float*)(b + p.off[1]);
    ws->dhb = (float*)(b + p.off[2]);
    ws->dvb = (float*)(b + p.off[3]);
    ws->tp = (float*)(b + p.off[4]);
    ws->partial = (float*)(b + p.off[5]);
    ws->grad = (float*)(b + p.off[6]);
    ws->normpart = (float*)(b + p.off[7]);
    ws->tp_count = p.tp_count;
    return MG_OK;
}

int check_matrix_layout(const mg_policy_view& pv) {
    const uint32_t E = MG_EMBED, H = pv.hidden;
    MG_CHECK(pv.embed == E && H % 128 == 0, MG_ERR_INVALID, "policy: embed 128 and hidden a multiple of 128 required");
    for (uint32_t l = 0; l < pv.layers; ++l)
        MG_CHECK(pv.off_up[l] == pv.float_group + 2 * l * E * H && pv.off_down[l] == pv.off_up[l] + E * H &&
                     pv.off_head == pv.float_group + 2 * pv.layers * E * H,
                 MG_ERR_INVALID, "policy: block matrices must be contiguous from float_group");
    for (uint32_t l = 0; l <= pv.layers; ++l)
        MG_CHECK(pv.off_ln_gamma[l] == pv.off_ln_gamma[0] + 2 * l * E && pv.off_ln_beta[l] == pv.off_ln_gamma[l] + E,
                 MG_ERR_INVALID, "policy: LN parameters must be contiguous (gamma, beta per LN)");
    return MG_OK;
}

int launch_derive_blocks(hipStream_t st, const mg_policy_view& pv) {
    int rc = check_matrix_layout(pv);
    if (rc) return rc;
    hipLaunchKernelGGL(dev::derive_blocks_kernel, dim3(mat_tiles(pv)), dim3(256), 0, st, pv.params, pv.frag_fwd32,
                       pv.frag_fwd16, pv.frag_bwd16, pv.frag_fwd32_bf, pv.frag_fwd16_bf, pv.frag_bwd16_bf,
                       pv.float_group, pv.hidden);
    MG_HIP(hipGetLastError(), "derive blocks launch");
    return MG_OK;
}

// The weight-gradient jobs of one minibatch: per block, dUp and dDown from
// the captures (T: their element type); tile x tile tiles.
template <class T>
dev::DwArgsT<T> dw_args(const mg_policy_view& pv, const TrainWs& ws, uint32_t B, uint32_t splits, uint32_t tile,
                        uint32_t tile_n = 0) {
    if (!tile_n) tile_n = tile;
    const uint32_t E = MG_EMBED, H = pv.hidden;
    const T* x = reinterpret_cast<const T*>(ws.x);
    const T* v = reinterpret_cast<const T*>(ws.v);
    const T* dh = reinterpret_cast<const T*>(ws.dhb);
    const T* dv = reinterpret_cast<const T*>(ws.dvb);
    dev::DwArgsT<T> da;
    memset(&da, 0, sizeof(da));
    da.rows = B;
    da.splits = splits;
    da.count = pv.count;
    da.partial = ws.partial;
    uint32_t nb = 0, tiles = 0;
    for (uint32_t l = 0; l < pv.layers; ++l) {
        // dUp_l[k][j] = sum_r x_l[r][k] dV_l[r][j]  (model/mlp.metal:201-203)
        da.big[nb] = {x + (size_t)l * B * E, dv + (size_t)l * B * H, E, H, E, H, pv.off_up[l], 0};
        da.tiles_per_big[nb] = (E / tile) * (H / tile_n);
        tiles += da.tiles_per_big[nb++];
        // dDown_l[j][c] = sum_r V_l[r][j] dh_l[r][c]  (model/mlp.metal:205-207)
        da.big[nb] = {v + (size_t)l * B * H, dh + (size_t)l * B * E, H, E, H, E, pv.off_down[l], 0};
        da.tiles_per_big[nb] = (H / tile) * (E / tile_n);
        tiles += da.tiles_per_big[nb++];
    }
    da.nbig = nb;
    da.big_tiles = tiles;
    return da;
}

// The split row pass with the head width's compile-time bound.
template <int W>
void launch_rows_split(hipStream_t st, uint32_t B, const mg_policy_view& pv, const dev::RowsArgs& ra) {
    if (pv.head_dim <= 4)
        hipLaunchKernelGGL((dev::train_rows_split_kernel<W, 4>), dim3(B / dev::kTR), dim3(64 * W), 0, st, ra);
    else if (pv.head_dim <= 8)
        hipLaunchKernelGGL((dev::train_rows_split_kernel<W, 8>), dim3(B / dev::kTR), dim3(64 * W), 0, st, ra);
    else
        hipLaunchKernelGGL((dev::train_rows_split_kernel<W, 16>), dim3(B / dev::kTR), dim3(64 * W), 0, st, ra);
}

int launch_train_step(hipStream_t st, const mg_policy_view& pv, const mg_ppo_hparams& hp, float lr,
                      const TrainWs& ws, const TrainStep& step, const float* obs_slots, const void* action_slots,
                      const float* adv_slots, const float* ret_slots, const float* logp_slots,
                      const float* adv_stats, float* m, float* v, float* head_out, float* mb_stats) {
    const uint32_t B = step.rows;
    MG_CHECK(B % 64 == 0, MG_ERR_INVALID, "train: minibatch %u must be a multiple of 64", B);
    MG_CHECK(pv.obs_dim <= (uint32_t)dev::kMaxObsT && pv.head_dim <= (uint32_t)dev::kMaxHeadT, MG_ERR_INVALID,
             "train: OBS_DIM <= 64 and ACT_DIM + 1 <= 64 required");
    const uint32_t E = MG_EMBED, L = pv.layers, H = pv.hidden;
    const bool bf = pv.precision == MG_PRECISION_BF16;
    // weight-gradient tiles over all block matrices: 128 x 64 (fp32) or 64 x 64 (bf16)
    const uint32_t dw_tiles = bf ? 2 * L * (E / 64) * (H / 64) : 2 * L * (E * H / (dev::kDwTileM * dev::kDwTileN));
    // row splits of the block-matrix gradient sums: fp32, each split covers a
    // multiple of 32 rows and about one workgroup per CU in all; bf16, a
    // multiple of 64 rows and about two workgroups per CU (fewer splits, fewer
    // partial sums to write and add)
    const uint32_t split_rows = bf ? 16 * dev::kDwbWaves : dev::kDwRows;
    const uint32_t max_wgs = bf ? 512 : 256;
    uint32_t splits = kSplits;
    while (splits > 1 && (B % (splits * split_rows) != 0 || dw_tiles * splits > max_wgs)) splits /= 2;
    MG_CHECK(B % (splits * split_rows) == 0, MG_ERR_INVALID, "train: minibatch %u must be a multiple of %u", B,
             split_rows);

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
        if (bf)
            hipLaunchKernelGGL(dev::train_rows_kernel<true>, dim3(B / dev::kTR), dim3(dev::kTNT), 0, st, ra);
        else if (dev::rows_split_waves(pv) == 8)
            launch_rows_split<8>(st, B, pv, ra);
        else if (dev::rows_split_waves(pv) == 4)
            launch_rows_split<4>(st, B, pv, ra);
        else
            hipLaunchKernelGGL(dev::train_rows_kernel<false>, dim3(B / dev::kTR), dim3(dev::kTNT), 0, st, ra);
        MG_HIP(hipGetLastError(), "train rows launch");
    }
    dev::ReduceArgs ga;
    ga.partial = ws.partial;
    ga.tp = ws.tp;
    ga.grad = ws.grad;
    ga.normpart = ws.normpart;
    ga.splits = splits;
    ga.tiles = B / kTileRows;
    ga.tp_count = ws.tp_count;
    ga.count = pv.count;
    ga.float_group = pv.float_group;
    ga.off_head = pv.off_head;
    ga.head_count = E * pv.head_dim;
    ga.mb_stats = mb_stats;
    ga.inv_rows = 1.0f / (float)B;
    // kRedCols tile-partial columns per small workgroup, at most half the grid
    const uint32_t cols = pv.float_group + E * pv.head_dim + 5, cw = dev::kRedCols;
    ga.small_wgs = (cols + cw - 1) / cw < kReduceBlocks / 2 ? (cols + cw - 1) / cw : kReduceBlocks / 2;
    // 128 to 1024 tiles of 32 x 32: weight gradients without row splits,
    // fused with the tile-partial sums (one launch instead of two; fp32 at
    // 4096 rows, 2 blocks, hidden 512: 71.8 -> 67.9 us per minibatch)
    const uint32_t tiles32 = 2 * L * (E / 32) * (H / 32);
    if (bf && tiles32 >= 128 && tiles32 <= (uint32_t)kReduceBlocks && B % (16 * dev::kDwfWaves) == 0) {
        TimedLaunch tl(MG_K_TRAIN_DW, st);
        dev::DwFusedArgs<uint16_t> fa;
        fa.dw = dw_args<uint16_t>(pv, ws, B, 1, 32);
        fa.red = ga;
        const uint32_t grid = tiles32 + ga.small_wgs <= (uint32_t)kReduceBlocks ? tiles32 + ga.small_wgs : tiles32;
        hipLaunchKernelGGL((dev::train_dw_bf16_fused_kernel<dev::kDwfWaves, 4>), dim3(grid),
                           dim3(64 * dev::kDwfWaves), 0, st, fa);
        MG_HIP(hipGetLastError(), "train dW launch");
    } else if (!bf && tiles32 >= 128 && tiles32 <= (uint32_t)kReduceBlocks &&
               B % (2 * dev::kDwf32Waves * dev::kDwf32U * dev::kDwf32Sets) == 0) {
        TimedLaunch tl(MG_K_TRAIN_DW, st);
        dev::DwFusedArgs<float> fa;
        fa.dw = dw_args<float>(pv, ws, B, 1, 32);
        fa.red = ga;
        // the tile-partial columns on small_wgs extra workgroups where the
        // partial norms have room for them, else on the first tile workgroups
        const uint32_t grid = tiles32 + ga.small_wgs <= (uint32_t)kReduceBlocks ? tiles32 + ga.small_wgs : tiles32;
        hipLaunchKernelGGL((dev::train_dw_fused_kernel<dev::kDwf32Waves, dev::kDwf32U, dev::kDwf32Sets>), dim3(grid),
                           dim3(64 * dev::kDwf32Waves), 0, st, fa);
        MG_HIP(hipGetLastError(), "train dW launch");
    } else {
        {  // 2. block-matrix weight gradients
            TimedLaunch tl(MG_K_TRAIN_DW, st);
            if (bf) {
                const auto da = dw_args<uint16_t>(pv, ws, B, splits, 64);
                hipLaunchKernelGGL((dev::train_dw_bf16_kernel<dev::kDwbWaves, 2>), dim3(dw_tiles * splits),
                                   dim3(64 * dev::kDwbWaves), 0, st, da);
            } else {
                const auto da = dw_args<float>(pv, ws, B, splits, dev::kDwTileM, dev::kDwTileN);
                hipLaunchKernelGGL(dev::train_dw_kernel, dim3(dw_tiles * splits), dim3(64 * dev::kDwWaves), 0, st,
                                   da);
            }
            MG_HIP(hipGetLastError(), "train dW launch");
        }
        {  // 3. gradient assembly + partial norms
            TimedLaunch tl(MG_K_GRAD_REDUCE, st);
            hipLaunchKernelGGL(dev::grad_reduce_kernel, dim3(kReduceBlocks), dim3(256), 0, st, ga);
            MG_HIP(hipGetLastError(), "grad reduce launch");
        }
    }
    {  // 4. Adam
        TimedLaunch tl(MG_K_ADAM, st);
        dev::AdamArgs aa;
        aa.param = pv.params;
        // only the copies the next minibatch's row pass reads; the others are
        // derived once before the next collect or forward
        aa.frag_fwd32 = nullptr;
        aa.frag_fwd16 = bf ? nullptr : pv.frag_fwd16;
        aa.frag_bwd16 = bf ? nullptr : pv.frag_bwd16;
        aa.frag_fwd32_bf = nullptr;
        aa.frag_fwd16_bf = bf ? pv.frag_fwd16_bf : nullptr;
        aa.frag_bwd16_bf = bf ? pv.frag_bwd16_bf : nullptr;
        aa.grad = ws.grad;
        aa.mom = m;
        aa.var = v;
        aa.normpart = ws.normpart;
        aa.mb_stats = mb_stats;
        aa.count = pv.count;
        aa.float_group = pv.float_group;
        aa.off_head = pv.off_head;
        aa.hidden = H;
        aa.mat_tiles = mat_tiles(pv);
        aa.lr = lr;
        aa.beta1_pow = step.beta1_pow;
        aa.beta2_pow = step.beta2_pow;
        aa.max_grad_norm = hp.max_grad_norm;
        const uint32_t lin = pv.float_group + (pv.count - pv.off_head);
        hipLaunchKernelGGL(dev::adam_kernel, dim3(aa.mat_tiles + (lin + 255) / 256), dim3(256), 0, st, aa);
        MG_HIP(hipGetLastError(), "adam launch");
    }
    return MG_OK;
}

}  // namespace mg
