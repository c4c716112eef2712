// The fp32 row pass of a PPO minibatch (the work of train_rows_kernel<false>:
// forward recompute with capture, loss, backward dX chain, tile partials) with
// the hidden units split over the waves, so that no chunk GEMM waits on a
// barrier. Included by train_kernels.hip.
//
// A workgroup owns 16 rows on W waves (W = 4: one per SIMD; W = 8: two). Wave
// w owns the S = 8 / W 16-unit strips 128 c + 16 (S w + s), s < S, of every
// 128-wide chunk c and runs its chunks without synchronising with the other
// waves:
//   - the first GEMM computes its share of the chunk transposed, V^T = W0 X^T
//     (16 units x 16 rows per strip on v_mfma_f32_16x16x4_f32, one
//     accumulator chain per strip): the weights are the A operand, streamed
//     from the fragment-tiled copies, and the block input X (the LN output, or
//     dh in the backward) is the B operand, loaded from LDS into registers
//     once per block;
//   - the result registers, after relu (or the relu mask), are exactly the A
//     operand of the second GEMM, which adds V W1 for this wave's units to a
//     private 16 x 128 partial of the block output.
// Once per block the W partials are added in LDS in wave order. Outside the
// GEMMs each thread holds CPT = 32 / W consecutive columns of one row, so
// LayerNorm, the head and the loss reduce over TPR = 4 W lanes (DPP and
// readlane) and need no LDS round trip. The captures for the weight gradients
// have the row-major layouts of train_rows_kernel<false>.
#pragma once

namespace mg {
namespace dev {

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

// The chunk a wave's GEMM pair works on: the forward's blocks 0 .. L-1, then
// the backward's L-1 .. 0, chunks in this wave's order. Wave w of workgroup b
// starts block by block at chunk (w + b / 8) mod NC (workgroups go to the 8
// XCDs round robin), so at any time the waves of a CU and the CUs of an XCD
// stream different chunks' weights instead of all requesting the same lines
// from L2 at once after a barrier. The order changes only the summation order
// of a wave's partial over the chunks.
struct SkPos {
    int bwd, l, k;  // k: position in the wave's chunk order
};

// Where a chunk's operands live, from the contiguous block matrices (up_l at
// float_group + 2 l E H, down_l right after it). Role 0 is W0 = up^T
// (forward) or down as stored (backward), both [hidden][128]: the wave's S
// strips 8 c + S w + s, each of eight 16-wide k-groups, all contiguous
// (frag_index<16>, K = 128). Role 1 is W1 = down^T (forward) or up as stored
// (backward), both [128][hidden]: k-groups 8 c + S w + s in each of the eight
// 16-row strips (K = hidden), contiguous within a strip, the strips 16 hidden
// rows apart.
template <int S>
struct SkSeq {
    const float* fwd;  // frag_fwd16 + float_group
    const float* bwd;  // frag_bwd16 + float_group
    int L, nc, wave, rot;
    uint32_t EH;  // 128 hidden: elements of one block matrix
    __device__ __forceinline__ int chunk(const SkPos& p) const {
        const int c = p.k + rot;
        return c < nc ? c : c - nc;
    }
    __device__ __forceinline__ const float* role0(const SkPos& p) const {
        const float* m = p.bwd ? bwd + (size_t)(2 * p.l + 1) * EH : fwd + (size_t)(2 * p.l) * EH;
        return m + (size_t)(8 * chunk(p) + S * wave) * (16 * kEmbed);
    }
    __device__ __forceinline__ const float* role1(const SkPos& p) const {
        const float* m = p.bwd ? bwd + (size_t)(2 * p.l) * EH : fwd + (size_t)(2 * p.l + 1) * EH;
        return m + (size_t)chunk(p) * (16 * kChunk) + 256 * S * wave;
    }
    __device__ __forceinline__ uint32_t stride1() const { return EH / 8; }  // 16 hidden rows: 16 H
    // The next chunk of the sequence; past its end, p itself.
    __device__ __forceinline__ SkPos next(SkPos p) const {
        if (++p.k < nc) return p;
        p.k = 0;
        if (!p.bwd) {
            if (++p.l < L) return p;
            p.bwd = 1;
            p.l = L - 1;
            return p;
        }
        if (--p.l >= 0) return p;
        return SkPos{1, 0, nc - 1};
    }
};

// The operand registers of both roles (8 S float4s each per lane): w0[8 s + g]
// is k-group g of strip s, w1[S ct + s] strip s's k-group in column strip ct.
// The loads are buffer loads with the k-group offset in an SGPR: the 64-bit
// address arithmetic of global loads ran on the VALU between the MFMAs and
// cost 3 us of the fp32 row pass. Each float4 is refilled for the same role
// of the next chunk right after its MFMAs; past the end of the sequence a GEMM
// reloads its own operand, so every path issues the same loads and the
// vector-memory wait counts stay exact.
template <int S>
struct SkStream {
    f32x4 w0[8 * S], w1[8 * S];

    // one k-group: 16 bytes per lane of the 1 KB run at float offset off
    __device__ __forceinline__ static f32x4 load(const float* p, uint32_t off) {
        return buffer_load16(p, 16 * (threadIdx.x & 63), 4 * off);
    }
    __device__ __forceinline__ void start(const SkSeq<S>& seq, const SkPos& p) {
        const float* a = seq.role0(p);
        const float* b = seq.role1(p);
        const uint32_t s1 = seq.stride1();
#pragma unroll
        for (int k = 0; k < 8 * S; ++k) w0[k] = load(a, 256 * k);
#pragma unroll
        for (int ct = 0; ct < 8; ++ct)
#pragma unroll
            for (int s = 0; s < S; ++s) w1[S * ct + s] = load(b, s1 * ct + 256 * s);
    }
    // acc[s] += W0 strip s . xb: acc[s] lane l register r = unit 4 (l / 16) +
    // r of strip s, row l % 16; refills from nx (role 0 of the next chunk)
    __device__ __forceinline__ void gemm0(f32x4 (&acc)[S], const f32x4 (&xb)[8], const float* nx) {
#pragma unroll
        for (int g = 0; g < 8; ++g) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int s = 0; s < S; ++s) acc[s] = mfma16x16x4(w0[8 * s + g][j], xb[g][j], acc[s]);
#pragma unroll
            for (int s = 0; s < S; ++s) w0[8 * s + g] = load(nx, 256 * (8 * s + g));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // hp[ct] += v W1: v[s] is role 0's result for strip s; hp[ct] lane l
    // register r = row 4 (l / 16) + r, column 16 ct + l % 16; refills from nx
    // (role 1 of the next chunk, column strips s1 apart)
    __device__ __forceinline__ void gemm1(f32x4 (&hp)[8], const f32x4 (&v)[S], const float* nx, uint32_t s1) {
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int j = 0; j < 4; ++j) hp[ct] = mfma16x16x4(v[s][j], w1[S * ct + s][j], hp[ct]);
#pragma unroll
            for (int s = 0; s < S; ++s) w1[S * ct + s] = load(nx, s1 * ct + 256 * s);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// The block input's B-operand registers: lane (n = l % 16, q = l / 16) holds
// X[n][16 g + 4 q .. + 3] for k-group g (the K order of the fragment layout).
__device__ __forceinline__ void sk_load_input(const float* xs, f32x4 (&xb)[8]) {
    const int lane = threadIdx.x & 63;
    const float* p = xs + (lane & 15) * kLds + 4 * (lane >> 4);
#pragma unroll
    for (int g = 0; g < 8; ++g) xb[g] = *reinterpret_cast<const f32x4*>(p + 16 * g);
}

// A thread's CPT consecutive columns of one row.
template <int NV>
struct RowVec {
    float c[4 * NV];
    __device__ __forceinline__ float& operator[](int i) { return c[i]; }
    __device__ __forceinline__ float operator[](int i) const { return c[i]; }
};

template <int NV>
__device__ __forceinline__ RowVec<NV> rv_load(const float* p) {
    RowVec<NV> r;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const f32x4 t = *reinterpret_cast<const f32x4*>(p + 4 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) r.c[4 * i + j] = t[j];
    }
    return r;
}
template <int NV>
__device__ __forceinline__ void rv_store(float* p, const RowVec<NV>& r) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
        *reinterpret_cast<f32x4*>(p + 4 * i) = f32x4{r.c[4 * i], r.c[4 * i + 1], r.c[4 * i + 2], r.c[4 * i + 3]};
}
template <int NV>
__device__ __forceinline__ RowVec<NV> rv_zero() {
    RowVec<NV> r;
#pragma unroll
    for (int i = 0; i < 4 * NV; ++i) r.c[i] = 0.0f;
    return r;
}
template <int NV>
__device__ __forceinline__ RowVec<NV> rv_add(const RowVec<NV>& a, const RowVec<NV>& b) {
    RowVec<NV> r;
#pragma unroll
    for (int i = 0; i < 4 * NV; ++i) r.c[i] = a.c[i] + b.c[i];
    return r;
}

// The block output: this wave's partial to LDS, a barrier, then the thread's
// row and columns summed over the waves in order.
template <int W>
__device__ __forceinline__ RowVec<SkShape<W>::NV> sk_reduce(SkSmem<W>& L, const f32x4 (&hp)[8], int wave, int row,
                                                            int c0) {
    constexpr int NV = SkShape<W>::NV;
    const int lane = threadIdx.x & 63;
    float* rw = L.red[wave] + 4 * (lane >> 4) * kLds + (lane & 15);
#pragma unroll
    for (int ct = 0; ct < 8; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) rw[r * kLds + 16 * ct] = hp[ct][r];
    __syncthreads();
    RowVec<NV> s = rv_load<NV>(L.red[0] + row * kLds + c0);
#pragma unroll
    for (int w = 1; w < W; ++w) s = rv_add(s, rv_load<NV>(L.red[w] + row * kLds + c0));
    return s;
}

// model/layernorm.metal:10-71 on a row held by TPR lanes (CPT columns each).
template <int TPR, int NV>
__device__ __forceinline__ void sk_layernorm(const RowVec<NV>& h, const float* gamma, const float* beta, int c0,
                                             RowVec<NV>& x, RowVec<NV>& xn, float& sd) {
    constexpr int CPT = 4 * NV;
    float s = h[0];
#pragma unroll
    for (int c = 1; c < CPT; ++c) s += h[c];
    s = group_sum<TPR>(s);
    const float mean = s / (float)kEmbed;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const float d = h[c] - mean;
        q += d * d;
    }
    q = group_sum<TPR>(q);
    sd = sqrtf(q / (float)kEmbed + 1e-5f);
    const float rstd = 1.0f / sd;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        xn[c] = (h[c] - mean) * rstd;
        x[c] = gamma[c0 + c] * xn[c] + beta[c0 + c];
    }
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
        const float o0 = tid < n_obs ? a.obs_slots[g0 * O + tid] : 0.0f;
        const float h0 = tid < n_wh ? pv.params[pv.off_head + tid] : 0.0f;
        const float w0 = tid < n_win ? pv.params[pv.off_in_w + tid] : 0.0f;
        const float b0 = tid < kEmbed ? pv.params[pv.off_in_b + tid] : 0.0f;
        const float l0 = tid < n_ln ? lnp[tid] : 0.0f;
        const float l1 = tid + NT < n_ln ? lnp[tid + NT] : 0.0f;
        if (tid < n_obs) L.obs[tid] = o0;
        if (tid < n_wh) L.wh[tid] = h0;
        if (tid < n_win) winL[tid] = w0;
        if (tid < kEmbed) binL[tid] = b0;
        if (tid < n_ln) L.ln[tid] = l0;
        if (tid + NT < n_ln) L.ln[tid + NT] = l1;
    }
    // the rest, four elements' loads ahead of their stores (VoxelNav16's
    // 3840-float W_in: 51.0 -> 50.4 us per minibatch; CartPole's arrays need
    // no second element)
#pragma unroll 4
    for (int idx = tid + NT; idx < n_obs; idx += NT) L.obs[idx] = a.obs_slots[g0 * O + idx];
#pragma unroll 4
    for (int idx = tid + NT; idx < n_wh; idx += NT) L.wh[idx] = pv.params[pv.off_head + idx];
#pragma unroll 4
    for (int idx = tid + NT; idx < n_win; idx += NT) winL[idx] = pv.params[pv.off_in_w + idx];
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
