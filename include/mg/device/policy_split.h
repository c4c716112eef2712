// The hidden-unit split of a 16-row policy tile: the layout of the fp32 row
// pass of a PPO minibatch (metalgym_amd/csrc/rows_split.h) and of collect's
// fp32 16-row tiles (split_forward16 below).
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
// LayerNorm and the head reduce over TPR = 4 W lanes (DPP and readlane) and
// need no LDS round trip.
#pragma once
#include "policy.h"

namespace mg {
namespace dev {

constexpr int kSplitRows = 16;  // rows of a split tile

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
template <int S, bool FWD_ONLY = false>
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
    // The next chunk of the sequence; past its end, p itself (FWD_ONLY: the
    // forward's blocks only, then the first chunk again).
    __device__ __forceinline__ SkPos next(SkPos p) const {
        if (++p.k < nc) return p;
        p.k = 0;
        if (!p.bwd) {
            if (++p.l < L) return p;
            if (FWD_ONLY) return SkPos{0, 0, 0};  // wraps: the next forward's first chunk
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
    template <class Seq>
    __device__ __forceinline__ void start(const Seq& seq, const SkPos& p) {
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
// red: W buffers of kSplitRows x kLds floats, one per wave.
template <int W, int NV>
__device__ __forceinline__ RowVec<NV> sk_reduce_buf(float* red, const f32x4 (&hp)[8], int wave, int row, int c0) {
    constexpr int RB = kSplitRows * kLds;  // floats per wave buffer
    const int lane = threadIdx.x & 63;
    float* rw = red + wave * RB + 4 * (lane >> 4) * kLds + (lane & 15);
#pragma unroll
    for (int ct = 0; ct < 8; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) rw[r * kLds + 16 * ct] = hp[ct][r];
    __syncthreads();
    RowVec<NV> s = rv_load<NV>(red + row * kLds + c0);
#pragma unroll
    for (int w = 1; w < W; ++w) s = rv_add(s, rv_load<NV>(red + w * RB + row * kLds + c0));
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


// LDS of split_forward16: the block input broadcast and the waves' partials
// of a block output.
template <int W>
struct alignas(16) SplitFwdSmem {
    float xs[kSplitRows * kLds];
    float red[W][kSplitRows * kLds];
};

// Policy forward of a 16-row tile in the split layout (model/ppo.h:575-626:
// embed, L blocks h += relu(LN(h) Up) Down, final LN, head): obs staged in
// obsL ([16][O], LDS) -> head in headL ([16][HD], LDS), ending with a
// barrier. sp: the small parameters (arena or LDS copies). OC: O at compile
// time. Reads frag_fwd16. The same arithmetic as the row pass's forward,
// without its captures. wst carries the weight stream from one call to the
// next (first: the first call, which starts it): the last chunk's refills
// load the next call's first operands, so they arrive during the caller's
// work between the forwards.
template <int W, int OC>
__device__ __forceinline__ void split_forward16(const mg_policy_view& pv, const SmallParams& sp, SplitFwdSmem<W>& sm,
                                                SkStream<8 / W>& wst, bool first, const float* obsL, float* headL,
                                                int HD) {
    constexpr int NT = 64 * W, S = 8 / W, TPR = NT / kSplitRows, CPT = kEmbed / TPR, NV = CPT / 4;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = tid / TPR, lk = tid % TPR, c0 = CPT * lk;
    const int H = (int)pv.hidden, NL = (int)pv.layers, NC = H / kChunk;
    const int rot = (wave + (int)(blockIdx.x >> 3)) % NC;
    const SkSeq<S, true> seq{pv.frag_fwd16 + pv.float_group, pv.frag_bwd16 + pv.float_group, NL, NC, wave, rot,
                             (uint32_t)kEmbed * (uint32_t)H};
    SkPos pos{0, 0, 0};
    if (first) wst.start(seq, pos);
    // model/input.metal:11-27
    RowVec<NV> h;
#pragma unroll
    for (int c = 0; c < CPT; ++c) h[c] = sp.bin[c0 + c];
#pragma unroll
    for (int k = 0; k < OC; ++k) {
        const float ok = obsL[row * OC + k];
#pragma unroll
        for (int c = 0; c < CPT; ++c) h[c] += ok * sp.win[k * kEmbed + c0 + c];
    }
    for (int l = 0; l < NL; ++l) {
        RowVec<NV> x, xn;
        float sd;
        sk_layernorm<TPR>(h, sp.ln + l * 2 * kEmbed, sp.ln + l * 2 * kEmbed + kEmbed, c0, x, xn, sd);
        rv_store(sm.xs + row * kLds + c0, x);
        __syncthreads();  // X complete; every wave is past its reads of red
        f32x4 xb[8];
        sk_load_input(sm.xs, xb);
        f32x4 hp[8];
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) hp[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = 0; k < NC; ++k) {  // model/mlp.metal:18-86 for this wave's units of a chunk
            const SkPos nx = seq.next(pos);
            f32x4 v[S];
#pragma unroll
            for (int s = 0; s < S; ++s) v[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            wst.gemm0(v, xb, seq.role0(nx));
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[s][r] = v[s][r] > 0.0f ? v[s][r] : 0.0f;
            wst.gemm1(hp, v, seq.role1(nx), seq.stride1());
            pos = nx;
        }
        h = rv_add(h, sk_reduce_buf<W, NV>(&sm.red[0][0], hp, wave, row, c0));  // model/elementwise.metal:4-13
    }
    RowVec<NV> x, xn;
    float sd;
    sk_layernorm<TPR>(h, sp.ln + NL * 2 * kEmbed, sp.ln + NL * 2 * kEmbed + kEmbed, c0, x, xn, sd);
    // model/linear.metal:17-37: head[row][j] = x_f[row] . W_head[:, j]
    for (int j = 0; j < HD; ++j) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < CPT; ++c) acc += x[c] * sp.wh[(c0 + c) * HD + j];
        acc = group_sum<TPR>(acc);
        if (lk == 0) headL[row * HD + j] = acc;
    }
    __syncthreads();
}

}  // namespace dev
}  // namespace mg
