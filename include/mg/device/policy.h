// Fused residual-MLP policy forward for a tile of M rows (M = 32 or 64) on one
// 256-thread workgroup, fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// Network (model/ppo.h:575-626): embed h = obs W_in + b_in; per block
// h += relu(LN(h) Up) Down; final LN; head = LN(h) W_head (no bias).
//
// Mapping: wave w owns embed columns [32w, 32w + 32) of the residual stream h,
// held in MFMA accumulator layout (f32x16 per 32-row tile). Each block runs the
// hidden dimension in 128-wide chunks so the hidden activations never leave the
// CU: V_c = relu(x Up[:, c]) is computed by the four waves (32 hidden columns
// each), staged in LDS, and immediately contracted with Down[c, :] into the
// block output accumulator. LN outputs and hidden chunks are the A operands
// (LDS, float4 reads); weights are the B operands, read straight from L2 (the
// whole 1 MB policy stays L2-resident across the grid).
//
// K-order permutation: for a group of 8 k-values, lane (m, h) reads
// x[m][8g + 4h .. 8g + 4h + 3] as one float4 and MFMA step j contracts
// k = 8g + 4h + j, so B supplies W[8g + 4h + j][n]. Every k is covered once;
// only the fp32 summation order differs from a sequential loop.
#pragma once
#include "common.h"

namespace mg {
namespace dev {

constexpr int kLds = kEmbed + 4;  // LDS row stride in floats (pad against bank conflicts)
constexpr int kChunk = 128;       // hidden columns per chunk

template <int M>
struct FwdSmem {
    float xs[M * kLds];  // LN output (A operand of the up GEMM)
    float vs[M * kLds];  // relu'd hidden chunk (A operand of the down GEMM)
};

template <int M>
struct FwdRegs {
    static constexpr int RT = M / 32;
    f32x16 h[RT];  // residual stream; tile rt, register r -> row 32 rt + c32_row(r, lane), col 32 w + lane % 32
};

// model/input.metal:11-27: h = b_in + sum_k obs[k] W_in[k], in k order.
// obsL is [M][O] in LDS.
template <int M>
__device__ __forceinline__ void fwd_embed(const mg_policy_view& pv, const float* obsL, int O, FwdRegs<M>& R) {
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int col = 32 * w + (lane & 31);
    const float* W = pv.params + pv.off_in_w + col;
    const float b = pv.params[pv.off_in_b + col];
#pragma unroll
    for (int rt = 0; rt < FwdRegs<M>::RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) R.h[rt][r] = b;
    for (int k = 0; k < O; ++k) {
        const float wk = W[k * kEmbed];
#pragma unroll
        for (int rt = 0; rt < FwdRegs<M>::RT; ++rt)
#pragma unroll
            for (int r = 0; r < 16; ++r) R.h[rt][r] += obsL[(32 * rt + c32_row(r, lane)) * O + k] * wk;
    }
}

// model/layernorm.metal:10-71 on the register tile; the result goes to sm.xs.
// If xn_out/sd_out are given, the normalised values and the standard deviation
// are also written there ([M][128] and [M], row-major) for the backward pass.
template <int M>
__device__ __forceinline__ void fwd_layernorm(FwdSmem<M>& sm, const FwdRegs<M>& R, const float* gamma,
                                              const float* beta, float* xn_out = nullptr, float* sd_out = nullptr,
                                              float* x_out = nullptr) {
    constexpr int TPR = 256 / M;       // threads per row
    constexpr int CPT = kEmbed / TPR;  // columns per thread
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int rt = 0; rt < FwdRegs<M>::RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) sm.xs[(32 * rt + c32_row(r, lane)) * kLds + 32 * w + (lane & 31)] = R.h[rt][r];
    __syncthreads();
    const int row = tid / TPR, part = tid % TPR, c0 = part * CPT;
    float* xr = sm.xs + row * kLds + c0;
    float x[CPT];
#pragma unroll
    for (int c = 0; c < CPT; c += 4) {
        f32x4 v = *reinterpret_cast<const f32x4*>(xr + c);
        x[c] = v[0], x[c + 1] = v[1], x[c + 2] = v[2], x[c + 3] = v[3];
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) s += x[c];
    s = group_sum<TPR>(s);
    const float mean = s / (float)kEmbed;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        float d = x[c] - mean;
        q += d * d;
    }
    q = group_sum<TPR>(q);
    const float var = q / (float)kEmbed;
    const float sd = sqrtf(var + 1e-5f);
    const float rstd = 1.0f / sd;
#pragma unroll
    for (int c = 0; c < CPT; c += 4) {
        f32x4 o, xn;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            xn[u] = (x[c + u] - mean) * rstd;
            o[u] = gamma[c0 + c + u] * xn[u] + beta[c0 + c + u];
        }
        *reinterpret_cast<f32x4*>(xr + c) = o;
        if (xn_out) *reinterpret_cast<f32x4*>(xn_out + row * kEmbed + c0 + c) = xn;
        if (x_out) *reinterpret_cast<f32x4*>(x_out + row * kEmbed + c0 + c) = o;
    }
    if (sd_out && part == 0) sd_out[row] = sd;
    __syncthreads();
}

// One residual block (model/mlp.metal:18-86 + model/elementwise.metal:4-13):
// h += relu(xs Up) Down, the hidden dimension in 128-wide chunks. xs holds
// LN(h). If v_out is given, the relu'd hidden activations are also written
// there ([M][hidden], row-major).
template <int M>
__device__ __forceinline__ void fwd_block(const mg_policy_view& pv, int l, FwdSmem<M>& sm, FwdRegs<M>& R,
                                          float* v_out = nullptr) {
    constexpr int RT = FwdRegs<M>::RT;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, n = lane & 31, hh = lane >> 5;
    const int H = (int)pv.hidden;
    const float* Up = pv.params + pv.off_up[l];
    const float* Dn = pv.params + pv.off_down[l];
    f32x16 o[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) o[rt] = f32x16{};
    for (int c = 0; c < H / kChunk; ++c) {
        f32x16 v[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) v[rt] = f32x16{};
        const float* bp = Up + (size_t)(4 * hh) * H + kChunk * c + 32 * w + n;
        const float* ap = sm.xs + n * kLds + 4 * hh;
#pragma unroll
        for (int g = 0; g < kEmbed / 8; ++g) {
            float b[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = bp[(size_t)(8 * g + j) * H];
            f32x4 a[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) a[rt] = *reinterpret_cast<const f32x4*>(ap + 32 * rt * kLds + 8 * g);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) v[rt] = mfma32x32x2(a[rt][j], b[j], v[rt]);
        }
        __syncthreads();  // every wave is done reading the previous chunk from vs
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 32 * rt + c32_row(r, lane);
                const float x = v[rt][r] > 0.0f ? v[rt][r] : 0.0f;
                sm.vs[row * kLds + 32 * w + n] = x;
                if (v_out) v_out[(size_t)row * H + kChunk * c + 32 * w + n] = x;
            }
        __syncthreads();
        const float* dp = Dn + (size_t)(kChunk * c + 4 * hh) * kEmbed + 32 * w + n;
        const float* vp = sm.vs + n * kLds + 4 * hh;
#pragma unroll
        for (int g = 0; g < kChunk / 8; ++g) {
            float b[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = dp[(size_t)(8 * g + j) * kEmbed];
            f32x4 a[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) a[rt] = *reinterpret_cast<const f32x4*>(vp + 32 * rt * kLds + 8 * g);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) o[rt] = mfma32x32x2(a[rt][j], b[j], o[rt]);
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) R.h[rt] = R.h[rt] + o[rt];
}

// model/linear.metal:17-37: head[row][j] = sum_k xs[row][k] W_head[k][j] for
// j < HD, into headL ([M][HD] in LDS). Ends with a barrier.
template <int M>
__device__ __forceinline__ void fwd_head(const mg_policy_view& pv, FwdSmem<M>& sm, float* headL, int HD) {
    constexpr int TPR = 256 / M, CPT = kEmbed / TPR;
    const int tid = threadIdx.x, row = tid / TPR, part = tid % TPR, c0 = part * CPT;
    const float* Wh = pv.params + pv.off_head + c0 * HD;
    const float* xr = sm.xs + row * kLds + c0;
    float x[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) x[c] = xr[c];
    for (int j = 0; j < HD; ++j) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < CPT; ++c) acc += x[c] * Wh[c * HD + j];
        acc = group_sum<TPR>(acc);
        if (part == 0) headL[row * HD + j] = acc;
    }
    __syncthreads();
}

// Whole forward: obs staged in obsL ([M][O], LDS) -> head in headL ([M][HD], LDS).
template <int M>
__device__ __forceinline__ void policy_forward(const mg_policy_view& pv, FwdSmem<M>& sm, FwdRegs<M>& R,
                                               const float* obsL, int O, float* headL, int HD) {
    fwd_embed<M>(pv, obsL, O, R);
    for (uint32_t l = 0; l < pv.layers; ++l) {
        fwd_layernorm<M>(sm, R, pv.params + pv.off_ln_gamma[l], pv.params + pv.off_ln_beta[l]);
        fwd_block<M>(pv, (int)l, sm, R);
    }
    fwd_layernorm<M>(sm, R, pv.params + pv.off_ln_gamma[pv.layers], pv.params + pv.off_ln_beta[pv.layers]);
    fwd_head<M>(pv, sm, headL, HD);
}

}  // namespace dev
}  // namespace mg
