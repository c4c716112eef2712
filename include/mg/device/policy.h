// Fused residual-MLP policy forward for a tile of M rows (M = 16, 32 or 64) on
// one workgroup of W waves (W = 4, or 8 for 16-row tiles), fp32 MFMA.
//
// Network (model/ppo.h:575-626): embed h = obs W_in + b_in; per block
// h += relu(LN(h) Up) Down; final LN; head = LN(h) W_head (no bias).
//
// Mapping: wave w owns the 128 / W embed columns [SW w, SW w + SW) of the
// residual stream h, held in MFMA accumulator layout. 32- and 64-row tiles use
// v_mfma_f32_32x32x2_f32; 16-row tiles use v_mfma_f32_16x16x4_f32, so a
// 4096-row minibatch still spreads over 256 workgroups. Each block runs the
// hidden dimension in 128-wide chunks so the hidden activations never leave
// the CU: V_c = relu(x Up[:, c]) is computed by all waves, staged in LDS, and
// immediately contracted with Down[c, :] into the residual stream. LN outputs
// and hidden chunks are the A operands (LDS, float4 reads); weights are the B
// operands, streamed from L2 into registers one GEMM ahead of their use (the
// whole 1 MB policy stays L2-resident across the grid).
//
// K-order permutation: with KS k-values per MFMA step, a k-group holds 4*KS
// k-values; lane (m, q) (q = lane / MT) reads x[m][g*4KS + 4q .. + 3] as one
// float4 and MFMA step j contracts k = g*4KS + 4q + j, so B supplies
// W[g*4KS + 4q + j][n]. Every k is covered once; only the fp32 summation order
// differs from a sequential loop.
#pragma once
#include "../bf16.h"
#include "common.h"

namespace mg {
namespace dev {

constexpr int kLds = kEmbed + 4;  // LDS row stride in floats (pad against bank conflicts)
constexpr int kChunk = 128;       // hidden columns per chunk
static_assert(kChunk == kEmbed, "every chunk GEMM contracts over 128");

// MFMA shape used by an M-row tile on W waves.
template <int M, int W = 4>
struct Shape {
    static constexpr int NT = 64 * W;             // threads
    static constexpr int SW = kEmbed / W;         // columns per wave
    static constexpr int MT = M >= 32 ? 32 : 16;  // MFMA M = N
    static constexpr int KS = MT == 32 ? 2 : 4;   // k per MFMA step
    static constexpr int KG = 4 * KS;             // k per float4 group
    static constexpr int RT = M / MT;             // row tiles
    static constexpr int CT = SW / MT;            // column tiles per wave
    static constexpr int REGS = MT == 32 ? 16 : 4;
    using Acc = typename std::conditional<MT == 32, f32x16, f32x4>::type;
    static_assert(M == 16 || M == 32 || M == 64, "tile rows");
    static_assert(W == 4 || W == 8, "waves");
    static_assert(SW % MT == 0, "a wave's strip holds whole MFMA tiles");

    __device__ static __forceinline__ Acc mfma(float a, float b, Acc c) {
        if constexpr (MT == 32)
            return mfma32x32x2(a, b, c);
        else
            return mfma16x16x4(a, b, c);
    }
    // Row (within the MT x MT tile) of accumulator register r of `lane`.
    __device__ static __forceinline__ int row(int r, int lane) {
        if constexpr (MT == 32)
            return c32_row(r, lane);
        else
            return c16_row(r, lane);
    }
    __device__ static __forceinline__ int col(int lane) { return lane % MT; }
    __device__ static __forceinline__ int quad(int lane) { return lane / MT; }
};

// NV = 2 double-buffers the hidden chunk: chunk c writes vs[c & 1], so the
// write never races the previous chunk's readers and one barrier per chunk
// suffices.
template <int M, int NV = 1>
struct FwdSmem {
    float xs[M * kLds];      // LN output (A operand of the up GEMM)
    float vs[NV][M * kLds];  // relu'd hidden chunk (A operand of the down GEMM)
};

// Residual stream of an M-row tile. Element (rt, ct, r) of wave w, lane l is
// row MT rt + Shape::row(r, l), column SW w + MT ct + l % MT.
template <int M, int W = 4>
struct FwdRegs {
    using S = Shape<M, W>;
    typename S::Acc h[S::RT][S::CT];
};

// A wave's accumulator tiles of an M-row tile.
template <int M, int W = 4>
using AccTile = typename Shape<M, W>::Acc[Shape<M, W>::RT][Shape<M, W>::CT];

template <int M, int W = 4>
__device__ __forceinline__ void zero(AccTile<M, W>& a) {
#pragma unroll
    for (int rt = 0; rt < Shape<M, W>::RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < Shape<M, W>::CT; ++ct) a[rt][ct] = typename Shape<M, W>::Acc{};
}

// Calls f(rt, ct, r, row, col) for every accumulator element this thread holds.
template <int M, int W = 4, class F>
__device__ __forceinline__ void for_each_elem(F f) {
    using S = Shape<M, W>;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < S::CT; ++ct)
#pragma unroll
            for (int r = 0; r < S::REGS; ++r)
                f(rt, ct, r, S::MT * rt + S::row(r, lane), S::SW * w + S::MT * ct + S::col(lane));
}

// B operand (weights) of NG k-groups of a 128-deep chunk GEMM for one wave's
// strip, held in registers.
template <int M, int W, int NG>
struct BFrag {
    float b[NG][Shape<M, W>::CT][4];
};

// Offset of element (n, k) of a matrix read as rows n of contraction length K
// (K a multiple of 128) in the fragment-tiled layout for MT x MT MFMA tiles
// (MT = 16: 16x16x4, KG = 16 k per float4 group; MT = 32: 32x32x2, KG = 8):
// strips of MT rows cut into MT x 128 tiles, tile (n / MT, k / 128) at
// (n / MT) MT K + (k / 128) MT 128, and inside a tile k-group g = k % 128 / KG
// at g 256 as 64 float4s in lane order, lane q MT + n % MT holding the four
// k = g KG + 4 q + j, q = k % KG / 4, j = k % 4. One k-group of one strip is
// then 1 KB of consecutive memory in exactly the lane layout of the B operand.
template <int MT>
__host__ __device__ constexpr uint32_t frag_index(uint32_t n, uint32_t k, uint32_t K) {
    constexpr uint32_t KG = MT == 32 ? 8u : 16u;
    return (n / MT) * MT * K + (k >> 7) * MT * 128u + ((k & 127u) / KG) * 256u + ((k % KG) >> 2) * MT * 4u +
           (n % MT) * 4u + (k & 3u);
}

// Where the s-th weight operand of a GEMM sequence lives: p is the first
// element of the fragment-tiled strip holding the chunk's first output column
// at the chunk's first k, ld the matrix's contraction length K.
struct FragSrc {
    const float* p;
    uint32_t ld;
};

// The first element of column tile ct of this wave's strip (wave-uniform:
// scalar registers).
template <int M, int W>
__device__ __forceinline__ const float* frag_strip(const FragSrc& f, int ct) {
    using S = Shape<M, W>;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    return f.p + (size_t)(wave * S::CT + ct) * S::MT * f.ld;
}

// This lane's float4 of k-group g of a strip: one 1 KB run per wave
// instruction, a buffer load with the run's offset in a scalar register and
// the per-lane 16 bytes as the only vector operand.
__device__ __forceinline__ f32x4 frag_load(const float* strip, int g) {
    return buffer_load16(strip, 16 * (threadIdx.x & 63), 1024 * g);
}

// Loads k-groups [g0, g0 + NG) of a fragment-tiled operand: one float4 per lane
// and k-group, as buffer loads (BUF) or global loads.
template <int M, int W, int NG, bool BUF = true>
__device__ __forceinline__ void load_frag(BFrag<M, W, NG>& f, const FragSrc& src, int g0) {
    using S = Shape<M, W>;
#pragma unroll
    for (int ct = 0; ct < S::CT; ++ct) {
        const float* strip = frag_strip<M, W>(src, ct);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const f32x4 v = BUF ? frag_load(strip, g0 + g)
                                : *reinterpret_cast<const f32x4*>(strip + 4 * (threadIdx.x & 63) + 256 * (g0 + g));
#pragma unroll
            for (int j = 0; j < 4; ++j) f.b[g][ct][j] = v[j];
        }
    }
}

// acc[rt][ct] += A[rows][k-groups g0 .. g0 + NG) @ B for this wave's strip. A
// is in LDS (row stride kLds, A[m][k] at a_lds[m * kLds + k]).
template <int M, int W, int NG>
__device__ __forceinline__ void gemm_frag(AccTile<M, W>& acc, const float* a_lds, const BFrag<M, W, NG>& f, int g0) {
    using S = Shape<M, W>;
    const int lane = threadIdx.x & 63, n = S::col(lane), q = S::quad(lane);
    const float* ap = a_lds + n * kLds + 4 * q + S::KG * g0;
    // the whole A operand first (one LDS latency per GEMM instead of one per
    // k-group pair), then the MFMAs back to back
    f32x4 a[NG][S::RT];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int rt = 0; rt < S::RT; ++rt)
            a[g][rt] = *reinterpret_cast<const f32x4*>(ap + S::MT * rt * kLds + S::KG * g);
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
                for (int ct = 0; ct < S::CT; ++ct) acc[rt][ct] = S::mfma(a[g][rt][j], f.b[g][ct][j], acc[rt][ct]);
}

// Register double buffer for a sequence of 128-deep chunk GEMMs of 32- and
// 64-row tiles (two workgroups per CU) whose weight operands are known in
// advance: the two halves of the current GEMM's fragment, each refilled with
// the next GEMM's half once consumed, so the loads' L2 latency overlaps the MFMA
// work (and the barriers) in between instead of stalling every k-group. BUF:
// buffer loads (load_frag).
template <int M, int W = 4, bool BUF = true>
struct WStream {
    static_assert(Shape<M, W>::MT == 32, "32x32x2 tiles");
    static constexpr int NG = kEmbed / Shape<M, W>::KG / 2;  // k-groups per half
    BFrag<M, W, NG> b[2];
    int total;  // GEMMs in the sequence

    // n >= 2 GEMMs (a block has two per chunk).
    template <class Src>
    __device__ __forceinline__ void start(int n, Src src) {
        total = n;
        const FragSrc f0 = src(0);
        load_frag<M, W, NG, BUF>(b[0], f0, 0);
        load_frag<M, W, NG, BUF>(b[1], f0, NG);
    }

    // acc += A @ W_s for the s-th GEMM of the sequence, then refills the
    // consumed registers with the next GEMM's operand.
    template <int ROLE, class Src>
    __device__ __forceinline__ void gemm(AccTile<M, W>& acc, const float* a_lds, int s, Src src) {
        const bool more = s + 1 < total;
        FragSrc f{nullptr, 0};
        if (more) f = src(s + 1);
        // raised wave priority while issuing MFMAs: the other workgroup on the
        // CU is then in its LN / head / env phase, whose VALU and LDS work
        // fills the gaps instead of delaying the MFMA issue (0.6% on the
        // 262144-env collect while the small parameters came from L2; no
        // measurable difference since they are staged in LDS)
        __builtin_amdgcn_s_setprio(1);
        gemm_frag<M, W, NG>(acc, a_lds, b[0], 0);
        if (more) load_frag<M, W, NG, BUF>(b[0], f, 0);
        gemm_frag<M, W, NG>(acc, a_lds, b[1], NG);
        if (more) load_frag<M, W, NG, BUF>(b[1], f, NG);
        __builtin_amdgcn_s_setprio(0);
    }
};

// Weight stream for 16-row tiles (registers to spare): two whole fragments,
// one per GEMM role, each refilled two GEMMs ahead one k-group at a time right
// after that k-group's MFMAs, so a wave's loads leave one at a time over the
// GEMM instead of as a burst after it. Past the end of the sequence a GEMM
// reloads its own operand: every path issues the same loads, so the compiler's
// vector-memory wait counts stay exact at the chunk loop's head.
template <int M, int W>
struct TStream {
    using S = Shape<M, W>;
    static_assert(S::MT == 16, "16x16x4 tiles");
    static constexpr int NGF = kEmbed / S::KG;  // k-groups of one 128-deep GEMM
    BFrag<M, W, NGF> b[2];
    int total;

    template <class Src>
    __device__ __forceinline__ void start(int n, Src src) {
        total = n;
        load_frag<M, W, NGF>(b[0], src(0), 0);
        load_frag<M, W, NGF>(b[1], src(1), 0);
    }

    template <int ROLE, class Src>
    __device__ __forceinline__ void gemm(AccTile<M, W>& acc, const float* a_lds, int s, Src src) {
        const int lane = threadIdx.x & 63, n = S::col(lane), q = S::quad(lane);
        const FragSrc f = src(s + 2 < total ? s + 2 : s);
        const float* ap = a_lds + n * kLds + 4 * q;
        f32x4 a[NGF][S::RT];
#pragma unroll
        for (int g = 0; g < NGF; ++g)
#pragma unroll
            for (int rt = 0; rt < S::RT; ++rt)
                a[g][rt] = *reinterpret_cast<const f32x4*>(ap + S::MT * rt * kLds + S::KG * g);
#pragma unroll
        for (int g = 0; g < NGF; ++g) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
                    for (int ct = 0; ct < S::CT; ++ct)
                        acc[rt][ct] = S::mfma(a[g][rt][j], b[ROLE].b[g][ct][j], acc[rt][ct]);
#pragma unroll
            for (int ct = 0; ct < S::CT; ++ct) {
                const f32x4 v = frag_load(frag_strip<M, W>(f, ct), g);
#pragma unroll
                for (int j = 0; j < 4; ++j) b[ROLE].b[g][ct][j] = v[j];
            }
            // keep the interleave: the scheduler would otherwise sink every
            // load to the end of the GEMM to shorten their live ranges
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// Writes a register tile to LDS (row stride kLds), optionally through relu.
template <int M, int W = 4, bool RELU = false>
__device__ __forceinline__ void store_tile(const AccTile<M, W>& acc, float* lds) {
    for_each_elem<M, W>([&](int rt, int ct, int r, int row, int col) {
        float x = acc[rt][ct][r];
        if (RELU) x = x > 0.0f ? x : 0.0f;
        lds[row * kLds + col] = x;
    });
}

// Writes a register tile to global memory (global[row * ld + col]),
// optionally through relu. Issued before a barrier, the stores leave while
// the wave would otherwise wait.
template <int M, int W = 4, bool RELU = false>
__device__ __forceinline__ void store_tile_g(const AccTile<M, W>& acc, float* global, size_t ld) {
    for_each_elem<M, W>([&](int rt, int ct, int r, int row, int col) {
        float x = acc[rt][ct][r];
        if (RELU) x = x > 0.0f ? x : 0.0f;
        global[(size_t)row * ld + col] = x;
    });
}

// model/input.metal:11-27: h = b_in + sum_k obs[k] W_in[k].
// obsL is [M][O] in LDS; Win ([O][128]) and bias ([128]) are in global memory
// or LDS. OC: O when known at compile time.
// 32- and 64-row tiles: the product on v_mfma_f32_32x32x2_f32 straight into
// the residual accumulators (A = obs rows, B = W_in columns, k = 2 s + lane /
// 32, zero past O). Per element and k a lane otherwise reads the row's
// observation float from LDS: 960 reads per lane for VoxelNav16's 30 floats,
// whose embed phase then took 111 K cycles of a 64-row collect step (and its
// LN0 130 K, waiting at the barrier for the slowest wave) against CartPole's
// 2.5 K and 34 K. 16-row tiles (8 elements or fewer per lane): in k order,
// the k loop unrolled when OC is known (a row's consecutive floats read
// together).
template <int M, int W = 4, int OC = 0>
__device__ __forceinline__ void fwd_embed(const float* Win, const float* bias, const float* obsL, int O,
                                          FwdRegs<M, W>& R) {
    for_each_elem<M, W>([&](int rt, int ct, int r, int row, int col) { R.h[rt][ct][r] = bias[col]; });
    using S = Shape<M, W>;
    if constexpr (S::MT == 32) {
        const int lane = threadIdx.x & 63, n = lane & 31, q = lane >> 5;
        const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const int On = OC > 0 ? OC : O;
        const int steps = (On + 1) / 2;
        constexpr int kUnroll = OC > 0 ? (OC + 1) / 2 : 1;
#pragma unroll kUnroll
        for (int st = 0; st < steps; ++st) {
            const int k = 2 * st + q;
            const bool in = k < On;
            const int kk = in ? k : 0;  // every read in bounds; the padding step's operands are zeroed
            float a[S::RT], b[S::CT];
#pragma unroll
            for (int rt = 0; rt < S::RT; ++rt) {
                const float v = obsL[(S::MT * rt + n) * On + kk];
                a[rt] = in ? v : 0.0f;
            }
#pragma unroll
            for (int ct = 0; ct < S::CT; ++ct) {
                const float v = Win[kk * kEmbed + S::SW * wave + S::MT * ct + n];
                b[ct] = in ? v : 0.0f;
            }
#pragma unroll
            for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
                for (int ct = 0; ct < S::CT; ++ct) R.h[rt][ct] = mfma32x32x2(a[rt], b[ct], R.h[rt][ct]);
        }
    } else if constexpr (OC > 0) {
#pragma unroll
        for (int k = 0; k < OC; ++k) {
            for_each_elem<M, W>([&](int rt, int ct, int r, int row, int col) {
                R.h[rt][ct][r] += obsL[row * OC + k] * Win[k * kEmbed + col];
            });
        }
    } else {
        for (int k = 0; k < O; ++k) {
            for_each_elem<M, W>([&](int rt, int ct, int r, int row, int col) {
                R.h[rt][ct][r] += obsL[row * O + k] * Win[k * kEmbed + col];
            });
        }
    }
}

// A thread's part of a row sum: a pairwise tree for 16 or more terms, else in
// order (see fwd_layernorm). Overwrites t.
template <int N>
__device__ __forceinline__ float row_sum(float (&t)[N]) {
    if constexpr (N >= 16) {
        return tree_sum(t);
    } else {
        float s = t[0];
#pragma unroll
        for (int c = 1; c < N; ++c) s += t[c];
        return s;
    }
}

template <int M, int W, int HDC>
__device__ __forceinline__ void fwd_head_regs(const float (&x)[kEmbed / (Shape<M, W>::NT / M)], const float* Wh,
                                              float* headL, int HD);

// model/layernorm.metal:10-71 on the register tile; the result goes to sm.xs.
// If xn_out/sd_out/x_out are given, the normalised values, the standard
// deviation and the output are also written there ([M][128], [M], [M][128],
// row-major; global memory or LDS) for the backward pass; if xb_out is given,
// the output rounded to bfloat16 goes there too ([M] rows of stride kLdsB).
// Smem is any shared-memory layout with an fp32 xs tile. HF >= 0: the final
// LN, followed by the head straight from the registers (fwd_head_regs with
// HDC = HF, head weights Wh, output headL, HD columns) instead of through xs
// and a barrier; xs then keeps the LN input.
constexpr int kLdsB = kEmbed + 8;  // LDS row stride of a bfloat16 tile (elements)
template <int M, int W = 4, class Smem, int HF = -1>
__device__ __forceinline__ void fwd_layernorm(Smem& sm, const FwdRegs<M, W>& R, const float* gamma,
                                              const float* beta, float* xn_out = nullptr, float* sd_out = nullptr,
                                              float* x_out = nullptr, uint16_t* xb_out = nullptr,
                                              const float* Wh = nullptr, float* headL = nullptr, int HD = 0) {
    constexpr int TPR = Shape<M, W>::NT / M;  // threads per row
    constexpr int CPT = kEmbed / TPR;         // columns per thread
    static_assert(CPT % 4 == 0, "float4 columns");
    const int tid = threadIdx.x;
    store_tile<M, W>(R.h, sm.xs);
    __syncthreads();
    const int row = tid / TPR, part = tid % TPR, c0 = part * CPT;
    float* xr = sm.xs + row * kLds + c0;
    float x[CPT];
#pragma unroll
    for (int c = 0; c < CPT; c += 4) {
        f32x4 v = *reinterpret_cast<const f32x4*>(xr + c);
        x[c] = v[0], x[c + 1] = v[1], x[c + 2] = v[2], x[c + 3] = v[3];
    }
    // a thread's sums as pairwise trees where it holds 16 or 32 columns (32-
    // and 64-row tiles), whose 31-add chains lengthened the LN phase (the
    // 262144-env collect 35.19 -> 34.90 ms); in column order at 4 columns (the
    // train kernels, whose bf16 mode rounds the LN output)
    float t[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) t[c] = x[c];
    const float s = group_sum<TPR>(row_sum(t));
    const float mean = s / (float)kEmbed;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const float d = x[c] - mean;
        t[c] = d * d;
    }
    const float q = group_sum<TPR>(row_sum(t));
    const float var = q / (float)kEmbed;
    const float sd = sqrtf(var + 1e-5f);
    const float rstd = 1.0f / sd;
    float oall[CPT];  // the output, for a fused head
#pragma unroll
    for (int c = 0; c < CPT; c += 4) {
        f32x4 o, xn;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            xn[u] = (x[c + u] - mean) * rstd;
            o[u] = gamma[c0 + c + u] * xn[u] + beta[c0 + c + u];
            oall[c + u] = o[u];
        }
        if constexpr (HF < 0) *reinterpret_cast<f32x4*>(xr + c) = o;
        if (xn_out) *reinterpret_cast<f32x4*>(xn_out + row * kEmbed + c0 + c) = xn;
        if (xb_out) {
            uint16_t hb[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) hb[u] = bf16_rne(o[u]);
            const uint32_t lo = (uint32_t)hb[0] | ((uint32_t)hb[1] << 16);
            const uint32_t hi = (uint32_t)hb[2] | ((uint32_t)hb[3] << 16);
            *reinterpret_cast<uint2*>(xb_out + row * kLdsB + c0 + c) = make_uint2(lo, hi);
        }
        if (x_out) {
            *reinterpret_cast<f32x4*>(x_out + row * kEmbed + c0 + c) = o;
        }
    }
    if (sd_out && part == 0) sd_out[row] = sd;
    if constexpr (HF >= 0) {
        fwd_head_regs<M, W, HF>(oall, Wh, headL, HD);  // ends with a barrier
    } else {
        __syncthreads();
    }
}

// The forward's GEMM sequence: for block l and chunk c, GEMM 2 (l NC + c)
// is V_c = xs Up[:, c] (weights Up^T rows c, [H][128]) and the next one is
// h += V_c Down[c, :] (weights Down^T columns c, [128][H]), read from the
// fragment-tiled transposed copies for MT x MT tiles (frag_fwd32 or
// frag_fwd16): Up^T's chunk c (K = 128) starts at row 128 c, Down^T's chunk c
// (K = H) at tile column c.
template <int MT>
struct FwdSeq {
    const mg_policy_view* pv;
    int nc;
    __device__ __forceinline__ FragSrc operator()(int s) const {
        const int l = s / (2 * nc), c = (s >> 1) % nc;
        const float* base = MT == 32 ? pv->frag_fwd32 : pv->frag_fwd16;
        if ((s & 1) == 0) return {base + pv->off_up[l] + (size_t)kChunk * c * kEmbed, (uint32_t)kEmbed};
        return {base + pv->off_down[l] + MT * kChunk * c, pv->hidden};
    }
};

// One residual block (model/mlp.metal:18-86 + model/elementwise.metal:4-13):
// h += relu(xs Up) Down, the hidden dimension in 128-wide chunks whose Down
// products accumulate straight into the residual stream (the residual add
// folded into the GEMM accumulator). xs holds LN(h); ws streams a sequence
// whose first 2 L NC GEMMs are the forward's (FwdSeq, or a longer sequence
// that continues past the forward). With VOUT the relu'd hidden activations
// are also written to v_out ([M][hidden], row-major).
template <int M, int W, bool VOUT, int NV, class Seq, class Stream>
__device__ __forceinline__ void fwd_block(const mg_policy_view& pv, int l, FwdSmem<M, NV>& sm, FwdRegs<M, W>& R,
                                          Stream& ws, float* v_out, Seq seq) {
    using S = Shape<M, W>;
    const int H = (int)pv.hidden, NC = H / kChunk;
    for (int c = 0; c < NC; ++c) {
        const int s = 2 * (l * NC + c);
        float* vs = sm.vs[NV == 2 ? (c & 1) : 0];
        typename S::Acc v[S::RT][S::CT];
        zero<M, W>(v);
        ws.template gemm<0>(v, sm.xs, s, seq);
        if constexpr (VOUT) store_tile_g<M, W, true>(v, v_out + kChunk * c, H);
        if constexpr (NV == 1) __syncthreads();  // every wave is done reading the previous chunk from vs
        store_tile<M, W, true>(v, vs);
        __syncthreads();
        ws.template gemm<1>(R.h, vs, s + 1, seq);
    }
}

// model/linear.metal:17-37: head[row][j] = sum_k x[row][k] W_head[k][j] for
// j < HD, into headL ([M][HD] in LDS). Wh is W_head ([128][HD], global memory
// or LDS). Ends with a barrier.
// HDC: the head width when known at compile time (0: runtime HD only). Then a
// thread's block of W_head is read as float4s, G columns at a time (24 loads
// instead of 96 at 64-row tiles of a 3-column head: the 262144-env collect
// 34.70 -> 34.19 ms).
// fwd_head_regs: x is this thread's CPT columns of its row (the LayerNorm's
// thread layout, TPR threads per row).
template <int M, int W, int HDC>
__device__ __forceinline__ void fwd_head_regs(const float (&x)[kEmbed / (Shape<M, W>::NT / M)], const float* Wh,
                                              float* headL, int HD) {
    constexpr int TPR = Shape<M, W>::NT / M, CPT = kEmbed / TPR;
    const int tid = threadIdx.x, row = tid / TPR, part = tid % TPR, c0 = part * CPT;
    const float* wp = Wh + c0 * HD;
    // G columns at a time: the largest power of two whose G x HDC weights fit
    // 96 registers and start 16-byte aligned; heads of up to 4 columns only
    // (wider ones made VoxelNav16's collect spill)
    constexpr int G = HDC <= 0 ? 0 : (CPT * HDC <= 96 ? CPT : (CPT / 2) * HDC <= 96 ? CPT / 2 : CPT / 4);
    if constexpr (HDC > 0 && HDC <= 4 && G * HDC <= 96 && (G * HDC) % 4 == 0 && G >= 4) {
        float acc[HDC];
#pragma unroll
        for (int g0 = 0; g0 < CPT; g0 += G) {
            float w[G * HDC];  // W_head[c0 + g0 + c][j] at w[c HDC + j]
#pragma unroll
            for (int q = 0; q < G * HDC; q += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(wp + g0 * HDC + q);
                w[q] = v[0], w[q + 1] = v[1], w[q + 2] = v[2], w[q + 3] = v[3];
            }
#pragma unroll
            for (int j = 0; j < HDC; ++j) {
                float t[G];
#pragma unroll
                for (int c = 0; c < G; ++c) t[c] = x[g0 + c] * w[c * HDC + j];
                const float part_sum = row_sum(t);
                acc[j] = g0 == 0 ? part_sum : acc[j] + part_sum;
            }
        }
#pragma unroll
        for (int j = 0; j < HDC; ++j) {
            const float v = group_sum<TPR>(acc[j]);
            if (part == 0) headL[row * HDC + j] = v;
        }
        __syncthreads();
        return;
    }
    for (int j = 0; j < HD; ++j) {
        float t[CPT];
#pragma unroll
        for (int c = 0; c < CPT; ++c) t[c] = x[c] * wp[c * HD + j];
        const float acc = group_sum<TPR>(row_sum(t));
        if (part == 0) headL[row * HD + j] = acc;
    }
    __syncthreads();
}


// The head from the LN output in sm.xs (x = xs rows).
template <int M, int W = 4, int HDC = 0, class Smem>
__device__ __forceinline__ void fwd_head(const float* Wh, Smem& sm, float* headL, int HD) {
    constexpr int TPR = Shape<M, W>::NT / M, CPT = kEmbed / TPR;
    const int tid = threadIdx.x, row = tid / TPR, part = tid % TPR, c0 = part * CPT;
    const float* xr = sm.xs + row * kLds + c0;
    float x[CPT];
    static_assert(CPT % 4 == 0, "float4 columns");
#pragma unroll
    for (int c = 0; c < CPT; c += 4) {  // float4 reads: no bank conflicts between lanes
        const f32x4 v = *reinterpret_cast<const f32x4*>(xr + c);
        x[c] = v[0], x[c + 1] = v[1], x[c + 2] = v[2], x[c + 3] = v[3];
    }
    fwd_head_regs<M, W, HDC>(x, Wh, headL, HD);
}

// Where a forward reads its small parameters: W_in [O][128], b_in, the LN
// parameters (LN l: gamma at ln + 256 l, beta at ln + 256 l + 128; the arena
// keeps them contiguous) and W_head [128][HD]; the arena itself, or copies in
// LDS.
struct SmallParams {
    const float* win;
    const float* bin;
    const float* ln;
    const float* wh;
};
__device__ __forceinline__ SmallParams small_params(const mg_policy_view& pv) {
    return {pv.params + pv.off_in_w, pv.params + pv.off_in_b, pv.params + pv.off_ln_gamma[0],
            pv.params + pv.off_head};
}

// Whole forward: obs staged in obsL ([M][O], LDS) -> head in headL ([M][HD], LDS).
// 16-row tiles stream whole fragments (TStream), taller tiles half-fragments
// (WStream; BUF: with buffer loads). HDC, OC: HD and O when known at compile
// time.
template <int M, int W = 4, bool BUF = true, int HDC = 0, int OC = 0>
__device__ __forceinline__ void policy_forward(const mg_policy_view& pv, const SmallParams& sp, FwdSmem<M>& sm,
                                               FwdRegs<M, W>& R, const float* obsL, int O, float* headL, int HD) {
    using Stream = typename std::conditional<M == 16, TStream<M, W>, WStream<M, W, BUF>>::type;
    using Seq = FwdSeq<Shape<M, W>::MT>;
    const int NC = (int)pv.hidden / kChunk;
    const Seq seq{&pv, NC};
    Stream ws;
    // the embed first: its parameter reads (from global memory where the
    // small parameters are not staged in LDS) then do not wait behind the
    // weight stream's first loads (VoxelNav at 262144 envs: 66.0 -> 63.0 ms)
    fwd_embed<M, W, OC>(sp.win, sp.bin, obsL, O, R);
    ws.start(2 * (int)pv.layers * NC, seq);
    for (uint32_t l = 0; l < pv.layers; ++l) {
        const float* g = sp.ln + 2 * kEmbed * l;
        fwd_layernorm<M, W>(sm, R, g, g + kEmbed);
        fwd_block<M, W, false, 1, Seq>(pv, (int)l, sm, R, ws, nullptr, seq);
    }
    const float* g = sp.ln + 2 * kEmbed * pv.layers;
    fwd_layernorm<M, W, FwdSmem<M>, HDC>(sm, R, g, g + kEmbed, nullptr, nullptr, nullptr, nullptr, sp.wh, headL, HD);
}

}  // namespace dev
}  // namespace mg
