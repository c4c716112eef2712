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

// Loads k-groups [g0, g0 + NG) of a transposed weight operand: W^T element
// (k, n) at wt_ptr[n * wt_ld + k], so each lane's four k-values are one
// contiguous float4.
template <int M, int W, int NG>
__device__ __forceinline__ void load_frag_t(BFrag<M, W, NG>& f, const float* wt_ptr, size_t wt_ld, int g0) {
    using S = Shape<M, W>;
    const int lane = threadIdx.x & 63, n = S::col(lane), q = S::quad(lane), n0 = S::SW * (threadIdx.x >> 6);
    const float* bp = wt_ptr + (size_t)(n0 + n) * wt_ld + 4 * q + S::KG * g0;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int ct = 0; ct < S::CT; ++ct) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(bp + (size_t)(S::MT * ct) * wt_ld + S::KG * g);
#pragma unroll
            for (int j = 0; j < 4; ++j) f.b[g][ct][j] = v[j];
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

// gemm_frag fused with the refill of the same registers: k-group g's weights
// are replaced by k-group g of `next` as soon as its MFMAs have issued, so a
// wave's refill loads leave one at a time over the GEMM instead of as a burst
// after it (a burst from every wave of the CU backs up the CU's vector-memory
// address path and stalls the issuing waves).
template <int M, int W, int NG>
__device__ __forceinline__ void gemm_frag_refill(AccTile<M, W>& acc, const float* a_lds, BFrag<M, W, NG>& f,
                                                 const float* next_p, size_t next_ld, int g0) {
    using S = Shape<M, W>;
    const int lane = threadIdx.x & 63, n = S::col(lane), q = S::quad(lane), n0 = S::SW * (threadIdx.x >> 6);
    const float* ap = a_lds + n * kLds + 4 * q + S::KG * g0;
    const float* bp = next_p + (size_t)(n0 + n) * next_ld + 4 * q + S::KG * g0;
    f32x4 a[NG][S::RT];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int rt = 0; rt < S::RT; ++rt)
            a[g][rt] = *reinterpret_cast<const f32x4*>(ap + S::MT * rt * kLds + S::KG * g);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
                for (int ct = 0; ct < S::CT; ++ct) acc[rt][ct] = S::mfma(a[g][rt][j], f.b[g][ct][j], acc[rt][ct]);
#pragma unroll
        for (int ct = 0; ct < S::CT; ++ct) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(bp + (size_t)(S::MT * ct) * next_ld + S::KG * g);
#pragma unroll
            for (int j = 0; j < 4; ++j) f.b[g][ct][j] = v[j];
        }
        // keep the interleave: the scheduler would otherwise sink every load
        // to the end of the GEMM to shorten their live ranges
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Where the s-th weight operand of a GEMM sequence lives (transposed layout).
struct FragSrc {
    const float* p;
    uint32_t ld;
};

// Register double buffer for a sequence of 128-deep chunk GEMMs whose weight
// operands are known in advance (a forward or backward pass). The loads of a
// later GEMM's weights are issued as soon as registers free up, so their L2
// latency overlaps the MFMA work (and the barriers) in between instead of
// stalling every k-group. With whole fragments every GEMM issues the same
// loads on every path (past the end of the sequence it reloads its own
// operand): the compiler's vector-memory wait counts are then exact at the
// chunk loop's head instead of the conservative merge of paths with different
// numbers of loads in flight.
//  - 16-row tiles (registers to spare): two whole fragments, one per GEMM
//    role, each refilled two GEMMs ahead.
//  - 32/64-row tiles (two workgroups per CU): the two halves of the current
//    GEMM's fragment, each refilled with the next GEMM's half once consumed.
template <int M, int W = 4>
struct WStream {
    static constexpr int NGF = kEmbed / Shape<M, W>::KG;  // k-groups of one 128-deep GEMM
    static constexpr bool WHOLE = M == 16;
    static constexpr int NG = WHOLE ? NGF : NGF / 2;
    BFrag<M, W, NG> b[2];
    int total;  // GEMMs in the sequence

    // n >= 2 GEMMs (a block has two per chunk).
    template <class Src>
    __device__ __forceinline__ void start(int n, Src src) {
        total = n;
        const FragSrc f0 = src(0);
        if constexpr (WHOLE) {
            const FragSrc f1 = src(1);
            load_frag_t<M, W, NG>(b[0], f0.p, f0.ld, 0);
            load_frag_t<M, W, NG>(b[1], f1.p, f1.ld, 0);
        } else {
            load_frag_t<M, W, NG>(b[0], f0.p, f0.ld, 0);
            load_frag_t<M, W, NG>(b[1], f0.p, f0.ld, NG);
        }
    }

    // acc += A @ W_s for the s-th GEMM of the sequence (ROLE = s & 1), then
    // refills the consumed registers.
    template <int ROLE, class Src>
    __device__ __forceinline__ void gemm(AccTile<M, W>& acc, const float* a_lds, int s, Src src) {
        if constexpr (WHOLE) {
            const FragSrc f = src(s + 2 < total ? s + 2 : s);
            gemm_frag_refill<M, W, NG>(acc, a_lds, b[ROLE], f.p, f.ld, 0);
        } else {
            const bool more = s + 1 < total;
            FragSrc f{nullptr, 0};
            if (more) f = src(s + 1);
            gemm_frag<M, W, NG>(acc, a_lds, b[0], 0);
            if (more) load_frag_t<M, W, NG>(b[0], f.p, f.ld, 0);
            gemm_frag<M, W, NG>(acc, a_lds, b[1], NG);
            if (more) load_frag_t<M, W, NG>(b[1], f.p, f.ld, NG);
        }
    }
};

// Weight stream for 16-row tiles that stages each GEMM's weights through a
// private LDS scratch of the wave. The MFMA operand layout puts 16 different
// weight rows (64 B each) in one float4 load, 16 L1 requests per KB; here each
// load instruction covers two whole 512-byte rows (8 cache lines per KB), the
// rows go to the wave's scratch XOR-swizzled (slot r * 32 + (c ^ (r & 7)) for
// row r, 16-byte chunk c), and the GEMM reads them back in MFMA layout without
// bank conflicts. Only the owning wave touches its scratch, so no barrier is
// needed: a wave's LDS operations complete in order. Each GEMM writes its
// weights to the scratch first, then issues the loads of the GEMM two ahead,
// one per k-group between the MFMAs. (Writing the next GEMM's weights in the
// middle of this one measured slower: that write waits for loads issued only
// one GEMM earlier and stalls the MFMAs behind it.) Same interface as WStream.
template <int M, int W>
struct LStream {
    using S = Shape<M, W>;
    static_assert(S::MT == 16 && S::SW % 2 == 0, "16x16x4 tiles, two rows per load");
    static constexpr int NI = S::SW / 2;        // raw float4 loads per lane per GEMM
    static constexpr int NGF = kEmbed / S::KG;  // k-groups of one 128-deep GEMM
    static_assert(NI <= NGF, "one refill load per k-group at most");
    f32x4 raw[2][NI];
    float* scr;  // this wave's scratch: SW rows x 128 floats
    int total;

    __device__ __forceinline__ void load_raw(int role, const FragSrc& f, int i) {
        const int lane = threadIdx.x & 63, n0 = S::SW * (threadIdx.x >> 6);
        raw[role][i] = *reinterpret_cast<const f32x4*>(f.p + (size_t)(n0 + 2 * i + (lane >> 5)) * f.ld +
                                                       4 * (lane & 31));
    }
    static __device__ __forceinline__ int slot(int r, int c) { return r * 32 + (c ^ (r & 7)); }
    __device__ __forceinline__ void write_scratch(int role) {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int r = 2 * i + (lane >> 5);
            *reinterpret_cast<f32x4*>(scr + 4 * slot(r, lane & 31)) = raw[role][i];
        }
    }

    // n >= 2 GEMMs; scratch = SW * 128 floats of LDS owned by this wave.
    template <class Src>
    __device__ __forceinline__ void start(int n, Src src, float* scratch) {
        total = n;
        scr = scratch;
        const FragSrc f0 = src(0), f1 = src(1);
#pragma unroll
        for (int i = 0; i < NI; ++i) load_raw(0, f0, i);
#pragma unroll
        for (int i = 0; i < NI; ++i) load_raw(1, f1, i);
    }

    template <int ROLE, class Src>
    __device__ __forceinline__ void gemm(AccTile<M, W>& acc, const float* a_lds, int s, Src src) {
        const int lane = threadIdx.x & 63, n = S::col(lane), q = S::quad(lane);
        write_scratch(ROLE);
        const FragSrc f = src(s + 2 < total ? s + 2 : s);
        const float* ap = a_lds + n * kLds + 4 * q;
        f32x4 a[NGF][S::RT];
#pragma unroll
        for (int g = 0; g < NGF; ++g)
#pragma unroll
            for (int rt = 0; rt < S::RT; ++rt)
                a[g][rt] = *reinterpret_cast<const f32x4*>(ap + S::MT * rt * kLds + S::KG * g);
        f32x4 b[NGF][S::CT];
#pragma unroll
        for (int g = 0; g < NGF; ++g)
#pragma unroll
            for (int ct = 0; ct < S::CT; ++ct)
                b[g][ct] = *reinterpret_cast<const f32x4*>(scr + 4 * slot(n + S::MT * ct, 4 * g + q));
#pragma unroll
        for (int g = 0; g < NGF; ++g) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
                    for (int ct = 0; ct < S::CT; ++ct) acc[rt][ct] = S::mfma(a[g][rt][j], b[g][ct][j], acc[rt][ct]);
            if (g < NI) load_raw(ROLE, f, g);
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

// Copies an LDS tile ([M][128], row stride kLds) to global memory
// (global[row * ld + col]) as float4 rows, NT threads.
template <int M, int NT>
__device__ __forceinline__ void copy_rows_g(const float* lds, float* global, size_t ld) {
#pragma unroll
    for (int i = threadIdx.x; i < M * kEmbed / 4; i += NT) {
        const int row = i / (kEmbed / 4), c4 = 4 * (i % (kEmbed / 4));
        *reinterpret_cast<f32x4*>(global + (size_t)row * ld + c4) =
            *reinterpret_cast<const f32x4*>(lds + row * kLds + c4);
    }
}

// model/input.metal:11-27: h = b_in + sum_k obs[k] W_in[k], in k order.
// obsL is [M][O] in LDS.
template <int M, int W = 4>
__device__ __forceinline__ void fwd_embed(const mg_policy_view& pv, const float* obsL, int O, FwdRegs<M, W>& R) {
    const float* Win = pv.params + pv.off_in_w;
    const float* bias = pv.params + pv.off_in_b;
    for_each_elem<M, W>([&](int rt, int ct, int r, int row, int col) { R.h[rt][ct][r] = bias[col]; });
    for (int k = 0; k < O; ++k) {
        for_each_elem<M, W>([&](int rt, int ct, int r, int row, int col) {
            R.h[rt][ct][r] += obsL[row * O + k] * Win[k * kEmbed + col];
        });
    }
}

// model/layernorm.metal:10-71 on the register tile; the result goes to sm.xs.
// If xn_out/sd_out/x_out are given, the normalised values, the standard
// deviation and the output are also written there ([M][128], [M], [M][128],
// row-major; global memory or LDS) for the backward pass.
template <int M, int W = 4, int NV = 1>
__device__ __forceinline__ void fwd_layernorm(FwdSmem<M, NV>& sm, const FwdRegs<M, W>& R, const float* gamma,
                                              const float* beta, float* xn_out = nullptr, float* sd_out = nullptr,
                                              float* x_out = nullptr) {
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

// The forward's GEMM sequence: for block l and chunk c, GEMM 2 (l NC + c)
// is V_c = xs Up[:, c] (weights Up^T rows c, [H][128]) and the next one is
// h += V_c Down[c, :] (weights Down^T columns c, [128][H]); both from the
// transposed copies in params_t.
struct FwdSeq {
    const mg_policy_view* pv;
    int nc;
    __device__ __forceinline__ FragSrc operator()(int s) const {
        const int l = s / (2 * nc), c = (s >> 1) % nc;
        if ((s & 1) == 0) return {pv->params_t + pv->off_up[l] + (size_t)kChunk * c * kEmbed, (uint32_t)kEmbed};
        return {pv->params_t + pv->off_down[l] + kChunk * c, pv->hidden};
    }
};

// One residual block (model/mlp.metal:18-86 + model/elementwise.metal:4-13):
// h += relu(xs Up) Down, the hidden dimension in 128-wide chunks whose Down
// products accumulate straight into the residual stream (the residual add
// folded into the GEMM accumulator). xs holds LN(h); ws streams a sequence
// whose first 2 L NC GEMMs are the forward's (FwdSeq, or a longer sequence
// that continues past the forward). With VOUT the relu'd hidden activations
// are also written to v_out ([M][hidden], row-major).
template <int M, int W = 4, bool VOUT = false, int NV = 1, class Seq = FwdSeq, class Stream = WStream<M, W>>
__device__ __forceinline__ void fwd_block(const mg_policy_view& pv, int l, FwdSmem<M, NV>& sm, FwdRegs<M, W>& R,
                                          Stream& ws, float* v_out = nullptr, Seq seq = Seq{}) {
    using S = Shape<M, W>;
    const int H = (int)pv.hidden, NC = H / kChunk;
    if constexpr (std::is_same<Seq, FwdSeq>::value) seq = FwdSeq{&pv, NC};
    for (int c = 0; c < NC; ++c) {
        const int s = 2 * (l * NC + c);
        float* vs = sm.vs[NV == 2 ? (c & 1) : 0];
        typename S::Acc v[S::RT][S::CT];
        zero<M, W>(v);
        ws.template gemm<0>(v, sm.xs, s, seq);
        if constexpr (NV == 1) __syncthreads();  // every wave is done reading the previous chunk from vs
        store_tile<M, W, true>(v, vs);
        __syncthreads();
        if constexpr (VOUT) copy_rows_g<M, S::NT>(vs, v_out + kChunk * c, H);
        ws.template gemm<1>(R.h, vs, s + 1, seq);
    }
}

// model/linear.metal:17-37: head[row][j] = sum_k xs[row][k] W_head[k][j] for
// j < HD, into headL ([M][HD] in LDS). Wh is W_head ([128][HD], global memory
// or LDS). Ends with a barrier.
template <int M, int W = 4, int NV = 1>
__device__ __forceinline__ void fwd_head(const float* Wh, FwdSmem<M, NV>& sm, float* headL, int HD) {
    constexpr int TPR = Shape<M, W>::NT / M, CPT = kEmbed / TPR;
    const int tid = threadIdx.x, row = tid / TPR, part = tid % TPR, c0 = part * CPT;
    const float* wp = Wh + c0 * HD;
    const float* xr = sm.xs + row * kLds + c0;
    float x[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) x[c] = xr[c];
    for (int j = 0; j < HD; ++j) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < CPT; ++c) acc += x[c] * wp[c * HD + j];
        acc = group_sum<TPR>(acc);
        if (part == 0) headL[row * HD + j] = acc;
    }
    __syncthreads();
}

// Whole forward: obs staged in obsL ([M][O], LDS) -> head in headL ([M][HD], LDS).
// With STAGE (16-row tiles) the weights go through the per-wave LDS scratch of
// LStream (W * SW * 128 floats at wscr); otherwise they stream into registers.
template <int M, int W = 4, bool STAGE = false>
__device__ __forceinline__ void policy_forward(const mg_policy_view& pv, FwdSmem<M>& sm, FwdRegs<M, W>& R,
                                               const float* obsL, int O, float* headL, int HD,
                                               float* wscr = nullptr) {
    using Stream = typename std::conditional<STAGE, LStream<M, W>, WStream<M, W>>::type;
    Stream ws;
    const int NC = (int)pv.hidden / kChunk;
    if constexpr (STAGE)
        ws.start(2 * (int)pv.layers * NC, FwdSeq{&pv, NC}, wscr + (threadIdx.x >> 6) * Shape<M, W>::SW * kEmbed);
    else
        ws.start(2 * (int)pv.layers * NC, FwdSeq{&pv, NC});
    fwd_embed<M, W>(pv, obsL, O, R);
    for (uint32_t l = 0; l < pv.layers; ++l) {
        fwd_layernorm<M, W>(sm, R, pv.params + pv.off_ln_gamma[l], pv.params + pv.off_ln_beta[l]);
        fwd_block<M, W>(pv, (int)l, sm, R, ws);
    }
    fwd_layernorm<M, W>(sm, R, pv.params + pv.off_ln_gamma[pv.layers], pv.params + pv.off_ln_beta[pv.layers]);
    fwd_head<M, W>(pv.params + pv.off_head, sm, headL, HD);
}

}  // namespace dev
}  // namespace mg
