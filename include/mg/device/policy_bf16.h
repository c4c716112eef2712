// The policy forward with bfloat16 matrix operands and fp32 accumulation (the
// precision of the reference's matmuls: model/mlp.metal multiplies bfloat16
// tiles with MetalPerformancePrimitives into fp32 accumulators).
//
// Same tiling and data flow as the fp32 forward (policy.h): the residual
// stream, LN statistics, the final LN and the head stay fp32; the two block
// GEMMs take bf16 operands. The LN output feeding the up GEMM and the relu'd
// hidden chunk feeding the down GEMM are rounded to bf16 (round to nearest
// even) as they are written to LDS; the weights come from bf16 copies of the
// block matrices in the same fragment-tiled order as the fp32 copies, one
// 16-byte run of 8 bf16 per lane and k-group. 32- and 64-row tiles use
// v_mfma_f32_32x32x16_bf16 (16 k per instruction), 16-row tiles
// v_mfma_f32_16x16x32_bf16 (32 k). In both, lane (m, q) (q = lane / MT)
// supplies the 8 k values 8 q .. 8 q + 7 of its k-group for its row m of A
// and its column m of B, so A and B agree on every k.
#pragma once
#include "policy.h"

namespace mg {
namespace dev {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int M, int W = 4>
struct ShapeB {
    using S = Shape<M, W>;
    static constexpr int KB = S::MT == 32 ? 16 : 32;  // k per MFMA
    static constexpr int NGB = kEmbed / KB;           // MFMAs (k-groups) per 128-deep GEMM
    static constexpr int GROUP = S::MT * KB;          // bf16 elements of one k-group of one strip
    static_assert(GROUP == 512, "one k-group of one strip is 1 KB");
    __device__ static __forceinline__ typename S::Acc mfma(u32x4 a, u32x4 b, typename S::Acc c) {
        const bf16x8 av = __builtin_bit_cast(bf16x8, a), bv = __builtin_bit_cast(bf16x8, b);
        if constexpr (S::MT == 32)
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
    }
};

// Element (n, k) of a matrix read as rows n of contraction length K in the
// bf16 fragment-tiled layout for MT x MT tiles: strips of MT rows, MT x 128
// tiles, and inside a tile k-group g = k % 128 / KB as 64 lanes of 8
// consecutive k, lane q MT + n % MT holding k = g KB + 8 q .. + 7.
template <int MT>
__host__ __device__ constexpr uint32_t frag_index_b(uint32_t n, uint32_t k, uint32_t K) {
    constexpr uint32_t KB = MT == 32 ? 16u : 32u;
    return (n / MT) * MT * K + (k >> 7) * MT * 128u + ((k & 127u) / KB) * (MT * KB) + ((k % KB) >> 3) * MT * 8u +
           (n % MT) * 8u + (k & 7u);
}

// LDS of one forward tile: the fp32 LN output (staging, and the head's input
// after the final LN) and the bf16 GEMM operands; NV = 2 double-buffers the
// hidden chunk (one barrier per chunk).
template <int M, int NV = 1>
struct FwdSmemB {
    float xs[M * kLds];
    uint16_t xb[M * kLdsB];      // LN output of the block's input, bf16
    uint16_t vb[NV][M * kLdsB];  // relu'd hidden chunk, bf16
};

struct FragSrcB {
    const uint16_t* p;
    uint32_t ld;  // contraction length K of the matrix
};

template <int M, int W, int NG>
struct BFragB {
    u32x4 b[NG][Shape<M, W>::CT];
};

template <int M, int W>
__device__ __forceinline__ const uint16_t* frag_lane_b(const FragSrcB& f, int ct) {
    using S = Shape<M, W>;
    const uint32_t lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    return f.p + (size_t)(wave * S::CT + ct) * S::MT * f.ld + 8 * lane;
}

template <int M, int W, int NG>
__device__ __forceinline__ void load_frag_b(BFragB<M, W, NG>& f, const FragSrcB& src, int g0) {
    using S = Shape<M, W>;
#pragma unroll
    for (int ct = 0; ct < S::CT; ++ct) {
        const uint16_t* bp = frag_lane_b<M, W>(src, ct) + ShapeB<M, W>::GROUP * g0;
#pragma unroll
        for (int g = 0; g < NG; ++g) f.b[g][ct] = *reinterpret_cast<const u32x4*>(bp + ShapeB<M, W>::GROUP * g);
    }
}

// acc += A[rows][k-groups g0 .. g0 + NG) @ B; A is a bf16 LDS tile (row stride kLdsB).
template <int M, int W, int NG>
__device__ __forceinline__ void gemm_frag_b(AccTile<M, W>& acc, const uint16_t* a_lds, const BFragB<M, W, NG>& f,
                                            int g0) {
    using S = Shape<M, W>;
    using SB = ShapeB<M, W>;
    const int lane = threadIdx.x & 63, n = S::col(lane), q = S::quad(lane);
    const uint16_t* ap = a_lds + n * kLdsB + 8 * q + SB::KB * g0;
    u32x4 a[NG][S::RT];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int rt = 0; rt < S::RT; ++rt)
            a[g][rt] = *reinterpret_cast<const u32x4*>(ap + S::MT * rt * kLdsB + SB::KB * g);
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < S::CT; ++ct) acc[rt][ct] = SB::mfma(a[g][rt], f.b[g][ct], acc[rt][ct]);
}

// Weight streams over the bf16 copies, the counterparts of WStream (32/64-row
// tiles: the two halves of the current GEMM's fragment, each refilled with the
// next GEMM's half once consumed) and TStream (16-row tiles: two whole
// fragments, one per GEMM role, refilled two GEMMs ahead).
template <int M, int W = 4>
struct WStreamB {
    static_assert(Shape<M, W>::MT == 32, "32x32x16 tiles");
    static constexpr int NG = ShapeB<M, W>::NGB / 2;
    BFragB<M, W, NG> b[2];
    int total;

    template <class Src>
    __device__ __forceinline__ void start(int n, Src src) {
        total = n;
        const FragSrcB f0 = src(0);
        load_frag_b<M, W, NG>(b[0], f0, 0);
        load_frag_b<M, W, NG>(b[1], f0, NG);
    }

    template <int ROLE, class Src>
    __device__ __forceinline__ void gemm(AccTile<M, W>& acc, const uint16_t* a_lds, int s, Src src) {
        const bool more = s + 1 < total;
        FragSrcB f{nullptr, 0};
        if (more) f = src(s + 1);
        gemm_frag_b<M, W, NG>(acc, a_lds, b[0], 0);
        if (more) load_frag_b<M, W, NG>(b[0], f, 0);
        gemm_frag_b<M, W, NG>(acc, a_lds, b[1], NG);
        if (more) load_frag_b<M, W, NG>(b[1], f, NG);
    }
};

template <int M, int W>
struct TStreamB {
    using S = Shape<M, W>;
    static_assert(S::MT == 16, "16x16x32 tiles");
    static constexpr int NGF = ShapeB<M, W>::NGB;
    BFragB<M, W, NGF> b[2];
    int total;

    template <class Src>
    __device__ __forceinline__ void start(int n, Src src) {
        total = n;
        load_frag_b<M, W, NGF>(b[0], src(0), 0);
        load_frag_b<M, W, NGF>(b[1], src(1), 0);
    }

    template <int ROLE, class Src>
    __device__ __forceinline__ void gemm(AccTile<M, W>& acc, const uint16_t* a_lds, int s, Src src) {
        using SB = ShapeB<M, W>;
        const int lane = threadIdx.x & 63, n = S::col(lane), q = S::quad(lane);
        const FragSrcB f = src(s + 2 < total ? s + 2 : s);
        const uint16_t* ap = a_lds + n * kLdsB + 8 * q;
        u32x4 a[NGF][S::RT];
#pragma unroll
        for (int g = 0; g < NGF; ++g)
#pragma unroll
            for (int rt = 0; rt < S::RT; ++rt)
                a[g][rt] = *reinterpret_cast<const u32x4*>(ap + S::MT * rt * kLdsB + SB::KB * g);
#pragma unroll
        for (int g = 0; g < NGF; ++g) {
#pragma unroll
            for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
                for (int ct = 0; ct < S::CT; ++ct) acc[rt][ct] = SB::mfma(a[g][rt], b[ROLE].b[g][ct], acc[rt][ct]);
#pragma unroll
            for (int ct = 0; ct < S::CT; ++ct)
                b[ROLE].b[g][ct] = *reinterpret_cast<const u32x4*>(frag_lane_b<M, W>(f, ct) + SB::GROUP * g);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// The forward's GEMM sequence over the bf16 copies (see FwdSeq): Up^T's chunk
// c (K = 128) starts at row 128 c, Down^T's chunk c (K = H) at tile column c.
template <int MT>
struct FwdSeqB {
    const mg_policy_view* pv;
    int nc;
    __device__ __forceinline__ FragSrcB operator()(int s) const {
        const int l = s / (2 * nc), c = (s >> 1) % nc;
        const uint16_t* base = MT == 32 ? pv->frag_fwd32_bf : pv->frag_fwd16_bf;
        if ((s & 1) == 0) return {base + pv->off_up[l] + (size_t)kChunk * c * kEmbed, (uint32_t)kEmbed};
        return {base + pv->off_down[l] + MT * kChunk * c, pv->hidden};
    }
};

// Writes a register tile to a bf16 LDS tile (row stride kLdsB), optionally
// through relu.
template <int M, int W = 4, bool RELU = true>
__device__ __forceinline__ void store_tile_relu_b(const AccTile<M, W>& acc, uint16_t* lds) {
    for_each_elem<M, W>([&](int rt, int ct, int r, int row, int col) {
        const float x = acc[rt][ct][r];
        lds[row * kLdsB + col] = bf16_rne(RELU ? (x > 0.0f ? x : 0.0f) : x);
    });
}

// Row-group-packed layout of a bf16 matrix with C columns (the operand
// layout of the weight-gradient GEMMs, which contract over rows): element
// (r, c) at ((r / 8) C + c) 8 + r % 8, so 8 consecutive rows of one column are
// 16 contiguous bytes. Copies rows 0 .. 15 of a bf16 LDS tile (row stride
// kLdsB, 128 columns) to columns col0 .. col0 + 127 of such a matrix; g points
// at the tile's first row group (a multiple of 16 rows). NT threads.
template <int NT>
__device__ __forceinline__ void copy_tile_p8(const uint16_t* lds, uint16_t* g, uint32_t C, uint32_t col0) {
    for (int i = threadIdx.x; i < 2 * kEmbed; i += NT) {
        const int grp = i / kEmbed, c = i % kEmbed;
        const uint16_t* col = lds + 8 * grp * kLdsB + c;
        u32x4 w;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = (uint32_t)col[2 * j * kLdsB] | ((uint32_t)col[(2 * j + 1) * kLdsB] << 16);
        *reinterpret_cast<u32x4*>(g + ((size_t)grp * C + col0 + c) * 8) = w;
    }
}

// One residual block with bf16 GEMM operands: h += relu(xb Up) Down, chunked
// as in fwd_block; sm.xb holds the block input's LN output in bf16. With VOUT
// (16-row tiles) the relu'd hidden chunks, as the down GEMM saw them, are also
// written to v_out (row-group-packed, H columns, at the tile's first row group).
template <int M, int W, bool VOUT, int NV, class Seq, class Stream>
__device__ __forceinline__ void fwd_block_b(const mg_policy_view& pv, int l, FwdSmemB<M, NV>& sm,
                                            FwdRegs<M, W>& R, Stream& ws, uint16_t* v_out, Seq seq) {
    using S = Shape<M, W>;
    const int H = (int)pv.hidden, NC = H / kChunk;
    for (int c = 0; c < NC; ++c) {
        const int s = 2 * (l * NC + c);
        uint16_t* vb = sm.vb[NV == 2 ? (c & 1) : 0];
        typename S::Acc v[S::RT][S::CT];
        zero<M, W>(v);
        ws.template gemm<0>(v, sm.xb, s, seq);
        if constexpr (NV == 1) __syncthreads();  // every wave is done reading the previous chunk from vb
        store_tile_relu_b<M, W>(v, vb);
        __syncthreads();
        if constexpr (VOUT) {
            static_assert(M == 16, "captures are 16-row tiles");
            copy_tile_p8<S::NT>(vb, v_out, H, kChunk * c);
        }
        ws.template gemm<1>(R.h, vb, s + 1, seq);
    }
}

// Whole forward with bf16 GEMM operands: obs staged in obsL ([M][O], LDS) ->
// head in headL ([M][HD], LDS). HDC, OC: HD and O when known at compile time.
template <int M, int W = 4, int HDC = 0, int OC = 0>
__device__ __forceinline__ void policy_forward_b(const mg_policy_view& pv, const SmallParams& sp, FwdSmemB<M>& sm,
                                                 FwdRegs<M, W>& R, const float* obsL, int O, float* headL, int HD) {
    using Stream = typename std::conditional<M == 16, TStreamB<M, W>, WStreamB<M, W>>::type;
    using Seq = FwdSeqB<Shape<M, W>::MT>;
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
        fwd_layernorm<M, W>(sm, R, g, g + kEmbed, nullptr, nullptr, nullptr, sm.xb);
        fwd_block_b<M, W, false, 1, Seq>(pv, (int)l, sm, R, ws, nullptr, seq);
    }
    const float* g = sp.ln + 2 * kEmbed * pv.layers;
    fwd_layernorm<M, W, FwdSmemB<M>, HDC>(sm, R, g, g + kEmbed, nullptr, nullptr, nullptr, nullptr, sp.wh, headL, HD);
}

}  // namespace dev
}  // namespace mg
