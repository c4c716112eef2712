// Device-side building blocks shared by the env kernels (compiled per env by
// MG_DEFINE_ENV) and by the library's policy/PPO kernels. gfx950 (CDNA4) only:
// 64-lane wavefronts, fp32 MFMA, 160 KB LDS per CU.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../capi.h"
#include "../env.h"

namespace mg {
namespace dev {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;
constexpr int kEmbed = MG_EMBED;  // 128, compile-time as in the reference (model/config.h:7)

// v_mfma_f32_32x32x2_f32: D[32x32] += A[32x2] B[2x32].
// Operands: lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32].
// Result: register r of lane l holds D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
__device__ __forceinline__ f32x16 mfma32x32x2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
// v_mfma_f32_16x16x4_f32: D[16x16] += A[16x4] B[4x16].
// Operands: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16].
// Result: register r of lane l holds D[4 (l / 16) + r][l % 16].
__device__ __forceinline__ f32x4 mfma16x16x4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// 16 bytes per lane from a wave-uniform base: base + soff + voff bytes, as
// buffer_load_dwordx4 with the base in a buffer resource (SGPRs), soff in an
// SGPR and voff in a VGPR, so no per-load 64-bit address arithmetic runs on
// the VALU beside the MFMAs. The resource has no meaningful size limit (the
// callers' offsets stay inside their arrays by construction).
__device__ __forceinline__ f32x4 buffer_load16(const void* base, uint32_t voff, uint32_t soff) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                                                       0x00020000);
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

// One float per lane, addressed as buffer_load16.
__device__ __forceinline__ float buffer_load4(const void* base, uint32_t voff, uint32_t soff) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                                                       0x00020000);
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}

__device__ __forceinline__ int c32_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
__device__ __forceinline__ int c16_row(int r, int lane) { return 4 * (lane >> 4) + r; }

// v from another lane of its 16-lane row (a DPP move; CTRL is the dpp_ctrl
// pattern).
template <int CTRL>
__device__ __forceinline__ float dpp_lane(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// The values of lane l and lane l ^ 16 (X = 16: v_permlane16_swap, which
// exchanges the odd rows of its first operand with the even rows of its
// second, 16 lanes a row) or lane l ^ 32 (X = 32: v_permlane32_swap, the
// upper half of the first with the lower half of the second), both operands
// copies of v: the first then holds the lower lane's value and the second the
// upper lane's. Written as inline assembly because the compiler folds the
// builtins' two results into one when both inputs are the same value; the
// s_nop gives the two wait states a swap needs after a VALU write of its
// operands (the copies). Every lane of the wave must be active.
template <int X>
__device__ __forceinline__ void lane_pair(float v, float& lower, float& upper) {
    static_assert(X == 16 || X == 32, "row or half-wave partner");
    lower = v, upper = v;
    if constexpr (X == 16)
        asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(lower), "+v"(upper));
    else
        asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lower), "+v"(upper));
}

// Sum over groups of G consecutive lanes (G a power of two <= 64); every lane
// of a group gets the same bits. Inside a 16-lane row the partners come from
// DPP moves (quad_perm xor 1, xor 2, then the half-row and row mirrors, each
// pairing the group's halves); across rows from the permlane swaps (lane
// l ^ 16, then l ^ 32), each pair added lower lane first. Every lane of the
// wave must be active.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "power-of-two group");
    if constexpr (G >= 2) v += dpp_lane<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    if constexpr (G >= 4) v += dpp_lane<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    if constexpr (G >= 8) v += dpp_lane<0x141>(v);  // row_half_mirror
    if constexpr (G >= 16) v += dpp_lane<0x140>(v); // row_mirror
    if constexpr (G >= 32) {
        float lo, hi;
        lane_pair<16>(v, lo, hi);
        v = lo + hi;
    }
    if constexpr (G >= 64) {
        float lo, hi;
        lane_pair<32>(v, lo, hi);
        v = lo + hi;
    }
    return v;
}

// group_sum of each of N values, the steps of all N interleaved (the same
// bits per value as group_sum).
template <int G, int N>
__device__ __forceinline__ void group_sum_n(float (&v)[N]) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "power-of-two group");
#pragma unroll
    for (int i = 0; i < N; ++i)
        if constexpr (G >= 2) v[i] += dpp_lane<0xB1>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if constexpr (G >= 4) v[i] += dpp_lane<0x4E>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if constexpr (G >= 8) v[i] += dpp_lane<0x141>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if constexpr (G >= 16) v[i] += dpp_lane<0x140>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if constexpr (G >= 32) {
            float lo, hi;
            lane_pair<16>(v[i], lo, hi);
            v[i] = lo + hi;
        }
#pragma unroll
    for (int i = 0; i < N; ++i)
        if constexpr (G >= 64) {
            float lo, hi;
            lane_pair<32>(v[i], lo, hi);
            v[i] = lo + hi;
        }
}

// Sum of t[0..N) as a pairwise tree (t[c] + t[c + N/2], then halves again),
// five dependent adds for 32 terms instead of 31; N a power of two. Overwrites t.
template <int N>
__device__ __forceinline__ float tree_sum(float (&t)[N]) {
    static_assert(N >= 1 && (N & (N - 1)) == 0, "power-of-two count");
#pragma unroll
    for (int w = N / 2; w >= 1; w /= 2)
#pragma unroll
        for (int c = 0; c < w; ++c) t[c] = t[c] + t[c + w];
    return t[0];
}

// Maximum over groups of G consecutive lanes, the same partner pattern.
template <int G>
__device__ __forceinline__ float group_max(float v) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "power-of-two group");
    if constexpr (G >= 2) v = fmaxf(v, dpp_lane<0xB1>(v));
    if constexpr (G >= 4) v = fmaxf(v, dpp_lane<0x4E>(v));
    if constexpr (G >= 8) v = fmaxf(v, dpp_lane<0x141>(v));
    if constexpr (G >= 16) v = fmaxf(v, dpp_lane<0x140>(v));
    if constexpr (G >= 32) {
        float lo, hi;
        lane_pair<16>(v, lo, hi);
        v = fmaxf(lo, hi);
    }
    if constexpr (G >= 64) {
        float lo, hi;
        lane_pair<32>(v, lo, hi);
        v = fmaxf(lo, hi);
    }
    return v;
}

// Store OBS_DIM floats with the widest stores the row alignment allows.
template <int N>
__device__ __forceinline__ void store_floats(float* dst, const float* src) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i)
            reinterpret_cast<float4*>(dst)[i] = make_float4(src[4 * i], src[4 * i + 1], src[4 * i + 2], src[4 * i + 3]);
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) reinterpret_cast<float2*>(dst)[i] = make_float2(src[2 * i], src[2 * i + 1]);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

template <int N>
__device__ __forceinline__ void load_floats(float* dst, const float* src) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            float4 v = reinterpret_cast<const float4*>(src)[i];
            dst[4 * i] = v.x, dst[4 * i + 1] = v.y, dst[4 * i + 2] = v.z, dst[4 * i + 3] = v.w;
        }
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            float2 v = reinterpret_cast<const float2*>(src)[i];
            dst[2 * i] = v.x, dst[2 * i + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

// The states of ne <= MAXE consecutive envs (SD dwords each, contiguous in
// device memory at g) to LDS at STRIDE dwords per env, by NT threads, and back.
// With SD a multiple of 4 and g 16-byte aligned: 16-byte accesses, and every
// load of a thread issued before its first LDS store, so the workgroup waits
// one memory round trip (a load-then-store loop waits one per iteration: 17
// for four VoxelNav16 states).
template <uint32_t SD, uint32_t STRIDE, uint32_t MAXE, int NT>
__device__ __forceinline__ void states_to_lds(uint32_t* lds, const uint32_t* g, uint32_t ne) {
    const uint32_t tid = threadIdx.x;
    if constexpr (SD % 4 == 0) {
        if ((reinterpret_cast<uintptr_t>(g) & 15u) == 0) {
            constexpr uint32_t Q = SD / 4;
            constexpr int NQ = (int)((MAXE * Q + NT - 1) / NT);
            const uint32_t nq = ne * Q;  // ne >= 1
            const uint4* g4 = reinterpret_cast<const uint4*>(g);
            // Branch-free: a thread past the end loads and stores the last
            // 16 bytes again (the same values to the same LDS dwords), so no
            // load is sunk into a conditional store block behind the others.
            uint32_t kk[NQ];
            uint4 v[NQ];
#pragma unroll
            for (int u = 0; u < NQ; ++u) {
                const uint32_t k = tid + (uint32_t)(NT * u);
                kk[u] = k < nq ? k : nq - 1;
                v[u] = g4[kk[u]];
            }
#pragma unroll
            for (int u = 0; u < NQ; ++u) {
                uint32_t* d = lds + (kk[u] / Q) * STRIDE + (kk[u] % Q) * 4;
                d[0] = v[u].x, d[1] = v[u].y, d[2] = v[u].z, d[3] = v[u].w;
            }
            return;
        }
    }
    for (uint32_t k = tid; k < ne * SD; k += NT) lds[(k / SD) * STRIDE + k % SD] = g[k];
}

// Back to device memory: with HW < SD, of env e only dwords [0, HW) (rounded
// up to 16 bytes on the vector path) unless full[e] (LDS) is non-zero.
template <uint32_t SD, uint32_t STRIDE, uint32_t MAXE, int NT, uint32_t HW = SD>
__device__ __forceinline__ void states_from_lds(const uint32_t* lds, uint32_t* g, uint32_t ne,
                                                const uint32_t* full = nullptr) {
    const uint32_t tid = threadIdx.x;
    if constexpr (SD % 4 == 0) {
        if ((reinterpret_cast<uintptr_t>(g) & 15u) == 0) {
            constexpr uint32_t Q = SD / 4, HQ = (HW + 3) / 4;
            constexpr int NQ = (int)((MAXE * Q + NT - 1) / NT);
            const uint32_t nq = ne * Q;
            uint4* g4 = reinterpret_cast<uint4*>(g);
#pragma unroll
            for (int u = 0; u < NQ; ++u) {
                const uint32_t k = tid + (uint32_t)(NT * u);
                if (k < nq && (HQ >= Q || k % Q < HQ || full[k / Q])) {
                    const uint32_t* s = lds + (k / Q) * STRIDE + (k % Q) * 4;
                    g4[k] = make_uint4(s[0], s[1], s[2], s[3]);
                }
            }
            return;
        }
    }
    for (uint32_t k = tid; k < ne * SD; k += NT)
        if (HW >= SD || k % SD < HW || full[k / SD]) g[k] = lds[(k / SD) * STRIDE + k % SD];
}

// A uniformly random action from the env's stream (this build's random policy):
// rngInt(rng, ACT_DIM) for an integer action, uniform [-1, 1) per float.
template <typename Env>
__device__ __forceinline__ typename Env::Action random_action(uint32_t& rng) {
    using Action = typename Env::Action;
    if constexpr (EnvTraits<Env>::CONTINUOUS) {
        Action a;
        float* f = reinterpret_cast<float*>(&a);
#pragma unroll
        for (uint32_t k = 0; k < Env::ACT_DIM; ++k) f[k] = rngUniform(rng, -1.0f, 1.0f);
        return a;
    } else {
        return (Action)rngInt(rng, Env::ACT_DIM);
    }
}

}  // namespace dev
}  // namespace mg
