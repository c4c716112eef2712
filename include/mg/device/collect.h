// collect<Env>: the whole rollout of model/ppo.h:716-751 (minus GAE) in one
// launch. Each workgroup (4 waves; 8 for 16-row tiles) owns M envs for all T steps:
//
//   for t in 0..T:  policy forward on the staged obs (MFMA, see policy.h)
//                   t <  T: env lanes sample from the head with their own RNG,
//                           reset-if-done, Env::step, write the [T][n] slots
//                   t == T: write the bootstrap head (model/ppo.h:735)
//
// Env lanes are threads 0..M-1 (one wave). A small State lives in registers of
// its lane for the whole rollout; a larger one is staged in LDS for the T steps
// when the tile's envs fit beside the forward's LDS (copied in and out by the
// whole workgroup), else it is updated in place in device memory. Per env and
// step the RNG order is: sample draw(s), reset draws if done, then step
// (model/ppo.h:728-730, rollout.h:46-47). An env that declares a split
// observation (OBS_SPLIT, env.h) has its states stepped by the env lanes,
// which also write the observation's other floats; after a barrier all threads
// of the workgroup compute the tile's OBS_SPLIT parts per env.
#pragma once
#include "policy_bf16.h"
#include "policy_split.h"
#include "sample.h"

namespace mg {
namespace dev {

// Launch shape per tile height: 64- and 32-row tiles run 4 waves and two
// workgroups per CU (one when the env lane holds more than 32 observation
// floats, which do not fit beside the weights at two, unless WIDE); 16-row
// tiles (runs of at most 512 workgroups, one per CU) of envs with up to 16
// observation floats run 8 waves, 16 output columns each (a wider observation
// held by the env lane would not fit the register budget of 8 waves).
// WIDE: an env with a split observation whose states stay in device memory,
// two workgroups per CU (VoxelNav's 40 observation floats: 231 VGPRs, no
// spills), so one workgroup's env phase overlaps the other's GEMMs.
template <int M, int O, bool WIDE = false>
struct CollectShape {
    static constexpr int W = M == 16 && O <= 16 ? 8 : 4;
    static constexpr int NT = 64 * W;
    static constexpr int MIN_WG = M == 16 || (O > 32 && !WIDE) ? 1 : 2;  // workgroups per CU
};

// The forward of a tile: fp32 16-row tiles on 8 waves run the split layout
// (split_forward16: no barrier per chunk, and the relu'd hidden chunk never
// goes through LDS); the others stage each hidden chunk in LDS (policy.h,
// policy_bf16.h).
template <int M, int O, bool BF16>
struct CollectFwd {
    static constexpr bool SPLIT = !BF16 && M == 16 && CollectShape<M, O>::W == 8;
    using Smem = std::conditional_t<SPLIT, SplitFwdSmem<8>, std::conditional_t<BF16, FwdSmemB<M>, FwdSmem<M>>>;
};

// The tile's LDS: the forward's, then the staged observations and the head.
// Outside the split forward the observations ([M][O]) and the head ([M][HD])
// share the forward's hidden-chunk buffer: the observations are read only by
// the embed, before the first chunk is written (LN0's barriers between), and
// the head is written after the final LN's first barrier, when every wave is
// done with the last chunk; the env phase that reads the head and writes the
// next observations ends before the next forward. That leaves room at two
// workgroups per CU for VoxelNav16's small parameters but W_in (SmallStage).
// 16-byte aligned in size as well, so the dynamic LDS after the static
// arrays (the staged small parameters, read as float4s) starts 16-byte
// aligned: at 4 bytes past a 16-byte boundary the CartPole collect ran 8%
// slower, bf16 41%.
template <int M, int O, int HD, bool BF16>
struct alignas(16) CollectSmem {
    using Fwd = typename CollectFwd<M, O, BF16>::Smem;
    static constexpr size_t IO = (size_t)M * (O + HD);  // floats: obs, then head
    static constexpr bool ALIAS = !CollectFwd<M, O, BF16>::SPLIT && IO * 4 <= (BF16 ? (size_t)M * kLdsB * 2
                                                                                       : (size_t)M * kLds * 4);
    Fwd fwd;
    float io[ALIAS ? 1 : IO];
    __device__ __forceinline__ float* obs() {
        if constexpr (ALIAS) {
            if constexpr (BF16)
                return reinterpret_cast<float*>(&fwd.vb[0][0]);
            else
                return &fwd.vs[0][0];
        } else {
            return io;
        }
    }
    __device__ __forceinline__ float* head() { return obs() + M * O; }
};

// LDS staging of a State too large for registers: the tile's M states at an
// odd stride of dwords (env e at dword e * STRIDE), so the lanes' accesses to
// one field fall in different banks. Used when the states fit beside the
// forward's LDS at the kernel's workgroups per CU; gathers from a state (a
// VoxelNav heightmap's ray march) then cost an LDS round trip instead of a
// cache miss.
template <typename Env, int M, bool BF16, bool WIDE = false>
struct LdsState {
    using State = typename Env::State;
    static constexpr uint32_t SD = sizeof(State) / 4;           // dwords per state
    static constexpr uint32_t STRIDE = SD % 2 ? SD : SD + 1;   // odd dword stride
    static constexpr size_t BYTES = (size_t)M * STRIDE * 4;
    static constexpr int O = Env::OBS_DIM, HD = Env::ACT_DIM + 1;
    // 256 bytes of headroom for the compiler's alignment padding between the
    // two static LDS arrays
    static constexpr bool USE = !WIDE && !EnvTraits<Env>::STATE_IN_REGISTERS && sizeof(State) % 4 == 0 &&
                                alignof(State) <= 4 &&
                                sizeof(CollectSmem<M, O, HD, BF16>) + BYTES + 256 <=
                                    (size_t)163840 / CollectShape<M, O>::MIN_WG;
};

// LDS copies of the forward's small parameters for the T + 1 forwards of a
// collect (W_in, b_in, the layers + 1 LNs' gamma and beta, W_head), in the
// kernel's dynamic LDS: the embed, LN and head phases then read them without
// an L2 round trip (at one workgroup per CU no other workgroup's MFMAs overlap
// that latency; at two, 64-row tiles, it took the 262144-env CartPole collect
// from 36.0 to 35.4 ms). Used when they fit beside the kernel's static LDS at
// its workgroups per CU (kAll); else all but W_in where those fit (kNoWin:
// W_in is read once per step, by the embed's MFMAs), else none and the forward
// reads the arena. The launcher decides from the static size the compiler gave
// the kernel (padding included) and passes the decision as the kernel's
// second argument.
template <typename Env, int M, bool BF16>
struct SmallStage {
    static constexpr int O = Env::OBS_DIM, HD = Env::ACT_DIM + 1;
    static constexpr int WIN = O * kEmbed, BIN = kEmbed, WH = kEmbed * HD;
    static constexpr uint32_t kNone = 0, kAll = 1, kNoWin = 2;
    __host__ __device__ static constexpr uint32_t floats(uint32_t layers, uint32_t mode = kAll) {
        return (mode == kAll ? WIN : 0) + BIN + (layers + 1) * 2 * kEmbed + WH;
    }
};

// BF16: the policy forward multiplies bfloat16 operands (policy_bf16.h).
template <typename Env, int M, bool BF16, bool WIDE>
__global__ void __launch_bounds__((CollectShape<M, Env::OBS_DIM, WIDE>::NT),
                                  (CollectShape<M, Env::OBS_DIM, WIDE>::MIN_WG))
    collect_kernel(const mg_collect_args a, const uint32_t stage_small) {
    using Tr = EnvTraits<Env>;
    using State = typename Env::State;
    using Action = typename Env::Action;
    using Obs = typename Env::Obs;
    using CS = CollectShape<M, Env::OBS_DIM, WIDE>;
    using LS = LdsState<Env, M, BF16, WIDE>;
    constexpr int O = Env::OBS_DIM, A = Env::ACT_DIM, HD = A + 1;
    // the embed's observation width at compile time (its unrolled k loop reads
    // a row's floats together: VoxelNav at 262144 envs 70.8 -> 66.0 ms) at
    // 64-row and WIDE tiles; the others' register budgets it would overflow
    // (VoxelNav's 32-row tiles with states in LDS: 44 VGPRs spilled)
    constexpr int OE = M == 64 || WIDE ? O : 0;
    // parts of a split observation per env, spread over the whole workgroup
    // when the states sit in LDS or (WIDE) in device memory (0: the env lanes
    // call step()). A State held in registers is written back only at the end,
    // so the other threads could not read it: such an env always calls step().
    constexpr uint32_t KS = LS::USE || (WIDE && !Tr::STATE_IN_REGISTERS) ? Tr::OBS_SPLIT : 0;
    __shared__ CollectSmem<M, O, HD, BF16> sm;
    static_assert(sizeof(CollectSmem<M, O, HD, BF16>) % 16 == 0, "the staged small parameters start 16-byte aligned");
    __shared__ uint32_t lds_state[LS::USE ? M * LS::STRIDE : 1];
    using SS = SmallStage<Env, M, BF16>;
    extern __shared__ __align__(16) float small_lds[];  // SS::floats(layers, stage_small) floats
    FwdRegs<M, CS::W> R;
    std::conditional_t<CollectFwd<M, O, BF16>::SPLIT, SkStream<8 / CS::W>, char> wst;  // split forward's weights

    const int tid = threadIdx.x;
    const uint32_t n = a.n, T = a.horizon;
    const uint32_t i = blockIdx.x * M + (uint32_t)tid;
    const bool envLane = tid < M;
    State* states = static_cast<State*>(a.state);
    Action* actSlots = static_cast<Action*>(a.action_slots);
    const float* logStd = a.policy.params + a.policy.off_log_std;

    uint32_t rng = 0;
    uint8_t done = 0;
    // A small State lives in this register copy; a larger one in LDS or, if it
    // does not fit there, in place in device memory.
    std::conditional_t<Tr::STATE_IN_REGISTERS, State, char> sreg;
    auto S = [&]() -> State& {
        if constexpr (Tr::STATE_IN_REGISTERS)
            return sreg;
        else if constexpr (LS::USE)
            return *reinterpret_cast<State*>(lds_state + tid * LS::STRIDE);
        else
            return states[i];
    };
    if constexpr (LS::USE) {
        // the tile's states are contiguous in device memory: dword k of the run
        // is dword k % SD of env k / SD
        const uint32_t* gin = reinterpret_cast<const uint32_t*>(states + (size_t)blockIdx.x * M);
        states_to_lds<LS::SD, LS::STRIDE, M, CS::NT>(lds_state, gin, M);
        __syncthreads();
    }
    float obs[O];

    SmallParams sp = small_params(a.policy);
    // a runtime choice: a template parameter instead (LDS instructions for the
    // small parameters) measured slower at 4096 and 262144 envs, fp32 and bf16
    if (stage_small) {  // ordered before the forwards by the barrier below
        const int lnf = (int)(a.policy.layers + 1) * 2 * kEmbed;
        const bool all = stage_small == SS::kAll;
        float* win = small_lds;
        float* bin = win + (all ? SS::WIN : 0);
        float* ln = bin + SS::BIN;
        float* wh = ln + lnf;
        if (all)
            for (int k = tid; k < SS::WIN; k += CS::NT) win[k] = sp.win[k];
        for (int k = tid; k < SS::BIN; k += CS::NT) bin[k] = sp.bin[k];
        for (int k = tid; k < lnf; k += CS::NT) ln[k] = sp.ln[k];
        for (int k = tid; k < SS::WH; k += CS::NT) wh[k] = sp.wh[k];
        sp = {all ? win : sp.win, bin, ln, wh};
    }

    if (envLane) {
        rng = a.rng[i];
        done = a.done[i];
        if constexpr (Tr::STATE_IN_REGISTERS) sreg = states[i];
        if (a.first) {  // model/ppo.h:720-722: one step with action 0 into slot 0
            Action act{};
            if (done) Env::reset(S(), rng);
            Obs o{};
            float r = 0.0f;
            Env::step(S(), act, o, r, done);
            const float* of = reinterpret_cast<const float*>(&o);
#pragma unroll
            for (int k = 0; k < O; ++k) obs[k] = of[k];
            store_floats<O>(a.obs_slots + (size_t)i * O, obs);
            a.reward_slots[i] = r;
        } else {  // model/ppo.h:724: obs[T] -> obs[0]
            load_floats<O>(obs, a.obs_slots + ((size_t)T * n + i) * O);
            store_floats<O>(a.obs_slots + (size_t)i * O, obs);
        }
#pragma unroll
        for (int k = 0; k < O; ++k) sm.obs()[tid * O + k] = obs[k];
    }
    __syncthreads();

    for (uint32_t t = 0; t <= T; ++t) {
        if constexpr (CollectFwd<M, O, BF16>::SPLIT)
            split_forward16<CS::W, O>(a.policy, sp, sm.fwd, wst, t == 0, sm.obs(), sm.head(), HD);
        else if constexpr (BF16)
            policy_forward_b<M, CS::W, HD, OE>(a.policy, sp, sm.fwd, R, sm.obs(), O, sm.head(), HD);
        else
            // global weight loads when the env states sit in LDS: there the
            // buffer loads' scalar descriptors cost the heightmap env more
            // spilling than they save (VoxelNav at 262144 envs, 135 -> 151 ms)
            policy_forward<M, CS::W, !LS::USE, HD, OE>(a.policy, sp, sm.fwd, R, sm.obs(), O, sm.head(), HD);
        if (envLane) {
            const float* h = sm.head() + tid * HD;
            if (t == T) {  // bootstrap head for GAE and headValue()
#pragma unroll
                for (int j = 0; j < HD; ++j) a.head_out[(size_t)i * HD + j] = h[j];
            } else {
                const size_t k = (size_t)t * n + i;
                Action act;
                float lp;
                if constexpr (Tr::CONTINUOUS)
                    sample_gaussian(h, logStd, A, rng, reinterpret_cast<float*>(&act), lp);
                else
                    act = (Action)sample_categorical(h, A, rng, lp);
                actSlots[k] = act;
                a.logp_slots[k] = lp;
                a.value_slots[k] = h[A];
                if (done) Env::reset(S(), rng);
                Obs o{};
                float r = 0.0f;
                const float* of = reinterpret_cast<const float*>(&o);
                if constexpr (KS > 0) {  // the floats from KS on; the parts after the barrier below
                    Env::stepState(S(), act, r, done);
                    Env::observeRest(S(), o);
#pragma unroll
                    for (int q = KS; q < O; ++q) {
                        a.obs_slots[(k + n) * O + q] = of[q];
                        sm.obs()[tid * O + q] = of[q];
                    }
                } else {
                    Env::step(S(), act, o, r, done);
#pragma unroll
                    for (int q = 0; q < O; ++q) obs[q] = of[q];
                    store_floats<O>(a.obs_slots + (k + n) * O, obs);
#pragma unroll
                    for (int q = 0; q < O; ++q) sm.obs()[tid * O + q] = obs[q];
                }
                a.reward_slots[k] = r;
                a.done_slots[k] = done;
            }
        }
        if constexpr (KS > 0) {
            if (t < T) {
                __syncthreads();  // every env lane's state is stepped
                // part p of env e, consecutive threads on consecutive parts
                const size_t row0 = ((size_t)(t + 1) * n + (size_t)blockIdx.x * M) * O;
                for (uint32_t q = tid; q < M * KS; q += CS::NT) {
                    const uint32_t e = q / KS, p = q % KS;
                    const State& se = LS::USE ? *reinterpret_cast<const State*>(lds_state + e * LS::STRIDE)
                                              : states[(size_t)blockIdx.x * M + e];
                    const float v = Env::observePart(se, p);
                    sm.obs()[e * O + p] = v;
                    a.obs_slots[row0 + (size_t)e * O + p] = v;
                }
            }
        }
        __syncthreads();
    }
    if (envLane) {
        if constexpr (Tr::STATE_IN_REGISTERS) states[i] = sreg;
        a.rng[i] = rng;
        a.done[i] = done;
    }
    if constexpr (LS::USE) {  // every env lane's last step is before the loop's final barrier
        uint32_t* gout = reinterpret_cast<uint32_t*>(states + (size_t)blockIdx.x * M);
        states_from_lds<LS::SD, LS::STRIDE, M, CS::NT>(lds_state, gout, M);
    }
}

// The kernel's static LDS as the compiler laid it out (SIZE_MAX if the
// runtime cannot tell, which turns the small-parameter staging off).
template <typename Env, int M, bool BF16, bool WIDE>
size_t collect_static_lds() {
    static const size_t bytes = [] {
        hipFuncAttributes attr{};
        if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&collect_kernel<Env, M, BF16, WIDE>)) !=
            hipSuccess) {
            (void)hipGetLastError();  // not this launch's error
            return (size_t)SIZE_MAX;
        }
        return (size_t)attr.sharedSizeBytes;
    }();
    return bytes;
}

template <typename Env, int M, bool BF16, bool WIDE>
void launch_collect_mw(const mg_collect_args* a, hipStream_t st) {
    using SS = SmallStage<Env, M, BF16>;
    constexpr size_t kPerWg = (size_t)163840 / CollectShape<M, Env::OBS_DIM, WIDE>::MIN_WG;  // LDS per workgroup
    const size_t stat = collect_static_lds<Env, M, BF16, WIDE>();
    const size_t all = (size_t)SS::floats(a->policy.layers, SS::kAll) * 4;
    const size_t nowin = (size_t)SS::floats(a->policy.layers, SS::kNoWin) * 4;
    const size_t room = stat <= kPerWg ? kPerWg - stat : 0;
    const uint32_t stage = all <= room ? SS::kAll : nowin <= room ? SS::kNoWin : SS::kNone;
    const size_t dyn = stage == SS::kAll ? all : stage == SS::kNoWin ? nowin : 0;
    const dim3 grid(a->n / M), block(CollectShape<M, Env::OBS_DIM, WIDE>::NT);
    hipLaunchKernelGGL((collect_kernel<Env, M, BF16, WIDE>), grid, block, dyn, st, *a, stage);
}

// An env with a split observation runs WIDE where the grid has at least two
// workgroups per CU (VoxelNav, ms per collect of 32 steps, WIDE against its
// states in LDS at one workgroup per CU: 70.9 / 77.9 at 262144 envs, 4.53 /
// 5.47 at 16384; at 8192 envs, 256 workgroups, 3.23 / 2.81).
template <typename Env, int M, bool BF16>
void launch_collect_m(const mg_collect_args* a, hipStream_t st) {
    if constexpr (EnvTraits<Env>::OBS_SPLIT > 0 && M >= 32) {
        if (a->n / M >= 512) {
            launch_collect_mw<Env, M, BF16, true>(a, st);
            return;
        }
    }
    launch_collect_mw<Env, M, BF16, false>(a, st);
}

template <typename Env, bool BF16>
int launch_collect_tiles(const mg_collect_args* a) {
    hipStream_t st = static_cast<hipStream_t>(a->stream);
    // 64-row tiles reuse each weight fragment across the most rows; they need
    // n / 64 >= 512 workgroups (2 per CU) to fill the chip. Smaller runs use
    // 32-row, then 16-row tiles for more workgroups.
    if (a->n >= 64u * 512u)
        launch_collect_m<Env, 64, BF16>(a, st);
    else if (a->n >= 32u * 256u)
        launch_collect_m<Env, 32, BF16>(a, st);
    else
        launch_collect_m<Env, 16, BF16>(a, st);
    return (int)hipGetLastError();
}

template <typename Env>
int launch_collect(const mg_collect_args* a) {
    if (!a || a->n == 0 || a->n % 64 != 0 || a->horizon == 0) return MG_ERR_INVALID;
    if (a->policy.obs_dim != Env::OBS_DIM || a->policy.act_dim != Env::ACT_DIM ||
        a->policy.embed != (uint32_t)kEmbed || a->policy.hidden % kChunk != 0 || a->policy.layers == 0 ||
        a->policy.layers > MG_MAX_LAYERS)
        return MG_ERR_INVALID;
    if (a->policy.precision == MG_PRECISION_BF16 && (!a->policy.frag_fwd32_bf || !a->policy.frag_fwd16_bf))
        return MG_ERR_INVALID;
    return a->policy.precision == MG_PRECISION_BF16 ? launch_collect_tiles<Env, true>(a)
                                                      : launch_collect_tiles<Env, false>(a);
}

}  // namespace dev
}  // namespace mg
