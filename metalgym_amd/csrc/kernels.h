// Launchers of the library's env-agnostic kernels (policy_kernels.hip,
// train_kernels.hip). Each returns MG_OK or an MG_ERR_* code with the error set.
#pragma once
#include <hip/hip_runtime.h>

#include "internal.h"

namespace mg {

int launch_forward(hipStream_t st, const mg_policy_view& pv, const float* obs, uint32_t rows, float* head);
int launch_sample(hipStream_t st, const mg_policy_view& pv, const float* head, uint32_t rows, uint32_t* rng,
                  void* actions, float* logp, float* value);
int launch_gae(hipStream_t st, const float* reward, const uint8_t* done, const float* value, const float* head,
               uint32_t head_dim, uint32_t act_dim, uint32_t n, uint32_t horizon, float gamma, float lambda,
               float* adv, float* ret);
// Mean and 1 / (population std + 1e-8) of each minibatch block of the
// advantage slots (model/gae.metal:42-77), [blocks][2].
int launch_adv_stats(hipStream_t st, const float* adv, uint32_t n, uint32_t horizon, uint32_t minibatch,
                     float* stats);

// Everything one PPO minibatch update needs on the device.
struct TrainWs {
    float* x;         // [L][B][128] LN outputs entering the blocks
    float* v;         // [L][B][H] relu'd hidden activations
    float* dhb;       // [L][B][128] gradients at the block outputs
    float* dvb;       // [L][B][H] masked hidden gradients
    // Per row-tile partial sums of the vector parameters, the head and the
    // loss statistics: [B / kTileRows][tp_count], the vector group at its
    // arena offsets (0 .. float_group), the head [128 x HD] at float_group,
    // then the 5 LossStats sums.
    float* tp;
    float* partial;   // [kSplits][count] per-split sums of the block matrices' gradients
    float* grad;      // [count] the reduced gradient (pre-clip)
    float* normpart;  // [kReduceBlocks] per-workgroup squared norms
    uint32_t tp_count;
};
constexpr int kSplits = 16;        // row splits of the block-matrix gradient sums
constexpr int kTileRows = 16;      // rows per train_rows workgroup
constexpr int kReduceBlocks = 1024; // workgroups of the gradient reduction

struct TrainStep {
    uint32_t row0;       // first slot row of the minibatch (t * n + r0)
    uint32_t block;      // minibatch block id (index into adv stats)
    uint32_t rows;       // B
    uint32_t mb_index;   // index into the per-minibatch stats output
    float beta1_pow, beta2_pow;
};

// All fragment-tiled copies of the block matrices (frag_fwd32, frag_fwd16,
// frag_bwd16 and the bf16 ones that exist) from params.
int launch_derive_blocks(hipStream_t st, const mg_policy_view& pv);
// MG_OK if the block matrices sit contiguously from float_group (the layout
// the Adam and derive kernels tile).
int check_matrix_layout(const mg_policy_view& pv);

int train_ws_bytes(const mg_policy_view& pv, uint32_t rows, size_t* bytes);
int train_ws_bind(const mg_policy_view& pv, uint32_t rows, void* base, TrainWs* ws);
// One minibatch: rows pass, weight-gradient pass, reduce + norm, Adam. Adam
// rewrites only the fragment-tiled copies the row pass reads (frag_fwd16 and
// frag_bwd16, or their bf16 versions in bf16 mode); the others (frag_fwd32
// and, in bf16 mode, the fp32 copies and frag_fwd32_bf, read by collect and
// forward) are stale afterwards until launch_derive_blocks.
int launch_train_step(hipStream_t st, const mg_policy_view& pv, const mg_ppo_hparams& hp, float lr,
                      const TrainWs& ws, const TrainStep& step, const float* obs_slots, const void* action_slots,
                      const float* adv_slots, const float* ret_slots, const float* logp_slots,
                      const float* adv_stats, float* m, float* v, float* head_out, float* mb_stats);

}  // namespace mg
