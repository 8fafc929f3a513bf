// Kernel argument blocks and host launchers (internal to libglm53_moe.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace glm53 {

constexpr int kMaxTopK = 8;
constexpr int kMaxExperts = 1024;
constexpr int kMaxRouterExperts = 512;  // top-k selection bound (8 candidates per lane)
constexpr int kMaxDownRowsPerWg = 64;

// ---------------------------------------------------------------- decode --

struct GateUpArgs {
  const uint16_t* x;              // [H] bf16
  const int32_t* expert_ids;      // [top_k]
  int top_k;
  int64_t experts;
  const uint8_t* gate_up_weight;  // [E, 2I, H]
  const float* gate_up_scale;     // [E, 2*ceil(I/128), ceil(H/128)]
  int bank_group_log2;            // row groups of gate_up_weight (common.h; 0 = row-major)
  const uint8_t* shared_gate_weight;  // [Is, H] or null
  const float* shared_gate_scale;
  const uint8_t* shared_up_weight;
  const float* shared_up_scale;
  int64_t hidden, intermediate, shared_intermediate;
  float limit;
  int rows_per_wave;
  int64_t wgs_per_slot;
  uint16_t* hidden_out;           // [top_k, I] then [Is]
  int* error_flag;
  // fused top-k (router_logits non-null): selection replaces expert_ids
  const float* router_logits;     // [E] FP32
  const float* router_bias;       // [E]
  float routed_scaling_factor;
  int norm_topk_prob;
  int n_group, topk_group;        // group-limited selection (stream_gemv.h GroupLimit)
  int32_t* ids_out;               // [top_k], written by workgroup 0
  float* scores_out;              // [top_k]
  // device code flags (0 = no 0x7F/0xFF code, register decode allowed)
  const int32_t* routed_flags;
  const int32_t* shared_flags;    // shared gate
  const int32_t* shared_flags2;   // shared up
};

struct DownArgs {
  const uint16_t* hidden_in;      // [top_k, I] then shared [I]
  const int32_t* expert_ids;
  const float* scores;            // [top_k]
  int top_k;
  int64_t experts;
  const uint8_t* down_weight;     // [E, H, I]
  const float* down_scale;        // [E, ceil(H/128), ceil(I/128)]
  int bank_group_log2;            // row groups of down_weight (common.h; 0 = row-major)
  const uint8_t* shared_down_weight;  // [H, I] or null
  const float* shared_down_scale;
  int64_t hidden, intermediate;
  int64_t rows_per_wg;
  const uint16_t* residual;       // [H] bf16 or null: out = T(residual + T(moe))
  uint16_t* out;                  // [H] bf16 (may alias residual)
  int* error_flag;
  const int32_t* routed_flags;    // as GateUpArgs
  const int32_t* shared_flags;
};

// Three-launch decode step (step.hip).
struct StepArgs {
  const uint16_t* x;              // [H] bf16
  const uint16_t* residual;       // [H] bf16 or null
  uint16_t* out;                  // [H] bf16
  int64_t hidden, intermediate;   // H, I (shared expert width == I)
  int64_t experts;
  int top_k;
  float limit;
  const float* router_weight;     // [E, H] (null: ids / scores given)
  const float* router_bias;       // [E]
  float routed_scaling_factor;
  int norm_topk_prob;
  int n_group, topk_group;        // group-limited selection (stream_gemv.h GroupLimit)
  unsigned long long* route_words;  // [E] launch 1 exchange: sigmoid bits << 32 | selection key
  uint32_t* router_count;         // arrival counter of launch 1 (self-resetting)
  int32_t* ids;                   // [top_k]: launch 1 writes (router) or given
  float* scores;                  // [top_k]
  const uint8_t* gate_up_weight;
  const float* gate_up_scale;
  const uint8_t* down_weight;
  const float* down_scale;
  int bank_group_log2;            // row groups of both bank matrices (common.h; 0 = row-major)
  const uint8_t* shared_gate_weight;  // null: no shared expert
  const float* shared_gate_scale;
  const uint8_t* shared_up_weight;
  const float* shared_up_scale;
  const uint8_t* shared_down_weight;
  const float* shared_down_scale;
  const int32_t* routed_flags;
  const int32_t* shared_gate_flags;
  const int32_t* shared_up_flags;
  const int32_t* shared_down_flags;
  uint16_t* hidden_act;           // [top_k + 1, I] SwiGLU rows (routed slots, then shared)
  uint16_t* shared_out;           // [H] T(shared down)
  int* error_flag;
  int router_wgs;                 // ceil(E / 4) or 0
  int shared_rows_per_wave;       // launch 1 shared gate/up rows per wavefront
  int routed_wgs;                 // launch 2 workgroups over the routed units
  int shared_delay;               // launch 1: sleeps of ~512 clocks before the shared rows load
};

// Launch 1's shared-expert workgroups wait this many ~512-clock sleeps before
// loading, so the router rows (on the selection's critical path) meet an
// idle memory system.
constexpr int kStepSharedDelay = 2;
bool step_shape_supported(int64_t H, int64_t I);
int step_gate_up_occupancy(int64_t H, int64_t I);
hipError_t launch_step(const StepArgs& a, int stages, hipStream_t st);

struct RouterArgs {
  const uint16_t* x;       // [tokens, H] bf16
  const float* weight;     // [E, H]
  int64_t experts, hidden;
  int64_t tokens;          // 0 or 1: one token
  float* logits_out;       // [tokens, E] FP32
};

struct GenericLinearArgs {
  const uint16_t* x;
  int64_t x_row_stride, x_group_stride;
  const uint8_t* weight;
  int64_t w_expert_stride, w_row_offset;
  int w_group_log2;           // row groups of each expert matrix (common.h; 0 = row-major)
  const float* scale;
  int64_t s_expert_stride, s_row_offset, s_cols;
  const int32_t* expert_ids;  // [G] or null
  int64_t experts;
  int64_t M, G, N, K;
  int rows_per_wave;
  int tile_rows;              // activation rows staged in LDS per pass
  uint16_t* y;
  int64_t y_row_stride, y_group_stride;
  int* error_flag;
};

struct SwigluArgs {
  const uint16_t* gate;
  const uint16_t* up;
  int64_t gate_row_stride, up_row_stride;
  int64_t rows, cols;
  float limit;
  uint16_t* out;
  int64_t out_row_stride;
};

struct WeightedReductionArgs {
  const uint16_t* down;    // [top_k, H]
  const float* scores;     // [top_k]
  const uint16_t* addend;  // [H] or null
  int top_k;
  int64_t H;
  uint16_t* out;
};

struct GemvArgs {
  const uint16_t* x;      // [K] bf16
  const uint8_t* weight;  // [N, K]
  const float* scale;     // [ceil(N/128), ceil(K/128)]
  int64_t N, K;
  int rows_per_wave;
  uint16_t* y;            // [N] bf16
  const int32_t* flags;   // device code flag (null: exact SWAR decode)
};

struct TopkArgs {
  const float* logits;    // [splits][tokens, experts] FP32 partial sums, added in split order
  const float* bias;      // [experts]
  int64_t tokens, experts;
  int splits;             // 0 or 1: logits are whole
  int64_t split_stride;   // elements between partial planes
  int top_k;
  float routed_scaling_factor;
  int norm_topk_prob;
  int n_group, topk_group;  // group-limited selection (stream_gemv.h GroupLimit)
  int32_t* ids_out;       // [tokens, top_k]
  float* scores_out;      // [tokens, top_k]
};

constexpr int kGenericRows = 8;

bool fast_width_supported(int64_t K);
hipError_t launch_gate_up(const GateUpArgs& a, hipStream_t st);
hipError_t launch_down(const DownArgs& a, hipStream_t st);
hipError_t launch_router(const RouterArgs& a, hipStream_t st);
hipError_t launch_gemv(const GemvArgs& a, hipStream_t st);
constexpr int kMaxGemvParts = 16;  // split-K GEMV: one wavefront per 4096-wide part, K <= 65536
bool split_width_supported(int64_t K);
hipError_t launch_gemv_split(const GemvArgs& a, hipStream_t st);  // rows_per_wave = rows per workgroup
hipError_t launch_topk(const TopkArgs& a, hipStream_t st);

// Router logits for many tokens on BF16 MFMA (exact three-way BF16 split of
// the FP32 weights, done as the weights go into LDS): partial sums per K
// chunk, [splits][tokens][experts].
struct RouterGemmArgs {
  const uint16_t* x;      // [tokens, hidden] bf16, 16-byte aligned rows
  float* partial;         // [splits, tokens, experts]
  int64_t tokens, hidden, experts;
  int64_t token_groups, expert_groups, k_chunk, splits;
};
constexpr int kMaxRouterSplits = 16;
struct RouterGemmShape {
  int64_t token_groups, expert_groups, k_chunk, splits;  // splits <= kMaxRouterSplits
};
bool router_gemm_supported(int64_t hidden, int64_t experts, const void* x, const void* weight);
RouterGemmShape router_gemm_shape(int64_t tokens, int64_t hidden, int64_t experts);
hipError_t launch_router_logits(const RouterGemmArgs& a, const float* weight, hipStream_t st);
hipError_t launch_linear_generic(const GenericLinearArgs& a, hipStream_t st);
hipError_t launch_swiglu(const SwigluArgs& a, hipStream_t st);
hipError_t launch_swiglu_stages(const SwigluArgs& a, uint16_t* sigma, uint16_t* silu, hipStream_t st);
hipError_t launch_weighted_reduction(const WeightedReductionArgs& a, hipStream_t st);
hipError_t launch_sigmoid_bf16(const uint16_t* g, uint16_t* out, int64_t n, hipStream_t st);
hipError_t launch_add_bf16(const uint16_t* a, const uint16_t* b, uint16_t* out, int64_t n, hipStream_t st);

}  // namespace glm53
