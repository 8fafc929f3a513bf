// Prefill (grouped-expert) kernel argument blocks and launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace glm53 {

constexpr int kPlanMaxExperts = 1024;
constexpr int kGroupedTileRows = 32;   // routes per descriptor of the reference (grouped_fp8.py:20)
constexpr int kGemmTileRows = 64;      // routes per descriptor of the MFMA grouped GEMM (many routes per expert)
constexpr int kGemmMinTileRows = 32;   // its narrow form (one group per wavefront, deeper ring)
constexpr int kGemmWideRows = 128;     // its wide form (128-route descriptors x 512 weight rows per item)
constexpr int kMaxReduceTopK = 16;
enum { GEMM_PLAIN = 0, GEMM_SWIGLU = 1 };

// The wide shape's direct loads address a weight matrix of `rows` rows and
// an activation plane of `act_rows` rows (K bytes each) through unsigned
// 32-bit offsets from a wave-uniform base, and split each weight row index
// into a wave-uniform multiple of 8 and the lane's 0 .. 7; it is taken only
// where both stay under 2 GiB and rows is a multiple of 8.
inline bool wide_offsets_fit(int64_t rows, int64_t K, int64_t act_rows) {
  const int64_t limit = int64_t{1} << 31;
  return rows % 8 == 0 && rows >= 8 && (rows + 128) * K < limit && act_rows * K < limit;
}

struct RoutePlanArgs {
  const int32_t* expert_ids;  // [routes] flat (token-major, slot-minor)
  const float* scores;        // [routes] or null
  int64_t routes;
  int top_k;
  int experts;
  int tile_rows;
  int64_t blocks;             // ceil(routes / 256)
  int64_t capacity;           // ceil(routes / tile_rows) + experts
  unsigned* block_counts;     // [blocks, experts] scratch
  unsigned* block_invalid;    // [blocks] scratch
  int32_t* sorted_route;      // [routes] order
  int32_t* inverse;           // [routes]
  int32_t* sorted_expert;     // [routes]
  int32_t* sorted_token;      // [routes]
  float* sorted_score;        // [routes]
  unsigned* route_offsets;    // [experts + 1]
  unsigned* tile_offsets;     // [experts + 1]
  int32_t* tile_expert;       // [capacity]
  int32_t* tile_start;        // [capacity]
  int32_t* tile_len;          // [capacity]
  unsigned* status;           // [2]: invalid routes, valid descriptors
};

struct SplitArgs {
  const uint16_t* x;          // [rows, cols] bf16
  int64_t x_row_stride;
  int64_t rows, cols;         // cols % 128 == 0
  uint8_t* hi;                // [rows, cols] E4M3
  uint8_t* lo;                // [rows, cols] E4M3 (residual * 16)
  float* scale;               // [rows, cols / 128] power of two
};

struct GroupedGemmArgs {
  const uint8_t* a_hi;
  const uint8_t* a_lo;
  const float* a_scale;       // [act_rows, K / 128]
  const int32_t* a_row_index; // [routes] -> activation row, or null (identity)
  int64_t K;                  // % 128 == 0
  int64_t routes;
  const int32_t* tile_expert; // descriptors, or null: implicit expert 0, 32-route tiles
  const int32_t* tile_start;
  const int32_t* tile_len;
  int64_t experts;
  const uint8_t* weight;      // expert e rows at weight + e * w_expert_stride, [rows, K]
  const uint8_t* weight_up;   // SwiGLU mode: up rows, same strides
  int64_t w_expert_stride;
  int w_group_log2;           // row groups of each expert matrix (common.h; 0 = row-major)
  const float* scale;         // expert e block scales, [ceil(rows/128), s_cols]
  const float* scale_up;
  int64_t s_expert_stride;
  int64_t s_cols;
  int64_t N;                  // output columns (PLAIN) / intermediate columns (SWIGLU)
  float limit;
  uint16_t* out;              // [routes, out_row_stride] bf16
  int64_t out_row_stride;
  const int32_t* fixup;       // device flag: weights hold 0x7F/0xFF codes (or null)
  const int32_t* fixup_up;    // SwiGLU mode: the up weights' flag when kept apart (or null)
  int tile_rows;                 // routes per descriptor: kGemmMinTileRows, kGemmTileRows (also 0) or kGemmWideRows
  int64_t n_tiles, descriptors;  // set by the launcher
  // device count of the routed descriptors in use (the route plan's
  // status[1]), or null: all `descriptors`.  Work items are dealt over
  // the descriptors in use only, so unused capacity costs no XCD share.
  const unsigned* used_descriptors;
  // A dense problem run by the same launch after the routed descriptors (the
  // shared expert): x_descriptors implicit descriptors of tile_rows rows over
  // rows 0 .. x_routes - 1 (identity activation rows), with its own
  // activation planes, weights, block scales and output; same K, N and scale
  // layout as the routed problem.  x_descriptors = 0: none.
  int64_t x_descriptors, x_routes;
  const uint8_t* x_a_hi;
  const uint8_t* x_a_lo;
  const float* x_a_scale;
  const uint8_t* x_weight;
  const uint8_t* x_weight_up;
  int x_w_group_log2;         // row groups of the dense problem's weights
  const float* x_scale;
  const float* x_scale_up;
  uint16_t* x_out;
  int64_t x_out_row_stride;
  const int32_t* x_fixup;     // the dense problem's weight flags (either may be null)
  const int32_t* x_fixup_up;
};

struct ReduceArgs {
  const uint16_t* route_out;  // [routes, H] in sorted order
  const int32_t* inverse;     // [tokens * top_k] -> sorted position
  const float* sorted_score;  // [routes] (grouped order)
  const float* route_score;   // [tokens * top_k] (Direct order)
  const int32_t* expert_ids;  // [tokens * top_k] (Direct order)
  const uint16_t* shared;     // [tokens, H] or null
  int64_t tokens, H;
  int top_k;
  uint16_t* out;              // [tokens, H] (unused when hc_out is set)
  // Hyper-connection expand epilogue (metal:2362-2388), kHcBranches streams:
  // hc_out[t, b, h] = T(post[t, b] * moe[t, h] + fma-chain_s comb[t, s, b] *
  // residual[t, s, h]), moe = the BF16 MoE output; hc_out null: plain out.
  const uint16_t* hc_residual;  // [tokens, kHcBranches, H]
  const float* hc_post;         // [tokens, kHcBranches]
  const float* hc_comb;         // [tokens, kHcBranches (source), kHcBranches (branch)]
  uint16_t* hc_out;             // [tokens, kHcBranches, H]
};
constexpr int kHcBranches = 4;

hipError_t launch_route_plan(const RoutePlanArgs& a, hipStream_t st);
hipError_t launch_split_activations(const SplitArgs& a, hipStream_t st);
hipError_t launch_grouped_gemm(const GroupedGemmArgs& a, int mode, int64_t descriptors, hipStream_t st);
hipError_t launch_reduce(const ReduceArgs& a, bool direct_order, hipStream_t st);
hipError_t launch_scan_480(const uint8_t* codes, int64_t n, int32_t* flag, bool clear, hipStream_t st);

}  // namespace glm53
