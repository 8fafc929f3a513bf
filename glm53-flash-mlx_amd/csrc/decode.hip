// Batch-1 decode kernels for the FP8 block-scaled packed MoE layer.
//
// Streaming GEMV design for CDNA4: one wavefront owns a run of consecutive
// weight rows; each lane owns a fixed slice of the reduction dimension, so
// its activations are loaded once (into registers, as exact FP16 pairs) and
// every weight row is read with 16- or 8-byte vector loads that coalesce into
// 1 KB / 512 B contiguous segments per wave instruction.  E4M3 bytes are
// decoded in registers (common.h) and contracted with v_dot2_f32_f16; the
// 128-column block scale is applied once per chunk.  Row totals come from a
// DPP wave reduction.  Nothing is ever expanded to a BF16 weight copy.
//
// Reference semantics: packed.py:100-179 (fused gate/up/SwiGLU, down,
// weighted reduction), packed.py:181-235 (shared expert), fp8.py:41-116
// (block_fp8_linear), patch.py:131-142 (FP32 router).
#include "common.h"
#include "kernels.h"
#include "stream_gemv.h"

namespace glm53 {

// --------------------------------------------- fused routed gate/up/SwiGLU --
//
// packed.py:100-166 for the top_k selected experts (slots 0..k-1) plus, as
// slot k, packed.py:181-235 for the shared expert.  One wavefront computes
// `rows_per_wave` consecutive intermediate rows r of one slot: it streams
// gate row r and up row r (the bank's rows r and I + r), and lane 0 stores
// h = SwiGLU(T(gate), T(up)) with the reference's rounding sequence.
//
// With router logits given, wavefront 0 of every routed workgroup runs the
// top-k itself (288 logits from L2), so the router launch needs no
// cross-workgroup reduction; workgroup 0 also publishes ids and weights for
// the down kernel.
template <int VB, int CH, bool HW>
__device__ __forceinline__ void gate_up_rows(const GateUpArgs& a, const uint8_t* __restrict__ gate_w,
                                             const uint8_t* __restrict__ up_w, const float* __restrict__ gate_s,
                                             const float* __restrict__ up_s, uint16_t* __restrict__ out,
                                             int64_t r0, int64_t r_end, int g, int lane) {
  const int64_t K = a.hidden;
  const int64_t SC = (K + kBlock - 1) / kBlock;
  const RowWalk walk = row_walk<VB>(lane, g);
  XRaw<VB, CH> raw;
  load_x_raw<VB, CH>(a.x, lane, raw);
  XSlice<VB, CH, HW> xs;
  bool packed = false;
  int64_t r = r0;
  for (; r + 1 < r_end; r += 2) {
    WRow<VB, CH> g0, u0, g1, u1;
    const int64_t o0 = group_row_base(r, K, g), o1 = group_row_base(r + 1, K, g);
    load_wrow_walk<VB, CH>(g0, gate_w + o0, gate_s + (r >> 7) * SC, lane, walk);
    load_wrow_walk<VB, CH>(u0, up_w + o0, up_s + (r >> 7) * SC, lane, walk);
    load_wrow_walk<VB, CH>(g1, gate_w + o1, gate_s + ((r + 1) >> 7) * SC, lane, walk);
    load_wrow_walk<VB, CH>(u1, up_w + o1, up_s + ((r + 1) >> 7) * SC, lane, walk);
    if (!packed) {
      pack_x_raw<VB, CH, HW>(raw, xs);
      packed = true;
    }
    float tg0 = wave_sum(wrow_partial<VB, CH, HW>(g0, xs)), tu0 = wave_sum(wrow_partial<VB, CH, HW>(u0, xs));
    float tg1 = wave_sum(wrow_partial<VB, CH, HW>(g1, xs)), tu1 = wave_sum(wrow_partial<VB, CH, HW>(u1, xs));
    if (lane == 0) {
      out[r] = swiglu_mlx(tg0, tu0, a.limit);
      out[r + 1] = swiglu_mlx(tg1, tu1, a.limit);
    }
  }
  if (r < r_end) {
    WRow<VB, CH> g0, u0;
    const int64_t o0 = group_row_base(r, K, g);
    load_wrow_walk<VB, CH>(g0, gate_w + o0, gate_s + (r >> 7) * SC, lane, walk);
    load_wrow_walk<VB, CH>(u0, up_w + o0, up_s + (r >> 7) * SC, lane, walk);
    if (!packed) pack_x_raw<VB, CH, HW>(raw, xs);
    float tg0 = wave_sum(wrow_partial<VB, CH, HW>(g0, xs));
    float tu0 = wave_sum(wrow_partial<VB, CH, HW>(u0, xs));
    if (lane == 0) out[r] = swiglu_mlx(tg0, tu0, a.limit);
  }
}

template <int VB, int CH>
__global__ __launch_bounds__(256) void gate_up_swiglu_kernel(GateUpArgs a) {
  __shared__ int32_t s_ids[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slots_routed = a.top_k;
  const int bid = blockIdx.x;
  int slot, chunk;
  int64_t rows;
  if (bid < slots_routed * a.wgs_per_slot) {
    slot = bid / a.wgs_per_slot;
    chunk = bid % a.wgs_per_slot;
    rows = a.intermediate;
  } else {
    slot = slots_routed;
    chunk = bid - slots_routed * a.wgs_per_slot;
    rows = a.shared_intermediate;
  }
  int32_t e = 0;
  if (slot < slots_routed) {
    if (a.router_logits != nullptr) {  // uniform per workgroup
      if (wave == 0) {
        wave_topk_narrow(a.router_logits, a.router_bias, a.experts, a.top_k, a.routed_scaling_factor, a.norm_topk_prob,
                         lane, s_ids, s_w, GroupLimit{a.n_group, a.topk_group});
        if (lane == 0 && bid == 0) {
          for (int s = 0; s < a.top_k; ++s) {
            a.ids_out[s] = s_ids[s];
            a.scores_out[s] = s_w[s];
          }
        }
      }
      __syncthreads();
      e = s_ids[slot];
    } else {
      e = a.expert_ids[slot];
    }
  }
  const int64_t r0 = (static_cast<int64_t>(chunk) * 4 + wave) * a.rows_per_wave;
  if (r0 >= rows) return;
  const int64_t K = a.hidden;
  const int64_t SC = (K + kBlock - 1) / kBlock;

  const uint8_t* gate_w;
  const uint8_t* up_w;
  const float* gate_s;
  const float* up_s;
  uint16_t* out;
  if (slot < slots_routed) {
    out = a.hidden_out + static_cast<int64_t>(slot) * a.intermediate;
    if (bad_expert(e, a.experts)) {
      if (lane == 0) {
        atomicOr(a.error_flag, 1);
        for (int64_t r = r0; r < r0 + a.rows_per_wave && r < rows; ++r) out[r] = 0x7FC0u;
      }
      return;
    }
    const int64_t SR = (a.intermediate + kBlock - 1) / kBlock;
    gate_w = a.gate_up_weight + static_cast<int64_t>(e) * 2 * a.intermediate * K;
    up_w = gate_w + a.intermediate * K;  // row I: a whole number of row groups (I % 128 == 0 when g > 0)
    gate_s = a.gate_up_scale + static_cast<int64_t>(e) * 2 * SR * SC;
    up_s = gate_s + SR * SC;
  } else {
    out = a.hidden_out + static_cast<int64_t>(slots_routed) * a.intermediate;
    gate_w = a.shared_gate_weight;
    up_w = a.shared_up_weight;
    gate_s = a.shared_gate_scale;
    up_s = a.shared_up_scale;
  }

  const int64_t r_end = (r0 + a.rows_per_wave < rows) ? r0 + a.rows_per_wave : rows;
  const int g = slot < slots_routed ? a.bank_group_log2 : 0;
  if (slot < slots_routed ? hw_decode_ok(a.routed_flags)
                           : (hw_decode_ok(a.shared_flags) && hw_decode_ok(a.shared_flags2)))
    gate_up_rows<VB, CH, true>(a, gate_w, up_w, gate_s, up_s, out, r0, r_end, g, lane);
  else
    gate_up_rows<VB, CH, false>(a, gate_w, up_w, gate_s, up_s, out, r0, r_end, g, lane);
}

// ------------------------------------- fused down + reduction + shared add --
//
// packed.py:66-98 (down for the k slots), packed.py:168-179 (ordered FP32
// weighted reduction), fp8.py:254-299 (shared down GEMV) and
// native_indexer_plan.metal:525-535 (BF16 add), in one launch.  A workgroup
// has one wavefront per slot (the k routed slots, then the shared expert)
// and owns `rows_per_wg` output rows h: each wavefront loads its slot's
// hidden vector once and issues the loads of all its rows in batches of 8
// before reducing any, parks T(dot) in LDS, and the first rows_per_wg lanes
// then form out[h] = T( T(sum_s T(down[s,h]) * score[s]) + T(shared[h]) ),
// summed in slot order (and T(residual[h] + that) with a residual).
template <int VB, int CH, bool HW>
__device__ __forceinline__ void down_rows(const DownArgs& a, const uint8_t* __restrict__ w,
                                          const float* __restrict__ s, float* parked_row, int slot, int64_t h0,
                                          int64_t h_end, int g, int lane) {
  const int64_t K = a.intermediate;
  const int64_t SC = (K + kBlock - 1) / kBlock;
  const RowWalk walk = row_walk<VB>(lane, g);
  XRaw<VB, CH> raw;
  load_x_raw<VB, CH>(a.hidden_in + static_cast<int64_t>(slot) * K, lane, raw);
  XSlice<VB, CH, HW> xs;
  bool packed = false;
  for (int64_t hb = h0; hb < h_end; hb += 8) {
    WRow<VB, CH> rowsv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (hb + j < h_end)
        load_wrow_walk<VB, CH>(rowsv[j], w + group_row_base(hb + j, K, g), s + ((hb + j) >> 7) * SC, lane, walk);
    if (!packed) {
      pack_x_raw<VB, CH, HW>(raw, xs);
      packed = true;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (hb + j < h_end) {
        const float t = wave_sum(wrow_partial<VB, CH, HW>(rowsv[j], xs));
        if (lane == 0) parked_row[hb + j - h0] = bf16_round(t);
      }
    }
  }
}

template <int VB, int CH>
__global__ __launch_bounds__(64 * (kMaxTopK + 1)) void down_reduce_kernel(DownArgs a) {
  __shared__ float parked[kMaxTopK + 1][kMaxDownRowsPerWg];
  const int lane = threadIdx.x & 63;
  const int slot = threadIdx.x >> 6;
  const int64_t h0 = static_cast<int64_t>(blockIdx.x) * a.rows_per_wg;
  const int64_t K = a.intermediate;
  const int64_t SC = (K + kBlock - 1) / kBlock;
  const int64_t SH = (a.hidden + kBlock - 1) / kBlock;
  const int64_t h_end = (h0 + a.rows_per_wg < a.hidden) ? h0 + a.rows_per_wg : a.hidden;

  const uint8_t* w = nullptr;
  const float* s = nullptr;
  bool ok = true;
  if (slot < a.top_k) {
    const int32_t e = a.expert_ids[slot];
    if (bad_expert(e, a.experts)) {
      ok = false;
      if (lane == 0) atomicOr(a.error_flag, 1);
    } else {
      w = a.down_weight + static_cast<int64_t>(e) * a.hidden * K;
      s = a.down_scale + static_cast<int64_t>(e) * SH * SC;
    }
  } else {
    w = a.shared_down_weight;
    s = a.shared_down_scale;
  }
  if (ok) {
    const int32_t* flag = slot < a.top_k ? a.routed_flags : a.shared_flags;
    const int g = slot < a.top_k ? a.bank_group_log2 : 0;
    if (hw_decode_ok(flag))
      down_rows<VB, CH, true>(a, w, s, parked[slot], slot, h0, h_end, g, lane);
    else
      down_rows<VB, CH, false>(a, w, s, parked[slot], slot, h0, h_end, g, lane);
  } else {
    for (int64_t h = h0 + lane; h < h_end; h += 64) parked[slot][h - h0] = __builtin_nanf("");
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < h_end - h0) {
    float total = 0.0f;
    for (int sl = 0; sl < a.top_k; ++sl) total = __fadd_rn(total, __fmul_rn(parked[sl][t], a.scores[sl]));
    float result = bf16_round(total);
    if (a.shared_down_weight != nullptr) result = __fadd_rn(result, parked[a.top_k][t]);
    if (a.residual != nullptr) {
      // decoder residual x + T(moe(x)): the MoE output is rounded first, as
      // it is when the decoder layer adds it outside the MoE module
      result = __fadd_rn(bf16_to_f32(a.residual[h0 + t]), bf16_round(result));
    }
    a.out[h0 + t] = f32_to_bf16(result);
  }
}

// ----------------------------------------------------------------- router --
//
// patch.py:133: logits = x_f32 . W_f32^T in FP32, one workgroup per (expert
// row, token) (16 KB of weights for H = 4096), no cross-workgroup traffic;
// selection runs in the consumer (topk_kernel).  The one-token router, and
// the many-token router for shapes the BF16-MFMA form does not take.
__global__ __launch_bounds__(256) void router_logits_kernel(RouterArgs a) {
  __shared__ float partial[4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t e = blockIdx.x;
  const int64_t tok = blockIdx.y;
  const float* w = a.weight + e * a.hidden;
  const uint16_t* x = a.x + tok * a.hidden;
  float acc = 0.0f;
  if ((a.hidden & 3) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 7) == 0 &&
      (reinterpret_cast<uintptr_t>(a.weight) & 15) == 0) {
    for (int64_t k = 4 * static_cast<int64_t>(threadIdx.x); k < a.hidden; k += 1024) {
      float4 wv = *reinterpret_cast<const float4*>(w + k);
      uint2 xv = *reinterpret_cast<const uint2*>(x + k);
      acc = fmaf(__uint_as_float(xv.x << 16), wv.x, acc);
      acc = fmaf(__uint_as_float(xv.x & 0xffff0000u), wv.y, acc);
      acc = fmaf(__uint_as_float(xv.y << 16), wv.z, acc);
      acc = fmaf(__uint_as_float(xv.y & 0xffff0000u), wv.w, acc);
    }
  } else {
    for (int64_t k = threadIdx.x; k < a.hidden; k += 256) acc = fmaf(bf16_to_f32(x[k]), w[k], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) partial[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) a.logits_out[tok * a.experts + e] = (partial[0] + partial[1]) + (partial[2] + partial[3]);
}

// ---------------------------------------------------------- plain GEMV ----
//
// fp8.py:41-72 `block_fp8_linear` for one activation row: y[n] = T(sum_k
// x[k] * LUT[w[n,k]] * s[n/128, k/128]).  Wave w of a workgroup streams
// rows [rows_per_wave * (4 * block + w), ...).
template <int VB, int CH, bool HW>
__device__ __forceinline__ void gemv_rows(const GemvArgs& a, int64_t n0, int64_t n_end, int lane) {
  const int64_t K = a.K;
  const int64_t SC = (K + kBlock - 1) / kBlock;
  XRaw<VB, CH> raw;
  load_x_raw<VB, CH>(a.x, lane, raw);
  XSlice<VB, CH, HW> xs;
  bool packed = false;
  int64_t n = n0;
  for (; n + 3 < n_end; n += 4) {
    WRow<VB, CH> w0, w1, w2, w3;
    load_wrow<VB, CH>(w0, a.weight + n * K, a.scale + (n >> 7) * SC, lane);
    load_wrow<VB, CH>(w1, a.weight + (n + 1) * K, a.scale + ((n + 1) >> 7) * SC, lane);
    load_wrow<VB, CH>(w2, a.weight + (n + 2) * K, a.scale + ((n + 2) >> 7) * SC, lane);
    load_wrow<VB, CH>(w3, a.weight + (n + 3) * K, a.scale + ((n + 3) >> 7) * SC, lane);
    if (!packed) {
      pack_x_raw<VB, CH, HW>(raw, xs);
      packed = true;
    }
    float t0 = wave_sum(wrow_partial<VB, CH, HW>(w0, xs));
    float t1 = wave_sum(wrow_partial<VB, CH, HW>(w1, xs));
    float t2 = wave_sum(wrow_partial<VB, CH, HW>(w2, xs));
    float t3 = wave_sum(wrow_partial<VB, CH, HW>(w3, xs));
    if (lane == 0) {
      a.y[n] = f32_to_bf16(t0);
      a.y[n + 1] = f32_to_bf16(t1);
      a.y[n + 2] = f32_to_bf16(t2);
      a.y[n + 3] = f32_to_bf16(t3);
    }
  }
  for (; n < n_end; ++n) {
    WRow<VB, CH> w0;
    load_wrow<VB, CH>(w0, a.weight + n * K, a.scale + (n >> 7) * SC, lane);
    if (!packed) {
      pack_x_raw<VB, CH, HW>(raw, xs);
      packed = true;
    }
    float t0 = wave_sum(wrow_partial<VB, CH, HW>(w0, xs));
    if (lane == 0) a.y[n] = f32_to_bf16(t0);
  }
}

template <int VB, int CH>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * a.rows_per_wave;
  if (n0 >= a.N) return;
  const int64_t K = a.K;
  const int64_t SC = (K + kBlock - 1) / kBlock;
  const int64_t n_end = (n0 + a.rows_per_wave < a.N) ? n0 + a.rows_per_wave : a.N;
  if (hw_decode_ok(a.flags)) gemv_rows<VB, CH, true>(a, n0, n_end, lane);
  else gemv_rows<VB, CH, false>(a, n0, n_end, lane);
}

// Wide rows (K a multiple of 4096 above 8192, e.g. an attention output
// projection of 16384): the workgroup holds one wavefront per 4096-wide K
// part; each streams its part of a batch of up to 4 rows exactly as
// gemv_rows does, lane 0 leaves the part's sums in LDS and the first
// threads add the parts in part order (deterministic) and store the row.
// Workgroup g covers rows [rows_per_wave * g, ...).
template <bool HW>
__device__ __forceinline__ void gemv_split_rows(const GemvArgs& a, int parts, int lane, int part) {
  constexpr int VB = 16, CH = 4;
  __shared__ float sums[kMaxGemvParts][4];
  const int64_t K = a.K;
  const int64_t SC = K / kBlock;
  const int64_t kp = static_cast<int64_t>(part) * 64 * VB * CH;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * a.rows_per_wave;
  const int64_t n_end = n0 + a.rows_per_wave < a.N ? n0 + a.rows_per_wave : a.N;
  XRaw<VB, CH> raw;
  load_x_raw<VB, CH>(a.x + kp, lane, raw);
  XSlice<VB, CH, HW> xs;
  pack_x_raw<VB, CH, HW>(raw, xs);
  for (int64_t n = n0; n < n_end; n += 4) {  // uniform across the workgroup: every wave reaches each barrier
    const int rows = n_end - n < 4 ? static_cast<int>(n_end - n) : 4;
    WRow<VB, CH> w[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = n + (r < rows ? r : 0);
      load_wrow<VB, CH>(w[r], a.weight + row * K + kp, a.scale + (row >> 7) * SC + kp / kBlock, lane);
    }
    float t[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) t[r] = wave_sum(wrow_partial<VB, CH, HW>(w[r], xs));
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sums[part][r] = t[r];
    }
    __syncthreads();
    if (threadIdx.x < rows) {
      float total = sums[0][threadIdx.x];
      for (int q = 1; q < parts; ++q) total += sums[q][threadIdx.x];
      a.y[n + threadIdx.x] = f32_to_bf16(total);
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(64 * kMaxGemvParts) void gemv_split_kernel(GemvArgs a, int parts) {
  const int lane = threadIdx.x & 63;
  const int part = threadIdx.x >> 6;
  if (hw_decode_ok(a.flags)) gemv_split_rows<true>(a, parts, lane, part);
  else gemv_split_rows<false>(a, parts, lane, part);
}

// ------------------------------------------------------ per-token top-k ----
// Every partial and the bias are requested before the first partial is added
// (splits <= 16); the selection is wave_topk_words_sorted over the token's
// (sigmoid, key) words, the order and arithmetic of wave_topk_regs.
template <int P>
__device__ __forceinline__ void topk_token_partials(const TopkArgs& a, int64_t t, int lane, TopkScratch& scratch) {
  const int splits = a.splits > 1 ? a.splits : 1;
  float part[P][kMaxRouterSplits];
  float bias[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int64_t c = lane + 64 * i;
    bias[i] = c < a.experts ? a.bias[c] : 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxRouterSplits; ++s)
      part[i][s] = s < splits && c < a.experts ? a.logits[s * a.split_stride + t * a.experts + c] : 0.0f;
  }
  unsigned long long wd[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    float v = part[i][0];
#pragma unroll
    for (int s = 1; s < kMaxRouterSplits; ++s)
      if (s < splits) v += part[i][s];
    const int64_t c = lane + 64 * i;
    wd[i] = 0ull;
    if (c < a.experts) {
      const float sg = router_sigmoid(v);
      const uint32_t key = max(orderable_bits(__fadd_rn(sg, bias[i])), 1u);
      wd[i] = (static_cast<unsigned long long>(__float_as_uint(sg)) << 32) | key;
    }
  }
  wave_topk_words_sorted<P>(wd, a.top_k, a.routed_scaling_factor, a.norm_topk_prob, lane, a.ids_out + t * a.top_k,
                            a.scores_out + t * a.top_k, scratch, GroupLimit{a.n_group, a.topk_group}, a.experts);
}

// kPartials: logits come as a.splits partial planes; otherwise whole.
template <bool kPartials>
__global__ __launch_bounds__(256) void topk_kernel(TopkArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= a.tokens) return;
  if constexpr (kPartials) {
    __shared__ TopkScratch scratch[4];
    TopkScratch& sc = scratch[threadIdx.x >> 6];
    if (a.experts <= 128) topk_token_partials<2>(a, t, lane, sc);
    else if (a.experts <= 320) topk_token_partials<5>(a, t, lane, sc);
    else topk_token_partials<kMaxRouterExperts / 64>(a, t, lane, sc);
  } else {
    wave_topk(a.logits + t * a.experts, a.bias, a.experts, a.top_k, a.routed_scaling_factor, a.norm_topk_prob,
              lane, a.ids_out + t * a.top_k, a.scores_out + t * a.top_k, GroupLimit{a.n_group, a.topk_group});
  }
}

// ------------------------------------------------------- generic path ----
//
// Any-shape block-FP8 linear (fp8.py:41-116 / packed.py:304-387 semantics)
// for odd widths that the vector fast path cannot tile: groups g select an
// expert (optional), the activation rows of the group are staged in LDS as
// FP32, and each wavefront reduces one output row per step with byte loads.
__global__ __launch_bounds__(256) void linear_generic_kernel(GenericLinearArgs a) {
  extern __shared__ float xs[];  // [tile_rows][K], tile_rows <= kGenericRows
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t g = blockIdx.y;
  const int64_t n_base = static_cast<int64_t>(blockIdx.x) * 4 * a.rows_per_wave;
  const int64_t K = a.K;
  const uint8_t* w = a.weight;
  const float* s = a.scale;
  if (a.expert_ids != nullptr) {
    int32_t e = a.expert_ids[g];
    if (bad_expert(e, a.experts)) {
      if (threadIdx.x == 0) atomicOr(a.error_flag, 1);
      for (int64_t m = 0; m < a.M; ++m)
        for (int64_t n = n_base + threadIdx.x; n < n_base + 4 * a.rows_per_wave && n < a.N; n += 256)
          a.y[g * a.y_group_stride + m * a.y_row_stride + n] = 0x7FC0u;
      return;
    }
    w += static_cast<int64_t>(e) * a.w_expert_stride;
    s += static_cast<int64_t>(e) * a.s_expert_stride;
  }
  s += a.s_row_offset * a.s_cols;
  const uint16_t* xg = a.x + g * a.x_group_stride;
  for (int64_t m0 = 0; m0 < a.M; m0 += a.tile_rows) {
    const int mt = static_cast<int>((a.M - m0) < a.tile_rows ? (a.M - m0) : a.tile_rows);
    __syncthreads();
    for (int64_t i = threadIdx.x; i < mt * K; i += 256) {
      int64_t m = i / K, k = i % K;
      xs[i] = bf16_to_f32(xg[(m0 + m) * a.x_row_stride + k]);
    }
    __syncthreads();
    for (int rr = 0; rr < a.rows_per_wave; ++rr) {
      const int64_t n = n_base + static_cast<int64_t>(wave) * a.rows_per_wave + rr;
      if (n >= a.N) break;
      float acc[kGenericRows];
#pragma unroll
      for (int m = 0; m < kGenericRows; ++m) acc[m] = 0.0f;
      const uint8_t* wr = w + group_row_base(a.w_row_offset + n, K, a.w_group_log2);
      const float* sr = s + (n >> 7) * a.s_cols;
      for (int64_t k = lane; k < K; k += 64) {
        uint32_t b = wr[group_col(k, a.w_group_log2)];
        float wv = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(
                       ((b & 0x7Fu) << 7) | ((b & 0x80u) << 8)))) * 256.0f * sr[k >> 7];
#pragma unroll
        for (int m = 0; m < kGenericRows; ++m)
          if (m < mt) acc[m] = fmaf(xs[m * K + k], wv, acc[m]);
      }
#pragma unroll
      for (int m = 0; m < kGenericRows; ++m) {
        float t = wave_sum(acc[m]);
        if (lane == 0 && m < mt) a.y[g * a.y_group_stride + (m0 + m) * a.y_row_stride + n] = f32_to_bf16(t);
      }
    }
  }
}

// packed.py:146-163 / grouped_fp8.py:265-270 elementwise SwiGLU on BF16
// projections (gate row-block / up row-block with independent strides).
// Each thread takes elements 2 t and 2 t + 1 (the last one twice when the
// count is odd) through swiglu_mlx_straight2, the form of the grouped GEMM
// epilogues, and recomputes them with swiglu_mlx where that form does not
// apply, so this entry point pins that form on whatever inputs it is given.
__global__ void swiglu_kernel(SwigluArgs a) {
  const int64_t n = a.rows * a.cols;
  const int64_t i0 = 2 * (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x);
  if (i0 >= n) return;
  const int64_t i1 = i0 + 1 < n ? i0 + 1 : i0;
  const int64_t r0 = i0 / a.cols, c0 = i0 % a.cols, r1 = i1 / a.cols, c1 = i1 % a.cols;
  const float g0 = bf16_to_f32(a.gate[r0 * a.gate_row_stride + c0]);
  const float u0 = bf16_to_f32(a.up[r0 * a.up_row_stride + c0]);
  const float g1 = bf16_to_f32(a.gate[r1 * a.gate_row_stride + c1]);
  const float u1 = bf16_to_f32(a.up[r1 * a.up_row_stride + c1]);
  SwigluCheck check;
  uint32_t h = swiglu_mlx_straight2(g0, u0, g1, u1, a.limit, check);
  if (!swiglu_straight_ok(check, a.limit))
    h = swiglu_mlx(g0, u0, a.limit) | static_cast<uint32_t>(swiglu_mlx(g1, u1, a.limit)) << 16;
  a.out[r0 * a.out_row_stride + c0] = static_cast<uint16_t>(h);
  if (i1 != i0) a.out[r1 * a.out_row_stride + c1] = static_cast<uint16_t>(h >> 16);
}

// swiglu_mlx with every rounding point kept (the routed-stage diagnostic):
// gate/up rows of `cols` at row strides gate_row_stride / up_row_stride ->
// sigma = T(sigmoid(g')), silu = T(g' * sigma), hidden = T(silu * u') with
// g' = T(min(g, L)), u' = T(clip(u, -L, L)) (packed.py:146-163), [rows, cols].
__global__ void swiglu_stages_kernel(SwigluArgs a, uint16_t* sigma_out, uint16_t* silu_out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= a.rows * a.cols) return;
  const int64_t r = i / a.cols, c = i % a.cols;
  const float g = bf16_to_f32(a.gate[r * a.gate_row_stride + c]);
  const float u = bf16_to_f32(a.up[r * a.up_row_stride + c]);
  float gv = (g < a.limit) ? g : a.limit;
  if (isnan(g)) gv = g;
  float uv = fminf(fmaxf(u, -a.limit), a.limit);
  if (isnan(u)) uv = u;
  const uint16_t ga = f32_to_bf16(gv);
  const float sigma = sigmoid_mlx_bf16(ga);
  const float silu = bf16_round(bf16_to_f32(ga) * sigma);
  sigma_out[r * a.out_row_stride + c] = f32_to_bf16(sigma);
  silu_out[r * a.out_row_stride + c] = f32_to_bf16(silu);
  a.out[r * a.out_row_stride + c] = f32_to_bf16(silu * bf16_round(uv));
}

// packed.py:168-179: out[h] = T(sum_s float(down[s,h]) * score[s]), FP32
// products summed in slot order; optional BF16 add of `addend`.
__global__ void weighted_reduction_kernel(WeightedReductionArgs a) {
  const int64_t h = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (h >= a.H) return;
  float total = 0.0f;
  for (int s = 0; s < a.top_k; ++s)
    total = __fadd_rn(total, __fmul_rn(bf16_to_f32(a.down[static_cast<int64_t>(s) * a.H + h]), a.scores[s]));
  float r = bf16_round(total);
  if (a.addend != nullptr) r = __fadd_rn(r, bf16_to_f32(a.addend[h]));
  a.out[h] = f32_to_bf16(r);
}

// The MLX BF16 sigmoid of the SwiGLU epilogues on its own, in the form they
// evaluate (diagnostic entry point; lets a test pin the device arithmetic
// against the reference's exhaustive sweep and the oracle over every BF16
// pattern).
__global__ void sigmoid_bf16_kernel(const uint16_t* g, uint16_t* out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f32_to_bf16(sigmoid_mlx_bf16_fast(g[i]));
}

__global__ void add_bf16_kernel(const uint16_t* a, const uint16_t* b, uint16_t* out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f32_to_bf16(__fadd_rn(bf16_to_f32(a[i]), bf16_to_f32(b[i])));
}

// --------------------------------------------------------------- launch ---

template <int VB, int CH>
static hipError_t launch_gate_up_t(const GateUpArgs& a, hipStream_t st) {
  int64_t rows_per_wg = 4 * static_cast<int64_t>(a.rows_per_wave);
  int64_t blocks = static_cast<int64_t>(a.top_k) * a.wgs_per_slot;
  if (a.shared_gate_weight != nullptr) blocks += (a.shared_intermediate + rows_per_wg - 1) / rows_per_wg;
  hipLaunchKernelGGL((gate_up_swiglu_kernel<VB, CH>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int VB, int CH>
static hipError_t launch_down_t(const DownArgs& a, hipStream_t st) {
  int64_t blocks = (a.hidden + a.rows_per_wg - 1) / a.rows_per_wg;
  const unsigned threads = 64u * static_cast<unsigned>(a.top_k + (a.shared_down_weight != nullptr ? 1 : 0));
  hipLaunchKernelGGL((down_reduce_kernel<VB, CH>), dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, st, a);
  return hipGetLastError();
}

// Reduction widths the vector fast path is instantiated for: K = 64*VB*CH.
bool fast_width_supported(int64_t K) {
  return K == 1024 || K == 2048 || K == 3072 || K == 4096 || K == 5120 || K == 6144 || K == 7168 ||
         K == 8192 || K == 512 || K == 1536;
}

hipError_t launch_gate_up(const GateUpArgs& a, hipStream_t st) {
  switch (a.hidden) {
    case 512: return launch_gate_up_t<8, 1>(a, st);
    case 1024: return launch_gate_up_t<16, 1>(a, st);
    case 1536: return launch_gate_up_t<8, 3>(a, st);
    case 2048: return launch_gate_up_t<16, 2>(a, st);
    case 3072: return launch_gate_up_t<16, 3>(a, st);
    case 4096: return launch_gate_up_t<16, 4>(a, st);
    case 5120: return launch_gate_up_t<16, 5>(a, st);
    case 6144: return launch_gate_up_t<16, 6>(a, st);
    case 7168: return launch_gate_up_t<16, 7>(a, st);
    case 8192: return launch_gate_up_t<16, 8>(a, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_down(const DownArgs& a, hipStream_t st) {
  switch (a.intermediate) {
    case 512: return launch_down_t<8, 1>(a, st);
    case 1024: return launch_down_t<16, 1>(a, st);
    case 1536: return launch_down_t<8, 3>(a, st);
    case 2048: return launch_down_t<16, 2>(a, st);
    case 3072: return launch_down_t<16, 3>(a, st);
    case 4096: return launch_down_t<16, 4>(a, st);
    case 5120: return launch_down_t<16, 5>(a, st);
    case 6144: return launch_down_t<16, 6>(a, st);
    case 7168: return launch_down_t<16, 7>(a, st);
    case 8192: return launch_down_t<16, 8>(a, st);
    default: return hipErrorInvalidValue;
  }
}

template <int VB, int CH>
static hipError_t launch_gemv_t(const GemvArgs& a, hipStream_t st) {
  int64_t rows_per_wg = 4 * static_cast<int64_t>(a.rows_per_wave);
  hipLaunchKernelGGL((gemv_kernel<VB, CH>), dim3(static_cast<unsigned>((a.N + rows_per_wg - 1) / rows_per_wg)),
                     dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_gemv(const GemvArgs& a, hipStream_t st) {
  switch (a.K) {
    case 512: return launch_gemv_t<8, 1>(a, st);
    case 1024: return launch_gemv_t<16, 1>(a, st);
    case 1536: return launch_gemv_t<8, 3>(a, st);
    case 2048: return launch_gemv_t<16, 2>(a, st);
    case 3072: return launch_gemv_t<16, 3>(a, st);
    case 4096: return launch_gemv_t<16, 4>(a, st);
    case 5120: return launch_gemv_t<16, 5>(a, st);
    case 6144: return launch_gemv_t<16, 6>(a, st);
    case 7168: return launch_gemv_t<16, 7>(a, st);
    case 8192: return launch_gemv_t<16, 8>(a, st);
    default: return hipErrorInvalidValue;
  }
}

bool split_width_supported(int64_t K) { return K > 8192 && K % 4096 == 0 && K / 4096 <= kMaxGemvParts; }

hipError_t launch_gemv_split(const GemvArgs& a, hipStream_t st) {
  if (!split_width_supported(a.K) || a.rows_per_wave < 1) return hipErrorInvalidValue;
  const int parts = static_cast<int>(a.K / 4096);
  hipLaunchKernelGGL(gemv_split_kernel, dim3(static_cast<unsigned>((a.N + a.rows_per_wave - 1) / a.rows_per_wave)),
                     dim3(static_cast<unsigned>(64 * parts)), 0, st, a, parts);
  return hipGetLastError();
}

hipError_t launch_topk(const TopkArgs& a, hipStream_t st) {
  if (a.tokens == 0) return hipSuccess;
  if (a.splits > kMaxRouterSplits) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>((a.tokens + 3) / 4));
  if (a.splits > 1) hipLaunchKernelGGL(topk_kernel<true>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(topk_kernel<false>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_router(const RouterArgs& a, hipStream_t st) {
  const unsigned tokens = a.tokens > 1 ? static_cast<unsigned>(a.tokens) : 1u;
  hipLaunchKernelGGL(router_logits_kernel, dim3(static_cast<unsigned>(a.experts), tokens), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_linear_generic(const GenericLinearArgs& a, hipStream_t st) {
  int64_t rows_per_wg = 4 * static_cast<int64_t>(a.rows_per_wave);
  dim3 grid(static_cast<unsigned>((a.N + rows_per_wg - 1) / rows_per_wg), static_cast<unsigned>(a.G));
  size_t lds = sizeof(float) * static_cast<size_t>(a.tile_rows) * static_cast<size_t>(a.K);
  hipLaunchKernelGGL(linear_generic_kernel, grid, dim3(256), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_swiglu_stages(const SwigluArgs& a, uint16_t* sigma, uint16_t* silu, hipStream_t st) {
  const int64_t n = a.rows * a.cols;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_stages_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, a, sigma,
                     silu);
  return hipGetLastError();
}

hipError_t launch_swiglu(const SwigluArgs& a, hipStream_t st) {
  int64_t n = a.rows * a.cols;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3(static_cast<unsigned>(((n + 1) / 2 + 255) / 256)), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_weighted_reduction(const WeightedReductionArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(weighted_reduction_kernel, dim3(static_cast<unsigned>((a.H + 255) / 256)), dim3(256), 0,
                     st, a);
  return hipGetLastError();
}

hipError_t launch_sigmoid_bf16(const uint16_t* g, uint16_t* out, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(sigmoid_bf16_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, g, out, n);
  return hipGetLastError();
}

hipError_t launch_add_bf16(const uint16_t* a, const uint16_t* b, uint16_t* out, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(add_bf16_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, a, b, out,
                     n);
  return hipGetLastError();
}

}  // namespace glm53
