// Batch-1 decode of one MoE layer in three launches, arranged so that every
// launch streams weights from its first cycle to its last:
//
//   1. router + shared gate/up: one wavefront per router logit (FP32, 16 KB
//      row, all loads in flight at once) and, in the same grid, the shared
//      expert's gate/up/SwiGLU rows, so the shared expert's 12.6 MB stream
//      beside the router's latency-bound rows.
//      The last router workgroup to arrive selects the top-k, so the routed
//      launch starts from the ids.
//   2. routed gate/up + shared down: the k selected experts' gate/up rows as
//      one flat list of (slot, row) units split evenly over a grid sized to
//      the resident capacity of the GPU (every CU gets the same bytes), with
//      two units of loads (weights and their block scales) in flight per
//      wavefront; beside them the shared expert's down rows.
//   3. routed down + reduction: one workgroup per 16 output rows, one
//      wavefront per slot; each half-wavefront owns a row so every lane reads
//      16-byte chunks, all 16 rows' loads are issued before the first is
//      reduced, and the ordered FP32 slot sum, the shared add and the
//      residual finish in the same workgroup.
//
// Arithmetic (packed.py:100-179, 181-235; fp8.py:254-299; patch.py:131-142;
// native_indexer_plan.metal:525-535): E4M3 weights decoded in registers,
// FP32 accumulation (v_dot2 over exact FP16 activation pairs, block scale
// per 128-column chunk), T(gate), T(up), MLX BF16 SwiGLU, T(down) per slot,
// out = T(T(sum_s T(down_s) * w_s) + T(shared)) summed in slot order, and
// T(residual + out) when a residual is given.
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "stream_gemv.h"

namespace glm53 {

namespace {

// Totals of the two half-wavefronts (lanes 0-31 and 32-63).
__device__ __forceinline__ void half_sums(float v, float& lo, float& hi) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  lo = a + b;
  hi = c + d;
}

// A half-wavefront's activation slice for a reduction of length 512 * CH:
// half-lane l (0..31) holds elements 16 l + 512 c .. + 15, c < CH, as exact
// FP16 pairs (paired as the weight decode wants them).
template <int CH, bool HW>
struct HalfSlice {
  uint32_t p[CH][8];
  float factor;
};

template <int CH>
struct HalfRaw {
  uint4 q[CH][2];
};

template <int CH>
__device__ __forceinline__ void load_half_raw(const uint16_t* __restrict__ x, int hl, HalfRaw<CH>& raw) {
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < 2; ++i) raw.q[c][i] = *reinterpret_cast<const uint4*>(x + 16 * hl + 512 * c + 8 * i);
}

template <int CH, bool HW>
__device__ __forceinline__ void pack_half_raw(const HalfRaw<CH>& raw, HalfSlice<CH, HW>& xs) {
  float v[CH][16];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t w[4] = {raw.q[c][i].x, raw.q[c][i].y, raw.q[c][i].z, raw.q[c][i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[c][8 * i + 2 * j] = __uint_as_float(w[j] << 16);
        v[c][8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    }
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[c][i]));
  // one shift for the whole wavefront keeps both halves' partials comparable
  amax = wave_max(amax);
  const int shift = f16_shift_for(amax);
  const float down = ldexpf(1.0f, -shift);
  xs.factor = ldexpf(1.0f, (HW ? 0 : 8) + shift);
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (HW) {
        xs.p[c][2 * j] = pack_f16x2(v[c][4 * j] * down, v[c][4 * j + 1] * down);
        xs.p[c][2 * j + 1] = pack_f16x2(v[c][4 * j + 2] * down, v[c][4 * j + 3] * down);
      } else {
        xs.p[c][2 * j] = pack_f16x2(v[c][4 * j] * down, v[c][4 * j + 2] * down);
        xs.p[c][2 * j + 1] = pack_f16x2(v[c][4 * j + 1] * down, v[c][4 * j + 3] * down);
      }
    }
}

// Partial dot of one 16-byte weight chunk with chunk c of the slice.
template <int CH, bool HW>
__device__ __forceinline__ float half_chunk_dot(const u32x4& w, const HalfSlice<CH, HW>& xs, int c) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (HW) {
      const half2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[j], 1.0f, false);
      const half2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[j], 1.0f, true);
      acc = __builtin_amdgcn_fdot2(lo, __builtin_bit_cast(half2_t, xs.p[c][2 * j]), acc, false);
      acc = __builtin_amdgcn_fdot2(hi, __builtin_bit_cast(half2_t, xs.p[c][2 * j + 1]), acc, false);
    } else {
      acc = dot4_e4m3(w[j], xs.p[c][2 * j], xs.p[c][2 * j + 1], acc);
    }
  }
  return acc;
}

// Rows [h0, h0 + 2 * PAIRS) of W [*, K = 512 CH] (E4M3 in row groups of
// 2^g rows, common.h, with 128 x 128 scales, SC = K / 128 per scale row; the
// rows must lie in one 128-row scale block): half-wavefront `half` owns rows
// h0 + 2 j + half.
// issue() puts every load in flight (weights and the block's scales in one
// batch); finish() reduces, returning T(dot) of pair j in t[j][half] (valid
// on lanes 0 and 32).
template <int CH, int PAIRS>
struct HalfRows {
  u32x4 q[PAIRS][CH];
  float sc[CH];

  __device__ __forceinline__ void issue(const uint8_t* __restrict__ w, const float* __restrict__ s, int64_t h0,
                                        int lane, int g) {
    constexpr int64_t K = 512 * CH;
    constexpr int64_t SC = K / 128;
    const int half = lane >> 5, hl = lane & 31;
    // half-lane hl's 16 bytes of chunk c: column 16 hl + 512 c
    const int64_t lane_off = group_col(16 * hl, g), stride = int64_t{512} << g;
#pragma unroll
    for (int j = 0; j < PAIRS; ++j) {
      const uint8_t* row = w + group_row_base(h0 + 2 * j + half, K, g) + lane_off;
#pragma unroll
      for (int c = 0; c < CH; ++c)
        q[j][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + c * stride));
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) sc[c] = s[(h0 >> 7) * SC + ((16 * hl + 512 * c) >> 7)];
  }

  template <bool HW>
  __device__ __forceinline__ void finish(const HalfSlice<CH, HW>& xs, float (&t)[PAIRS][2]) const {
#pragma unroll
    for (int j = 0; j < PAIRS; ++j) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c) acc += half_chunk_dot<CH, HW>(q[j][c], xs, c) * sc[c];
      float lo, hi;
      half_sums(acc * xs.factor, lo, hi);
      t[j][0] = bf16_round(lo);
      t[j][1] = bf16_round(hi);
    }
  }
};

// One gate/up unit (row r of the gate and up halves) loaded into registers.
template <int VB, int CH>
struct GateUpUnit {
  WRow<VB, CH> g, u;
};

}  // namespace

// ---------------------------------------------------------------- launch 1

// Router word of expert e (patch.py:131-142): the FP32 logit x_f32 . W_f32^T
// (lane l covers columns 4 l + 256 j; a batch's loads are all in flight at
// once), its sigmoid s and the selection key, the order-preserving image of
// the FP32 sum s + bias (at least 1, so 0 marks an absent expert), published
// as one word s_bits << 32 | key by a read-modify-write, performed where every
// workgroup's atomics meet, so the selecting workgroup reads it back without
// fences and does no per-expert arithmetic itself.
template <int kCols>
__device__ __forceinline__ void router_word(const StepArgs& a, int64_t e, int lane) {
  constexpr int kChunks = kCols / 256;
  constexpr int kBatch = kChunks <= 16 ? kChunks
                         : kChunks % 16 == 0 ? 16
                         : kChunks % 14 == 0 ? 14
                         : kChunks % 12 == 0 ? 12
                                             : 8;
  static_assert(kCols % 256 == 0 && kChunks % kBatch == 0, "router row must split into whole batches");
  const float* w = a.router_weight + e * kCols;
  const float bias = a.router_bias[e];
  float acc = 0.0f;
#pragma unroll
  for (int j0 = 0; j0 < kChunks; j0 += kBatch) {
    u32x4 wv[kBatch];
    uint2 xv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      wv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + 256 * (j0 + j) + 4 * lane));
      xv[j] = *reinterpret_cast<const uint2*>(a.x + 256 * (j0 + j) + 4 * lane);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      acc = fmaf(__uint_as_float(xv[j].x << 16), __uint_as_float(wv[j][0]), acc);
      acc = fmaf(__uint_as_float(xv[j].x & 0xffff0000u), __uint_as_float(wv[j][1]), acc);
      acc = fmaf(__uint_as_float(xv[j].y << 16), __uint_as_float(wv[j][2]), acc);
      acc = fmaf(__uint_as_float(xv[j].y & 0xffff0000u), __uint_as_float(wv[j][3]), acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    const float sg = router_sigmoid(acc);
    const uint32_t key = max(orderable_bits(__fadd_rn(sg, bias)), 1u);
    (void)atomicExch(a.route_words + e, (static_cast<unsigned long long>(__float_as_uint(sg)) << 32) | key);
  }
}

template <int VBH, int CHH>
__global__ __launch_bounds__(256) void step_router_shared_kernel(StepArgs a) {
  __shared__ int s_last;
  __shared__ int32_t s_ids[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  __shared__ TopkScratch s_topk;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int bid = blockIdx.x;
  if (bid < a.router_wgs) {
    // ---- router logit of expert e = 4 bid + wave
    const int64_t e = static_cast<int64_t>(bid) * 4 + wave;
    if (e < a.experts) router_word<VBH * CHH * 64>(a, e, lane);
    // the last workgroup to arrive selects: every logit is in place
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(a.router_count, 1u) == static_cast<unsigned>(a.router_wgs - 1);
    __syncthreads();
    if (s_last && wave == 0) {
      unsigned long long wd[5];
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        const int64_t c = lane + 64 * i;
        wd[i] = c < a.experts ? atomicOr(a.route_words + c, 0ull) : 0ull;
      }
      wave_topk_words_sorted<5>(wd, a.top_k, a.routed_scaling_factor, a.norm_topk_prob, lane, s_ids, s_w, s_topk,
                                GroupLimit{a.n_group, a.topk_group}, a.experts);
      if (lane < a.top_k) {
        a.ids[lane] = s_ids[lane];
        a.scores[lane] = s_w[lane];
      }
      if (lane == 0) (void)atomicExch(a.router_count, 0u);  // ready for the next launch
    }
    return;
  }
  // ---- shared gate/up rows (packed.py:181-235)
  const int64_t r0 = (static_cast<int64_t>(bid - a.router_wgs) * 4 + wave) * a.shared_rows_per_wave;
  if (r0 >= a.intermediate) return;
  const int64_t r_end = r0 + a.shared_rows_per_wave < a.intermediate ? r0 + a.shared_rows_per_wave : a.intermediate;
  const int64_t K = a.hidden, SC = K / kBlock;
  uint16_t* out = a.hidden_act + static_cast<int64_t>(a.top_k) * a.intermediate;
  if (a.router_wgs > 0)
    for (int i = 0; i < a.shared_delay; ++i) __builtin_amdgcn_s_sleep(8);
  XRaw<VBH, CHH> raw;
  load_x_raw<VBH, CHH>(a.x, lane, raw);
  auto run = [&](auto hw) {
    constexpr bool HW = decltype(hw)::value;
    XSlice<VBH, CHH, HW> xs;
    bool packed = false;
    for (int64_t r = r0; r < r_end; r += 2) {
      const bool two = r + 1 < r_end;
      WRow<VBH, CHH> g0, u0, g1, u1;
      load_wrow<VBH, CHH>(g0, a.shared_gate_weight + r * K, a.shared_gate_scale + (r >> 7) * SC, lane);
      load_wrow<VBH, CHH>(u0, a.shared_up_weight + r * K, a.shared_up_scale + (r >> 7) * SC, lane);
      if (two) {
        load_wrow<VBH, CHH>(g1, a.shared_gate_weight + (r + 1) * K, a.shared_gate_scale + ((r + 1) >> 7) * SC, lane);
        load_wrow<VBH, CHH>(u1, a.shared_up_weight + (r + 1) * K, a.shared_up_scale + ((r + 1) >> 7) * SC, lane);
      }
      if (!packed) {
        pack_x_raw<VBH, CHH, HW>(raw, xs);
        packed = true;
      }
      const float tg0 = wave_sum(wrow_partial<VBH, CHH, HW>(g0, xs));
      const float tu0 = wave_sum(wrow_partial<VBH, CHH, HW>(u0, xs));
      if (lane == 0) out[r] = swiglu_mlx(tg0, tu0, a.limit);
      if (two) {
        const float tg1 = wave_sum(wrow_partial<VBH, CHH, HW>(g1, xs));
        const float tu1 = wave_sum(wrow_partial<VBH, CHH, HW>(u1, xs));
        if (lane == 0) out[r + 1] = swiglu_mlx(tg1, tu1, a.limit);
      }
    }
  };
  if (hw_decode_ok(a.shared_gate_flags) && hw_decode_ok(a.shared_up_flags))
    run(std::true_type{});
  else
    run(std::false_type{});
}

// ---------------------------------------------------------------- launch 2

template <int VBH, int CHH, int CHI>
__global__ __launch_bounds__(256) void step_gate_up_kernel(StepArgs a) {
  __shared__ int32_t s_ids[kMaxTopK];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int bid = blockIdx.x;
  const int64_t I = a.intermediate;
  if (bid >= a.routed_wgs) {
    // ---- shared down rows (fp8.py:254-299 on the shared SwiGLU rows)
    if (a.shared_down_weight == nullptr) return;
    const int64_t h0 = (static_cast<int64_t>(bid - a.routed_wgs) * 4 + wave) * 16;
    if (h0 >= a.hidden) return;
    HalfRaw<CHI> raw;
    load_half_raw<CHI>(a.hidden_act + static_cast<int64_t>(a.top_k) * I, lane & 31, raw);
    HalfRows<CHI, 8> rows;
    rows.issue(a.shared_down_weight, a.shared_down_scale, h0, lane, 0);
    auto run = [&](auto hw) {
      constexpr bool HW = decltype(hw)::value;
      HalfSlice<CHI, HW> xs;
      pack_half_raw<CHI, HW>(raw, xs);
      float t[8][2];
      rows.template finish<HW>(xs, t);
      if (lane == 0 || lane == 32) {
        const int half = lane >> 5;
#pragma unroll
        for (int j = 0; j < 8; ++j) a.shared_out[h0 + 2 * j + half] = f32_to_bf16(t[j][half]);
      }
    };
    if (hw_decode_ok(a.shared_down_flags))
      run(std::true_type{});
    else
      run(std::false_type{});
    return;
  }
  // ---- routed gate/up units: flat (slot, row) list split evenly
  XRaw<VBH, CHH> raw;
  load_x_raw<VBH, CHH>(a.x, lane, raw);
  if (threadIdx.x < a.top_k) s_ids[threadIdx.x] = a.ids[threadIdx.x];
  __syncthreads();
  const int64_t units = static_cast<int64_t>(a.top_k) * I;
  const int64_t waves = static_cast<int64_t>(a.routed_wgs) * 4;
  const int64_t gw = static_cast<int64_t>(bid) * 4 + wave;
  const int64_t u_begin = gw * units / waves;
  const int64_t u_end = (gw + 1) * units / waves;
  if (u_begin >= u_end) return;
  const int64_t K = a.hidden, SC = K / kBlock, SR = I / kBlock;
  const int g = a.bank_group_log2;
  const RowWalk walk = row_walk<VBH>(lane, g);
  auto unit_ptrs = [&](int64_t u, const uint8_t*& gw_row, const uint8_t*& uw_row, const float*& gs, const float*& us,
                       int64_t& out_index, bool& ok) {
    const int slot = static_cast<int>(u / I);
    const int64_t r = u - static_cast<int64_t>(slot) * I;
    const int32_t e = s_ids[slot];
    out_index = u;
    ok = e >= 0 && e < a.experts;
    const int64_t ee = ok ? e : 0;
    const uint8_t* base = a.gate_up_weight + ee * 2 * I * K;
    gw_row = base + group_row_base(r, K, g);
    uw_row = gw_row + I * K;  // up row I + r: I is a whole number of row groups
    const float* sbase = a.gate_up_scale + ee * 2 * SR * SC;
    gs = sbase + (r >> 7) * SC;
    us = sbase + (SR + (r >> 7)) * SC;
  };
  auto run = [&](auto hw) {
    constexpr bool HW = decltype(hw)::value;
    XSlice<VBH, CHH, HW> xs;
    GateUpUnit<VBH, CHH> A, B;
    const uint8_t *ga, *ua, *gb, *ub;
    const float *gsa, *usa, *gsb, *usb;
    int64_t oa, ob;
    bool oka, okb;
    auto load = [&](GateUpUnit<VBH, CHH>& U, const uint8_t* gr, const uint8_t* up, const float* gs, const float* us,
                    bool ok) {
      if (ok) {
        load_wrow_walk<VBH, CHH>(U.g, gr, gs, lane, walk);
        load_wrow_walk<VBH, CHH>(U.u, up, us, lane, walk);
      }
    };
    auto finish = [&](const GateUpUnit<VBH, CHH>& U, int64_t o, bool ok) {
      if (!ok) {
        if (lane == 0) {
          a.hidden_act[o] = 0x7FC0u;
          atomicOr(a.error_flag, 1);
        }
        return;
      }
      const float tg = wave_sum(wrow_partial<VBH, CHH, HW>(U.g, xs));
      const float tu = wave_sum(wrow_partial<VBH, CHH, HW>(U.u, xs));
      if (lane == 0) a.hidden_act[o] = swiglu_mlx(tg, tu, a.limit);
    };
    int64_t u = u_begin;
    unit_ptrs(u, ga, ua, gsa, usa, oa, oka);
    load(A, ga, ua, gsa, usa, oka);
    pack_x_raw<VBH, CHH, HW>(raw, xs);  // waits for the activations only
    for (;;) {
      if (u + 1 < u_end) {
        unit_ptrs(u + 1, gb, ub, gsb, usb, ob, okb);
        load(B, gb, ub, gsb, usb, okb);
      }
      finish(A, oa, oka);
      if (++u >= u_end) break;
      if (u + 1 < u_end) {
        unit_ptrs(u + 1, ga, ua, gsa, usa, oa, oka);
        load(A, ga, ua, gsa, usa, oka);
      }
      finish(B, ob, okb);
      if (++u >= u_end) break;
    }
  };
  if (hw_decode_ok(a.routed_flags))
    run(std::true_type{});
  else
    run(std::false_type{});
}

// ---------------------------------------------------------------- launch 3

template <int CHI>
__global__ __launch_bounds__(512) void step_down_kernel(StepArgs a) {
  __shared__ float parked[kMaxTopK][16];
  const int lane = threadIdx.x & 63;
  const int slot = threadIdx.x >> 6;
  const int64_t I = a.intermediate;
  const int64_t h0 = static_cast<int64_t>(blockIdx.x) * 16;
  // The reduction's operands of output row h0 + r (threads r < 16): the
  // slot weights and the shared and residual rows, loaded before the
  // weight rows so that their round trips (cold: written by the earlier
  // launches) overlap the stream instead of following the barrier.
  float pre_score[kMaxTopK];
  float pre_shared = 0.0f, pre_residual = 0.0f;
  if (threadIdx.x < 16) {
#pragma unroll
    for (int sl = 0; sl < kMaxTopK; ++sl) pre_score[sl] = sl < a.top_k ? a.scores[sl] : 0.0f;
    if (a.shared_down_weight != nullptr) pre_shared = bf16_to_f32(a.shared_out[h0 + threadIdx.x]);
    if (a.residual != nullptr) pre_residual = bf16_to_f32(a.residual[h0 + threadIdx.x]);
  }
  if (slot < a.top_k) {
    const int32_t e = a.ids[slot];
    if (e < 0 || e >= a.experts) {
      if (lane == 0) atomicOr(a.error_flag, 1);
      if (lane < 16) parked[slot][lane] = __builtin_nanf("");
    } else {
      const int64_t SH = a.hidden / kBlock, SI = I / kBlock;
      const uint8_t* w = a.down_weight + static_cast<int64_t>(e) * a.hidden * I;
      const float* s = a.down_scale + static_cast<int64_t>(e) * SH * SI;
      HalfRaw<CHI> raw;
      load_half_raw<CHI>(a.hidden_act + static_cast<int64_t>(slot) * I, lane & 31, raw);
      HalfRows<CHI, 8> rows;
      rows.issue(w, s, h0, lane, a.bank_group_log2);
      auto run = [&](auto hw) {
        constexpr bool HW = decltype(hw)::value;
        HalfSlice<CHI, HW> xs;
        pack_half_raw<CHI, HW>(raw, xs);
        float t[8][2];
        rows.template finish<HW>(xs, t);
        if (lane == 0 || lane == 32) {
          const int half = lane >> 5;
#pragma unroll
          for (int j = 0; j < 8; ++j) parked[slot][2 * j + half] = t[j][half];
        }
      };
      if (hw_decode_ok(a.routed_flags))
        run(std::true_type{});
      else
        run(std::false_type{});
    }
  }
  __syncthreads();
  const int r = threadIdx.x;
  if (r < 16) {
    const int64_t h = h0 + r;
    float total = 0.0f;
#pragma unroll
    for (int sl = 0; sl < kMaxTopK; ++sl)
      if (sl < a.top_k) total = __fadd_rn(total, __fmul_rn(parked[sl][r], pre_score[sl]));
    float result = bf16_round(total);
    if (a.shared_down_weight != nullptr) result = __fadd_rn(result, pre_shared);
    if (a.residual != nullptr) result = __fadd_rn(pre_residual, bf16_round(result));
    a.out[h] = f32_to_bf16(result);
  }
}

// ----------------------------------------------------------------- hosts --

namespace {

template <int VBH, int CHH, int CHI>
hipError_t launch_step_t(const StepArgs& a, int stages, hipStream_t st) {
  if (stages & 1) {
    const int64_t shared_wgs =
        a.shared_gate_weight != nullptr ? (a.intermediate + 4 * a.shared_rows_per_wave - 1) / (4 * a.shared_rows_per_wave)
                                        : 0;
    const int64_t blocks = a.router_wgs + shared_wgs;
    if (blocks > 0) {
      hipLaunchKernelGGL((step_router_shared_kernel<VBH, CHH>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                         a);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  if (stages & 2) {
    const int64_t sd_wgs = a.shared_down_weight != nullptr ? (a.hidden + 63) / 64 : 0;
    hipLaunchKernelGGL((step_gate_up_kernel<VBH, CHH, CHI>), dim3(static_cast<unsigned>(a.routed_wgs + sd_wgs)),
                       dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stages & 4) {
    hipLaunchKernelGGL((step_down_kernel<CHI>), dim3(static_cast<unsigned>(a.hidden / 16)), dim3(512), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int VBH, int CHH, int CHI>
int step_occupancy_t() {
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, step_gate_up_kernel<VBH, CHH, CHI>, 256, 0) != hipSuccess)
    return 0;
  return blocks;
}

// (H, I) pairs the three-launch step is instantiated for: H = 64 VBH CHH,
// I = 512 CHI.
#define GLM53_STEP_SHAPES(X) \
  X(4096, 1536, 16, 4, 3)    \
  X(4096, 2048, 16, 4, 4)    \
  X(7168, 2048, 16, 7, 4)    \
  X(6144, 2048, 16, 6, 4)    \
  X(2048, 1024, 16, 2, 2)    \
  X(2048, 1536, 16, 2, 3)    \
  X(1024, 512, 16, 1, 1)     \
  X(1024, 1024, 16, 1, 2)

}  // namespace

bool step_shape_supported(int64_t H, int64_t I) {
#define GLM53_CASE(h, i, a, b, c) \
  if (H == h && I == i) return true;
  GLM53_STEP_SHAPES(GLM53_CASE)
#undef GLM53_CASE
  return false;
}

int step_gate_up_occupancy(int64_t H, int64_t I) {
#define GLM53_CASE(h, i, a, b, c) \
  if (H == h && I == i) return step_occupancy_t<a, b, c>();
  GLM53_STEP_SHAPES(GLM53_CASE)
#undef GLM53_CASE
  return 0;
}

hipError_t launch_step(const StepArgs& a, int stages, hipStream_t st) {
#define GLM53_CASE(h, i, va, ca, ci) \
  if (a.hidden == h && a.intermediate == i) return launch_step_t<va, ca, ci>(a, stages, st);
  GLM53_STEP_SHAPES(GLM53_CASE)
#undef GLM53_CASE
  return hipErrorInvalidValue;
}

}  // namespace glm53
