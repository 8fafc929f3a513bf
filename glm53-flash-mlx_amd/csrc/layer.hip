// One-launch batch-1 decode of a whole MoE layer (router, top-k, routed and
// shared gate/up/SwiGLU, down, ordered reduction, shared add, residual).
//
// Why one launch: the three-launch form drains and refills the GPU twice per
// layer and runs its 4.7 MB router as a latency-bound kernel of its own.
// Here every workgroup of a persistent grid takes work items from a ticket
// counter, in an order where an item only ever waits on items with smaller
// tickets:
//
//   router rows | shared gate/up | routed gate/up (slot-major) |
//   shared down | routed down + reduction
//
// so the shared expert streams while the router and the top-k are in
// flight, routed down items issue their weight loads before they wait for
// the SwiGLU rows they contract, and no item waits on one that has not been
// handed out (a ticket is only taken by a running workgroup, so the lowest
// unfinished item always has its inputs).  Every wait is a bounded spin that
// sets a bit of the error flag instead of hanging.
//
// Cross-workgroup data (router logits, SwiGLU rows, shared-expert outputs)
// travels through uncached device memory, with two levels of readiness.
// Each 8-byte word carries its launch epoch (high 32 bits) next to its
// payload, so a reader that sees the current epoch in a word has that word's
// data -- coherence of a single location is all correctness needs.  Waiting
// readers do not poll those words, though: every producing wavefront bumps a
// per-array completion counter after its stores have been acknowledged, one
// lane of a waiting wavefront polls that counter with a ~1 us back-off, and
// only then are the words read (and re-read in the rare case a tag is still
// old).  Polling the data itself from hundreds of waiting wavefronts would
// swamp the memory channels that hold it.  The last workgroup to leave
// resets the ticket, exit and completion counters and advances the epoch;
// the next launch reads them after the kernel boundary.
//
// Arithmetic is exactly that of the three-launch kernels (decode.hip): same
// lane-owned slices, E4M3 contraction, wave sums, MLX BF16 SwiGLU and the
// ordered FP32 slot reduction (packed.py:100-179; fp8.py:254-299;
// native_indexer_plan.metal:525-535).  The router logit of one expert is one
// wavefront's FP32 dot product (patch.py:133).
#include "common.h"
#include "kernels.h"
#include "stream_gemv.h"

namespace glm53 {

namespace {

constexpr uint32_t kSpinLimit = 1u << 17;  // ~1 us polls per wait: well under a second
constexpr int kErrRange = 1;               // expert id out of range
constexpr int kErrRouting = 2;             // the wait for the router logits gave up
constexpr int kErrActivations = 4;         // the wait for SwiGLU rows gave up
constexpr int kErrShared = 8;              // the wait for a shared-expert output gave up

// control words (uncached, u32)
constexpr int kCtlTicket = 0, kCtlExits = 1, kCtlEpoch = 2, kCtlRouter = 4, kCtlSharedDown = 5, kCtlHidden = 6;

__device__ __forceinline__ void store_word(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t load_word(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t pair_word(uint32_t epoch, uint16_t even, uint16_t odd) {
  return (static_cast<uint64_t>(epoch) << 32) | (static_cast<uint32_t>(odd) << 16) | even;
}
__device__ __forceinline__ bool wave_all(bool ok) { return __ballot(!ok) == 0; }

// After a wavefront's exchange stores: wait until the memory system has
// acknowledged them, then count the wavefront as done.
__device__ __forceinline__ void signal_done(uint32_t* counter, int lane) {
  __builtin_amdgcn_s_waitcnt(0);
  if (lane == 0) __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Wave-uniform wait until *counter >= want (one memory request per ~1 us).
// Returns false, with `err_bit` set, if the wait gave up.
__device__ __forceinline__ bool wait_counter(const uint32_t* counter, uint32_t want, int* err, int err_bit, int lane) {
  for (uint32_t spins = 0;; ++spins) {
    const uint32_t v = __hip_atomic_load(const_cast<uint32_t*>(counter), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (__builtin_amdgcn_readfirstlane(v) >= want) return true;
    if (spins > kSpinLimit) {
      if (lane == 0) atomicOr(err, err_bit);
      return false;
    }
    __builtin_amdgcn_s_sleep(32);
  }
}

// A lane's slice of a tagged pair array (element 2m in the low half of word
// m), read once its producers have all signalled, re-read while any word
// still carries an old epoch, then packed as an activation slice.
template <int VB, int CH, bool HW>
__device__ __forceinline__ void load_tagged_slice(const uint64_t* __restrict__ words, const uint32_t* counter,
                                                  uint32_t want, int lane, uint32_t epoch, XSlice<VB, CH, HW>& xs,
                                                  int* err) {
  float v[CH][VB];
  bool ok = wait_counter(counter, want, err, kErrActivations, lane);
  for (uint32_t spins = 0; ok; ++spins) {
    bool fresh = true;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int m = 0; m < VB / 2; ++m) {
        const uint64_t w = load_word(words + (VB * lane + 64 * VB * c) / 2 + m);
        fresh = fresh && static_cast<uint32_t>(w >> 32) == epoch;
        const uint32_t d = static_cast<uint32_t>(w);
        v[c][2 * m] = __uint_as_float(d << 16);
        v[c][2 * m + 1] = __uint_as_float(d & 0xffff0000u);
      }
    if (wave_all(fresh)) break;
    if (spins > kSpinLimit) {
      if (lane == 0) atomicOr(err, kErrActivations);
      break;
    }
    __builtin_amdgcn_s_sleep(32);
  }
  if (!ok) {
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int i = 0; i < VB; ++i) v[c][i] = 0.0f;
  }
  pack_x_slice<VB, CH, HW>(v, xs);
}

// ---------------------------------------------------------------- items --

// Router logit of expert e: one wavefront, lane l covers columns
// 4l + 256c (H % 256 == 0).
__device__ __forceinline__ void router_row(const LayerArgs& a, int64_t e, int lane, uint32_t epoch) {
  const float* w = a.router_weight + e * a.hidden;
  float acc = 0.0f;
  for (int64_t c0 = 0; c0 < a.hidden; c0 += 256 * 8) {
    u32x4 wv[8];
    uint2 xv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = c0 + 256 * j + 4 * lane;
      if (k < a.hidden) {
        wv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + k));
        xv[j] = *reinterpret_cast<const uint2*>(a.x + k);
      } else {
        wv[j] = u32x4{0u, 0u, 0u, 0u};
        xv[j] = make_uint2(0u, 0u);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc = fmaf(__uint_as_float(xv[j].x << 16), __uint_as_float(wv[j][0]), acc);
      acc = fmaf(__uint_as_float(xv[j].x & 0xffff0000u), __uint_as_float(wv[j][1]), acc);
      acc = fmaf(__uint_as_float(xv[j].y << 16), __uint_as_float(wv[j][2]), acc);
      acc = fmaf(__uint_as_float(xv[j].y & 0xffff0000u), __uint_as_float(wv[j][3]), acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) store_word(a.logits + e, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(acc));
  signal_done(a.control + kCtlRouter, lane);
}

// Gate/up rows [r0, r_end) (even bounds) of one slot: SwiGLU pairs go to the
// tagged array and to the plain BF16 diagnostic copy.
template <int VB, int CH, bool HW>
__device__ __forceinline__ void gate_up_pairs(const LayerArgs& a, const uint8_t* __restrict__ gate_w,
                                              const uint8_t* __restrict__ up_w, const float* __restrict__ gate_s,
                                              const float* __restrict__ up_s, uint64_t* tagged, uint16_t* plain,
                                              uint32_t* done, int64_t r0, int64_t r_end, int lane, uint32_t epoch) {
  const int64_t K = a.hidden;
  const int64_t SC = K / kBlock;
  XRaw<VB, CH> raw;
  load_x_raw<VB, CH>(a.x, lane, raw);
  XSlice<VB, CH, HW> xs;
  bool packed = false;
#pragma unroll 1
  for (int64_t r = r0; r < r_end; r += 2) {
    WRow<VB, CH> g0, u0, g1, u1;
    load_wrow<VB, CH>(g0, gate_w + r * K, gate_s + (r >> 7) * SC, lane);
    load_wrow<VB, CH>(u0, up_w + r * K, up_s + (r >> 7) * SC, lane);
    load_wrow<VB, CH>(g1, gate_w + (r + 1) * K, gate_s + ((r + 1) >> 7) * SC, lane);
    load_wrow<VB, CH>(u1, up_w + (r + 1) * K, up_s + ((r + 1) >> 7) * SC, lane);
    if (!packed) {
      pack_x_raw<VB, CH, HW>(raw, xs);
      packed = true;
    }
    const float pg0 = wrow_partial<VB, CH, HW>(g0, xs);
    const float pu0 = wrow_partial<VB, CH, HW>(u0, xs);
    const float pg1 = wrow_partial<VB, CH, HW>(g1, xs);
    const float pu1 = wrow_partial<VB, CH, HW>(u1, xs);
    const float tg0 = wave_sum(pg0), tu0 = wave_sum(pu0);
    const float tg1 = wave_sum(pg1), tu1 = wave_sum(pu1);
    if (lane == 0) {
      const uint16_t h0 = swiglu_mlx(tg0, tu0, a.limit);
      const uint16_t h1 = swiglu_mlx(tg1, tu1, a.limit);
      plain[r] = h0;
      plain[r + 1] = h1;
      store_word(tagged + r / 2, pair_word(epoch, h0, h1));
    }
  }
  signal_done(done, lane);
}

// Down rows [h0, h_end) of one matrix against the tagged SwiGLU rows of one
// slot, 8 rows per batch; the first batch's weight loads are issued before
// the wait for the activations.  T(dot) goes to `parked` (LDS) or, for the
// shared expert, to the tagged output pairs.
template <int VB, int CH, bool HW>
__device__ __forceinline__ void down_batch_rows(const LayerArgs& a, const uint8_t* __restrict__ w,
                                                const float* __restrict__ s, const uint64_t* act,
                                                const uint32_t* act_done, uint32_t act_want, int64_t h0,
                                                int64_t h_end, float* parked, uint64_t* tagged_out, int lane,
                                                uint32_t epoch) {
  const int64_t K = a.intermediate;
  const int64_t SC = K / kBlock;
  XSlice<VB, CH, HW> xs;
  bool have_x = false;
#pragma unroll 1
  for (int64_t hb = h0; hb < h_end; hb += 8) {
    WRow<VB, CH> rows[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (hb + j < h_end) load_wrow<VB, CH>(rows[j], w + (hb + j) * K, s + ((hb + j) >> 7) * SC, lane);
    if (!have_x) {
      load_tagged_slice<VB, CH, HW>(act, act_done, act_want, lane, epoch, xs, a.error_flag);
      have_x = true;
    }
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      t[j] = (hb + j < h_end) ? bf16_round(wave_sum(wrow_partial<VB, CH, HW>(rows[j], xs))) : 0.0f;
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        if (hb + j >= h_end) break;
        if (parked != nullptr) {
          parked[hb + j - h0] = t[j];
          parked[hb + j + 1 - h0] = t[j + 1];
        } else {
          store_word(tagged_out + (hb + j) / 2, pair_word(epoch, f32_to_bf16(t[j]), f32_to_bf16(t[j + 1])));
        }
      }
    }
  }
  if (tagged_out != nullptr) signal_done(a.control + kCtlSharedDown, lane);
}

}  // namespace

template <int VBH, int CHH, int VBI, int CHI>
__global__ __launch_bounds__(256) void decode_layer_kernel(LayerArgs a) {
  __shared__ int s_ticket;
  __shared__ int32_t s_ids[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  __shared__ float parked[kMaxTopK][kLayerDownRows];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint32_t epoch = __hip_atomic_load(a.control + kCtlEpoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  const int k = a.top_k;
  const int64_t I = a.intermediate;
  const int end_router = a.n_router;
  const int end_sgu = end_router + a.n_shared_gu;
  const int end_rgu = end_sgu + a.n_routed_gu;
  const int end_sdown = end_rgu + a.n_shared_down;
  const int total = end_sdown + a.n_down;
  const int gu_items_per_slot = a.n_routed_gu / k;
  const bool hw_routed = hw_decode_ok(a.routed_flags);

  // A workgroup's tickets only grow, so it meets the item kinds in ticket
  // order: one loop per kind keeps each kind's registers to itself.
  // producers per exchange array (wavefronts that own at least one row)
  const uint32_t gu_waves = static_cast<uint32_t>((I + a.gu_rows_per_wave - 1) / a.gu_rows_per_wave);
  const uint32_t sd_waves =
      static_cast<uint32_t>((a.hidden + a.shared_down_rows_per_wave - 1) / a.shared_down_rows_per_wave);
  auto take = [&]() {
    if (threadIdx.x == 0) {
      s_ticket = static_cast<int>(
          __hip_atomic_fetch_add(a.control + kCtlTicket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM));
    }
    __syncthreads();
    const int t = s_ticket;
    __syncthreads();
    return t;
  };
  int t = take();

  for (; t < end_router; t = take()) {  // ------------------------ router rows
    const int64_t e = static_cast<int64_t>(t) * 4 + wave;
    if (e < a.experts) router_row(a, e, lane, epoch);
  }

  for (; t < end_sgu; t = take()) {  // ------------------------ shared gate / up
    const int64_t r0 = (static_cast<int64_t>(t - end_router) * 4 + wave) * a.gu_rows_per_wave;
    if (r0 >= I) continue;
    const int64_t r_end = r0 + a.gu_rows_per_wave < I ? r0 + a.gu_rows_per_wave : I;
    uint64_t* tagged = a.hidden_words + static_cast<int64_t>(k) * (I / 2);
    uint16_t* plain = a.hidden_plain + static_cast<int64_t>(k) * I;
    if (hw_decode_ok(a.shared_gate_flags) && hw_decode_ok(a.shared_up_flags))
      gate_up_pairs<VBH, CHH, true>(a, a.shared_gate_weight, a.shared_up_weight, a.shared_gate_scale,
                                    a.shared_up_scale, tagged, plain, a.control + kCtlHidden + k, r0, r_end, lane,
                                    epoch);
    else
      gate_up_pairs<VBH, CHH, false>(a, a.shared_gate_weight, a.shared_up_weight, a.shared_gate_scale,
                                     a.shared_up_scale, tagged, plain, a.control + kCtlHidden + k, r0, r_end, lane,
                                     epoch);
  }

  // Routing, once per workgroup, before its first routed item (uniform per
  // workgroup: t is).
  bool routing = false;
  auto ensure_routing = [&]() {
    if (routing) return;
    routing = true;
    if (a.given_ids != nullptr) {
      if (threadIdx.x < k) {
        s_ids[threadIdx.x] = a.given_ids[threadIdx.x];
        s_w[threadIdx.x] = a.given_scores[threadIdx.x];
      }
    } else if (wave == 0) {
      float lg[5];
      bool ok = wait_counter(a.control + kCtlRouter, static_cast<uint32_t>(a.experts), a.error_flag, kErrRouting,
                             lane);
      for (uint32_t spins = 0;; ++spins) {
        bool fresh = true;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
          const int64_t c = lane + 64 * i;
          lg[i] = 0.0f;
          if (c < a.experts) {
            const uint64_t w = load_word(a.logits + c);
            fresh = fresh && static_cast<uint32_t>(w >> 32) == epoch;
            lg[i] = __uint_as_float(static_cast<uint32_t>(w));
          }
        }
        if (!ok || wave_all(fresh)) break;
        if (spins > kSpinLimit) {
          if (lane == 0) atomicOr(a.error_flag, kErrRouting);
          break;
        }
        __builtin_amdgcn_s_sleep(32);
      }
      wave_topk_regs<5>(lg, a.router_bias, a.experts, k, a.routed_scaling_factor, a.norm_topk_prob, lane, s_ids,
                        s_w);
    }
    __syncthreads();
  };
  if (t < end_rgu) ensure_routing();

  for (; t < end_rgu; t = take()) {  // ------------------------ routed gate / up
    const int local = t - end_sgu;
    const int slot = local / gu_items_per_slot;
    const int chunk = local % gu_items_per_slot;
    if (local == 0 && threadIdx.x < k) {  // publish the routing once
      a.ids_out[threadIdx.x] = s_ids[threadIdx.x];
      a.scores_out[threadIdx.x] = s_w[threadIdx.x];
    }
    const int64_t r0 = (static_cast<int64_t>(chunk) * 4 + wave) * a.gu_rows_per_wave;
    if (r0 >= I) continue;
    const int64_t r_end = r0 + a.gu_rows_per_wave < I ? r0 + a.gu_rows_per_wave : I;
    const int32_t e = s_ids[slot];
    uint64_t* tagged = a.hidden_words + static_cast<int64_t>(slot) * (I / 2);
    uint16_t* plain = a.hidden_plain + static_cast<int64_t>(slot) * I;
    uint32_t* done = a.control + kCtlHidden + slot;
    if (e < 0 || e >= a.experts) {
      if (lane == 0) {
        atomicOr(a.error_flag, kErrRange);
        for (int64_t r = r0; r < r_end; r += 2) {
          plain[r] = plain[r + 1] = 0x7FC0u;
          store_word(tagged + r / 2, pair_word(epoch, 0x7FC0u, 0x7FC0u));
        }
      }
      signal_done(done, lane);
      continue;
    }
    const int64_t SR = I / kBlock, SC = a.hidden / kBlock;
    const uint8_t* gate_w = a.gate_up_weight + static_cast<int64_t>(e) * 2 * I * a.hidden;
    const uint8_t* up_w = gate_w + I * a.hidden;
    const float* gate_s = a.gate_up_scale + static_cast<int64_t>(e) * 2 * SR * SC;
    const float* up_s = gate_s + SR * SC;
    if (hw_routed)
      gate_up_pairs<VBH, CHH, true>(a, gate_w, up_w, gate_s, up_s, tagged, plain, done, r0, r_end, lane, epoch);
    else
      gate_up_pairs<VBH, CHH, false>(a, gate_w, up_w, gate_s, up_s, tagged, plain, done, r0, r_end, lane, epoch);
  }

  for (; t < end_sdown; t = take()) {  // ------------------------ shared down
    const int64_t h0 = (static_cast<int64_t>(t - end_rgu) * 4 + wave) * a.shared_down_rows_per_wave;
    if (h0 >= a.hidden) continue;
    const int64_t h_end = h0 + a.shared_down_rows_per_wave < a.hidden ? h0 + a.shared_down_rows_per_wave : a.hidden;
    const uint64_t* act = a.hidden_words + static_cast<int64_t>(k) * (I / 2);
    if (hw_decode_ok(a.shared_down_flags))
      down_batch_rows<VBI, CHI, true>(a, a.shared_down_weight, a.shared_down_scale, act,
                                      a.control + kCtlHidden + k, gu_waves, h0, h_end, nullptr, a.shared_words,
                                      lane, epoch);
    else
      down_batch_rows<VBI, CHI, false>(a, a.shared_down_weight, a.shared_down_scale, act,
                                       a.control + kCtlHidden + k, gu_waves, h0, h_end, nullptr, a.shared_words,
                                       lane, epoch);
  }

  if (t < total) ensure_routing();
  for (; t < total; t = take()) {  // ------------------- routed down + reduction
    const int64_t h0 = static_cast<int64_t>(t - end_sdown) * kLayerDownRows;
    const int64_t h_end = h0 + kLayerDownRows < a.hidden ? h0 + kLayerDownRows : a.hidden;
    const int64_t SH = a.hidden / kBlock, SI = I / kBlock;
    for (int slot = wave; slot < k; slot += 4) {
      const int32_t e = s_ids[slot];
      if (e < 0 || e >= a.experts) {
        if (lane == 0) atomicOr(a.error_flag, kErrRange);
        for (int64_t h = h0 + lane; h < h_end; h += 64) parked[slot][h - h0] = __builtin_nanf("");
        continue;
      }
      const uint8_t* w = a.down_weight + static_cast<int64_t>(e) * a.hidden * I;
      const float* s = a.down_scale + static_cast<int64_t>(e) * SH * SI;
      const uint64_t* act = a.hidden_words + static_cast<int64_t>(slot) * (I / 2);
      if (hw_routed)
        down_batch_rows<VBI, CHI, true>(a, w, s, act, a.control + kCtlHidden + slot, gu_waves, h0, h_end,
                                        parked[slot], nullptr, lane, epoch);
      else
        down_batch_rows<VBI, CHI, false>(a, w, s, act, a.control + kCtlHidden + slot, gu_waves, h0, h_end,
                                         parked[slot], nullptr, lane, epoch);
    }
    if (a.shared_down_weight != nullptr && wave == 0)
      wait_counter(a.control + kCtlSharedDown, sd_waves, a.error_flag, kErrShared, lane);
    __syncthreads();
    const int r = threadIdx.x;
    if (r < h_end - h0) {
      const int64_t h = h0 + r;
      float total_s = 0.0f;
      for (int sl = 0; sl < k; ++sl) total_s = __fadd_rn(total_s, __fmul_rn(parked[sl][r], s_w[sl]));
      float result = bf16_round(total_s);
      if (a.shared_down_weight != nullptr) {
        uint64_t wv = 0;
        uint32_t spins = 0;
        for (;;) {
          wv = load_word(a.shared_words + h / 2);
          if (static_cast<uint32_t>(wv >> 32) == epoch) break;
          if (++spins > kSpinLimit) {
            atomicOr(a.error_flag, kErrShared);
            break;
          }
          __builtin_amdgcn_s_sleep(32);
        }
        const uint32_t d = static_cast<uint32_t>(wv);
        const uint16_t sh = (h & 1) ? static_cast<uint16_t>(d >> 16) : static_cast<uint16_t>(d & 0xffffu);
        result = __fadd_rn(result, bf16_to_f32(sh));
      }
      if (a.residual != nullptr) result = __fadd_rn(bf16_to_f32(a.residual[h]), bf16_round(result));
      a.out[h] = f32_to_bf16(result);
    }
    // parked is reused by this workgroup's next item; the barrier in take()
    // orders these reads before the next item's writes
  }

  // The last workgroup out resets the counters and advances the epoch.
  if (threadIdx.x == 0) {
    const uint32_t done =
        __hip_atomic_fetch_add(a.control + kCtlExits, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (done == gridDim.x - 1) {
      for (int c = 0; c < kCtlHidden + kMaxTopK + 1; ++c)
        if (c != kCtlEpoch) __hip_atomic_store(a.control + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(a.control + kCtlEpoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

namespace {

template <int VBH, int CHH, int VBI, int CHI>
hipError_t launch_layer_t(const LayerArgs& a, int grid, hipStream_t st) {
  hipLaunchKernelGGL((decode_layer_kernel<VBH, CHH, VBI, CHI>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, st,
                     a);
  return hipGetLastError();
}

template <int VBH, int CHH, int VBI, int CHI>
int occupancy_t() {
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_layer_kernel<VBH, CHH, VBI, CHI>, 256, 0) !=
      hipSuccess)
    return 0;
  return blocks;
}

// (H, I) pairs with an instantiated layer kernel; VB * CH * 64 == width.
#define GLM53_LAYER_SHAPES(X) \
  X(4096, 1536, 16, 4, 8, 3)  \
  X(4096, 2048, 16, 4, 16, 2) \
  X(2048, 1024, 16, 2, 16, 1) \
  X(1024, 512, 16, 1, 8, 1)

}  // namespace

bool layer_shape_supported(int64_t H, int64_t I) {
#define GLM53_CASE(h, i, a, b, c, d) \
  if (H == h && I == i) return true;
  GLM53_LAYER_SHAPES(GLM53_CASE)
#undef GLM53_CASE
  return false;
}

int layer_occupancy(int64_t H, int64_t I) {
#define GLM53_CASE(h, i, a, b, c, d) \
  if (H == h && I == i) return occupancy_t<a, b, c, d>();
  GLM53_LAYER_SHAPES(GLM53_CASE)
#undef GLM53_CASE
  return 0;
}

hipError_t launch_decode_layer(const LayerArgs& a, int grid, hipStream_t st) {
#define GLM53_CASE(h, i, va, ca, vb, cb) \
  if (a.hidden == h && a.intermediate == i) return launch_layer_t<va, ca, vb, cb>(a, grid, st);
  GLM53_LAYER_SHAPES(GLM53_CASE)
#undef GLM53_CASE
  return hipErrorInvalidValue;
}

}  // namespace glm53
