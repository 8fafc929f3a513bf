// Streaming-GEMV building blocks shared by the decode kernels: lane-owned
// activation slices (exact FP16 pairs), non-temporal weight chunks, E4M3
// contraction (software or gfx950 hardware decode), and the wave top-k.
#pragma once
#include "common.h"
#include "kernels.h"

namespace glm53 {

// ------------------------------------------------------------ helpers ----

// A lane's activation slice: CH chunks of VB consecutive elements at
// positions VB*lane + 64*VB*c, held as FP16 pairs.  HW = true pairs them
// (x0,x1),(x2,x3) for the gfx950 E4M3->FP16 converter; HW = false pairs
// them (x0,x2),(x1,x3) for the exact SWAR decode in common.h.
template <int VB, int CH, bool HW>
struct XSlice {
  uint32_t p[CH][VB / 2];
  float factor;  // 2^shift (HW) or 2^(8 + shift) (SWAR bias of 2^-8)
};

// Packs a lane's BF16 activations (as floats) into FP16 pairs scaled by a
// power of two chosen from their amax, so every value is exact in FP16.
template <int VB, int CH, bool HW>
__device__ __forceinline__ void pack_x_slice(const float (&v)[CH][VB], XSlice<VB, CH, HW>& xs) {
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < VB; ++i) amax = fmaxf(amax, fabsf(v[c][i]));
  const int shift = f16_shift_for(amax);
  const float down = ldexpf(1.0f, -shift);
  xs.factor = ldexpf(1.0f, (HW ? 0 : 8) + shift);
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int j = 0; j < VB / 4; ++j) {
      if (HW) {
        xs.p[c][2 * j] = pack_f16x2(v[c][4 * j] * down, v[c][4 * j + 1] * down);
        xs.p[c][2 * j + 1] = pack_f16x2(v[c][4 * j + 2] * down, v[c][4 * j + 3] * down);
      } else {
        xs.p[c][2 * j] = pack_f16x2(v[c][4 * j] * down, v[c][4 * j + 2] * down);
        xs.p[c][2 * j + 1] = pack_f16x2(v[c][4 * j + 1] * down, v[c][4 * j + 3] * down);
      }
    }
}

// The raw BF16 words of a lane's slice.  Issuing these loads first and
// packing after the weight loads are issued keeps the wait for the
// activations from also waiting for the weights (vector loads retire in
// order).
template <int VB, int CH>
struct XRaw {
  uint4 q[CH][VB / 8];
};

template <int VB, int CH>
__device__ __forceinline__ void load_x_raw(const uint16_t* __restrict__ x, int lane, XRaw<VB, CH>& raw) {
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < VB / 8; ++i)
      raw.q[c][i] = *reinterpret_cast<const uint4*>(x + VB * lane + 64 * VB * c + 8 * i);
}

template <int VB, int CH, bool HW>
__device__ __forceinline__ void pack_x_raw(const XRaw<VB, CH>& raw, XSlice<VB, CH, HW>& xs) {
  float v[CH][VB];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < VB / 8; ++i) {
      const uint32_t w[4] = {raw.q[c][i].x, raw.q[c][i].y, raw.q[c][i].z, raw.q[c][i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[c][8 * i + 2 * j] = __uint_as_float(w[j] << 16);
        v[c][8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    }
  pack_x_slice<VB, CH, HW>(v, xs);
}

template <int VB, int CH, bool HW>
__device__ __forceinline__ void load_x_slice(const uint16_t* __restrict__ x, int lane, XSlice<VB, CH, HW>& xs) {
  XRaw<VB, CH> raw;
  load_x_raw<VB, CH>(x, lane, raw);
  pack_x_raw<VB, CH, HW>(raw, xs);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// One lane's VB weight bytes of a chunk.  Weights are streamed exactly once
// per launch, so they are loaded non-temporally (no L2 / MALL retention).
template <int VB>
struct WChunk;
template <>
struct WChunk<16> {
  u32x4 q;
  __device__ __forceinline__ void load(const uint8_t* p) {
    q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ __forceinline__ uint32_t word(int j) const { return q[j]; }
};
template <>
struct WChunk<8> {
  u32x2 q;
  __device__ __forceinline__ void load(const uint8_t* p) {
    q = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
  }
  __device__ __forceinline__ uint32_t word(int j) const { return q[j]; }
};

// Unscaled partial dot of one chunk (VB weight bytes) with the lane's
// activations of that chunk.
template <int VB, int CH, bool HW>
__device__ __forceinline__ float chunk_dot(const WChunk<VB>& w, const XSlice<VB, CH, HW>& xs, int c) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < VB / 4; ++j) {
    if (HW) {
      // v_cvt_scalef32_pk_f16_fp8: two E4M3 bytes -> two exact FP16 (OCP;
      // only used when the weights hold no 0x7F / 0xFF code)
      const half2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.word(j), 1.0f, false);
      const half2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.word(j), 1.0f, true);
      acc = __builtin_amdgcn_fdot2(lo, __builtin_bit_cast(half2_t, xs.p[c][2 * j]), acc, false);
      acc = __builtin_amdgcn_fdot2(hi, __builtin_bit_cast(half2_t, xs.p[c][2 * j + 1]), acc, false);
    } else {
      acc = dot4_e4m3(w.word(j), xs.p[c][2 * j], xs.p[c][2 * j + 1], acc);
    }
  }
  return acc;
}

// One weight row as a lane sees it: its CH chunks and the block scale of
// each chunk.  The scales are loaded with the chunks, in the same batch of
// vector loads: loaded later, next to the arithmetic, they would make the
// compiler wait for every load in flight (prefetched rows included) before
// the first product, since vector loads retire in order.
template <int VB, int CH>
struct WRow {
  WChunk<VB> c[CH];
  float s[CH];
};

template <int VB, int CH>
__device__ __forceinline__ void load_wrow(WRow<VB, CH>& r, const uint8_t* __restrict__ row,
                                          const float* __restrict__ srow, int lane) {
#pragma unroll
  for (int c = 0; c < CH; ++c) r.c[c].load(row + VB * lane + 64 * VB * c);
#pragma unroll
  for (int c = 0; c < CH; ++c) r.s[c] = srow[(VB * lane + 64 * VB * c) >> 7];
}

// Where a lane's chunks of one row lie in a matrix of row groups of 2^g rows
// (common.h): chunk c at lane_off + c * stride bytes from the row's base
// group_row_base(n, K, g).  A lane's VB bytes never straddle a 128-byte
// block (VB divides 128) and a chunk spans 64 VB bytes, a multiple of 128,
// so the offsets split into a lane part and a chunk part.
struct RowWalk {
  int32_t lane_off;
  int32_t stride;
};

template <int VB>
__device__ __forceinline__ RowWalk row_walk(int lane, int g) {
  static_assert(VB >= 2 && 128 % VB == 0, "a lane's bytes stay inside one 128-byte block");
  return {static_cast<int32_t>(group_col(VB * lane, g)), (64 * VB) << g};
}

template <int VB, int CH>
__device__ __forceinline__ void load_wrow_walk(WRow<VB, CH>& r, const uint8_t* __restrict__ row,
                                               const float* __restrict__ srow, int lane, RowWalk walk) {
#pragma unroll
  for (int c = 0; c < CH; ++c) r.c[c].load(row + walk.lane_off + c * walk.stride);
#pragma unroll
  for (int c = 0; c < CH; ++c) r.s[c] = srow[(VB * lane + 64 * VB * c) >> 7];
}

template <int VB, int CH, bool HW>
__device__ __forceinline__ float wrow_partial(const WRow<VB, CH>& r, const XSlice<VB, CH, HW>& xs) {
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) acc += chunk_dot<VB, CH, HW>(r.c[c], xs, c) * r.s[c];
  return acc * xs.factor;
}

// The register decode is usable unless a (device) scan flagged 0x7F / 0xFF
// codes; a null flag means "not scanned" and keeps the exact SWAR decode.
__device__ __forceinline__ bool hw_decode_ok(const int32_t* flag) { return flag != nullptr && *flag == 0; }

__device__ __forceinline__ bool bad_expert(int32_t e, int64_t experts) {
  return e < 0 || static_cast<int64_t>(e) >= experts;
}

// ------------------------------------------------------------------ top-k --
//
// Selection half of the router (patch.py:131-142 with the DeepSeek-V3
// aux-loss-free rule): one wavefront reads the FP32 logits of one token,
// forms sigma = sigmoid(logit) and choice = sigma + bias, and picks top_k by
// (choice desc, expert id asc).  Lane l holds candidates l, l+64, ...
// Weights = sigma of the picks, normalised in slot order when norm, times
// the scaling factor.  Emits ids[slot] (lane 0) and weights[slot] (lane
// slot); dst may be LDS or global.  PER_LANE = candidates per lane, a
// compile-time bound (experts <= 64 * PER_LANE) that keeps the selection in
// a handful of registers.

// DPP wave reductions of unsigned 32-bit values (every lane gets the result).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return max(max(a, b), max(c, d));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp_u32<0xB1>(v));
  v = min(v, dpp_u32<0x4E>(v));
  v = min(v, dpp_u32<0x141>(v));
  v = min(v, dpp_u32<0x140>(v));
  const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return min(min(a, b), min(c, d));
}

// Order-preserving u32 image of a float (NaN ranks as -inf): a > b as floats
// iff image(a) > image(b), with +0 above -0.
__device__ __forceinline__ uint32_t orderable_bits(float v) {
  if (v != v) v = -__builtin_inff();
  const uint32_t u = __float_as_uint(v);
  return u ^ ((u & 0x80000000u) ? 0xFFFFFFFFu : 0x80000000u);
}

// sigmoid of a router logit, the one expression every selection path uses
// (so a score computed where the logit is made equals one computed later).
__device__ __forceinline__ float router_sigmoid(float logit) { return 1.0f / (1.0f + expf(-logit)); }

// The float an orderable image stands for (inverse of orderable_bits).
__device__ __forceinline__ float orderable_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// Group-limited selection, the DeepSeek-V3 rule that mlx-vlm's
// dsv32.group_expert_select applies when n_group > 1 (patch.py:134-142
// passes n_group and topk_group): the experts form n_group groups of
// experts / n_group consecutive ids; a group's score is the FP32 sum of its
// two largest biased scores; the n_group - topk_group groups of lowest score
// have every biased score replaced by 0.0 before the top-k.  Ties between
// group scores keep the lower group index (MLX's argpartition leaves them
// unspecified).  n_group = 1 selects over all experts unchanged.
struct GroupLimit {
  int n_group = 1;
  int topk_group = 1;
};

// Applies a GroupLimit to the keys of one token held as in wave_topk_regs
// (key[i] of expert lane + 64 i; 0 = absent).  One pass per group: each lane's
// two largest keys in the group, a wave max for the largest, a second wave
// max over every lane's next candidate (the second key of one lane holding
// the largest, the largest of the others) for the runner-up.  n_group <= 64,
// experts / n_group >= 2.
template <int PER_LANE>
__device__ __forceinline__ void group_limit_keys(uint32_t (&key)[PER_LANE], int64_t experts, GroupLimit gl, int lane) {
  const int64_t per = experts / gl.n_group;
  float gscore = 0.0f;  // lane g < n_group: the score of group g
#pragma unroll 1
  for (int g = 0; g < gl.n_group; ++g) {
    uint32_t b1 = 0u, b2 = 0u;
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) {
      const int64_t c = lane + 64 * i;
      if (c < experts && c / per == g) {
        const uint32_t k = key[i];
        if (k > b1) {
          b2 = b1;
          b1 = k;
        } else if (k > b2) {
          b2 = k;
        }
      }
    }
    const uint32_t m1 = wave_max_u32(b1);
    const unsigned long long holders = __ballot(b1 == m1);
    const int first = __ffsll(static_cast<long long>(holders)) - 1;
    const uint32_t m2 = wave_max_u32(lane == first ? b2 : b1);
    if (lane == g) gscore = __fadd_rn(orderable_value(m1), orderable_value(m2));
  }
  bool keep = false;
  if (lane < gl.n_group) {
    int rank = 0;
#pragma unroll 1
    for (int h = 0; h < gl.n_group; ++h) {
      const float sh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gscore), h));
      rank += (sh > gscore || (sh == gscore && h < lane)) ? 1 : 0;
    }
    keep = rank < gl.topk_group;
  }
  const unsigned long long kept = __ballot(keep);
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    const int64_t c = lane + 64 * i;
    if (c < experts && !((kept >> (c / per)) & 1ull)) key[i] = 0x80000000u;  // orderable image of +0.0
  }
}

// Core selection over logits already in registers: lg[i] is the logit of
// expert lane + 64 * i (ignored when that is >= experts).  Each of the top_k
// rounds is two DPP reductions: the largest biased score (as its orderable
// image), then the smallest expert id holding it, i.e. the order
// (choice desc, expert id asc).
template <int PER_LANE>
__device__ __forceinline__ void wave_topk_regs(const float (&lg)[PER_LANE], const float* __restrict__ bias,
                                               int64_t experts, int top_k, float scaling, int norm, int lane,
                                               int32_t* ids_dst, float* w_dst, GroupLimit gl = {}) {
  uint32_t key[PER_LANE];  // orderable image of the biased score; 0 = taken / absent
  float sigs[PER_LANE];
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    const int64_t c = lane + 64 * i;
    float sg = 0.0f;
    key[i] = 0u;
    if (c < experts) {
      sg = router_sigmoid(lg[i]);
      key[i] = max(orderable_bits(__fadd_rn(sg, bias[c])), 1u);
    }
    sigs[i] = sg;
  }
  if (gl.n_group > 1) group_limit_keys<PER_LANE>(key, experts, gl, lane);
  float total = 0.0f;
  float w_mine = 0.0f;  // lane `slot` keeps the weight of its slot
#pragma unroll 1
  for (int slot = 0; slot < top_k; ++slot) {
    uint32_t best = 0;
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) best = max(best, key[i]);
    best = wave_max_u32(best);
    uint32_t id = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i)
      if (key[i] == best) id = min(id, static_cast<uint32_t>(lane + 64 * i));
    id = wave_min_u32(id);
    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) {
      if (static_cast<uint32_t>(lane + 64 * i) == id) {
        mine = sigs[i];
        key[i] = 0u;  // taken
      }
    }
    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), static_cast<int>(id & 63)));
    total = __fadd_rn(total, w);
    if (lane == slot) w_mine = w;
    if (lane == 0) ids_dst[slot] = static_cast<int32_t>(id);
  }
  if (lane < top_k) {
    float v = w_mine;
    if (top_k > 1 && norm) v = v / total;
    w_dst[lane] = __fmul_rn(v, scaling);
  }
}

// Selection over published router words (sigmoid bits << 32 | key, key 0 =
// absent): wd[i] belongs to expert lane + 64 i.  Same order as
// wave_topk_regs, (key desc, expert id asc), with one reduction per pick:
// each lane keeps a head (its largest key, lowest id among equals), a DPP max
// over the heads finds the key, a ballot finds the lanes holding it (one
// lane: its head is the pick; several: a DPP min over their head ids), and
// the winning lane drops that entry and recomputes its head.
template <int PER_LANE>
__device__ __forceinline__ void wave_topk_words(const unsigned long long (&wd)[PER_LANE], int top_k, float scaling,
                                                int norm, int lane, int32_t* ids_dst, float* w_dst,
                                                GroupLimit gl = {}, int64_t experts = 0) {
  uint32_t key[PER_LANE];
  float sig[PER_LANE];
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    key[i] = static_cast<uint32_t>(wd[i]);
    sig[i] = __uint_as_float(static_cast<uint32_t>(wd[i] >> 32));
  }
  if (gl.n_group > 1) group_limit_keys<PER_LANE>(key, experts, gl, lane);
  uint32_t hk;
  int hi;
  float hs;
  auto head = [&]() {
    hk = key[0];
    hi = 0;
    hs = sig[0];
#pragma unroll
    for (int i = 1; i < PER_LANE; ++i)
      if (key[i] > hk) {
        hk = key[i];
        hi = i;
        hs = sig[i];
      }
  };
  head();
  float total = 0.0f;
  float w_mine = 0.0f;  // lane `slot` keeps the weight of its slot
#pragma unroll 1
  for (int slot = 0; slot < top_k; ++slot) {
    const uint32_t best = wave_max_u32(hk);
    const unsigned long long holders = __ballot(hk == best);
    int wl;
    uint32_t id;
    if (__popcll(holders) == 1) {
      wl = __ffsll(static_cast<long long>(holders)) - 1;
      id = static_cast<uint32_t>(wl + 64 * __builtin_amdgcn_readlane(hi, wl));
    } else {
      id = wave_min_u32(hk == best ? static_cast<uint32_t>(lane + 64 * hi) : 0xFFFFFFFFu);
      wl = static_cast<int>(id & 63);
    }
    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hs), wl));
    total = __fadd_rn(total, w);
    if (lane == slot) w_mine = w;
    if (lane == 0) ids_dst[slot] = static_cast<int32_t>(id);
    if (lane == wl) {
#pragma unroll
      for (int i = 0; i < PER_LANE; ++i)
        if (i == hi) key[i] = 0u;
      head();
    }
  }
  if (lane < top_k) {
    float v = w_mine;
    if (top_k > 1 && norm) v = v / total;
    w_dst[lane] = __fmul_rn(v, scaling);
  }
}

// Value held by lane (lane ^ J) for J = 1 .. 32: DPP within 16-lane rows
// (row_ror:4 reads lane (i - 4) mod 16, row_ror:12 lane (i + 4) mod 16,
// row_ror:8 lane i ^ 8), ds_swizzle across 16, a lane shuffle across 32.
template <int J>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int lane) {
  if constexpr (J == 1) {
    return dpp_u32<0xB1>(v);  // quad_perm [1,0,3,2]
  } else if constexpr (J == 2) {
    return dpp_u32<0x4E>(v);  // quad_perm [2,3,0,1]
  } else if constexpr (J == 4) {
    const uint32_t down = dpp_u32<0x124>(v);
    const uint32_t up = dpp_u32<0x12C>(v);
    return (lane & 4) ? down : up;
  } else if constexpr (J == 8) {
    return dpp_u32<0x128>(v);
  } else if constexpr (J == 16) {
    return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x401F));
  } else {
    return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 32));
  }
}

template <int K, int J>
__device__ __forceinline__ uint32_t bitonic_step(uint32_t v, int lane) {
  const uint32_t u = xor_lane<J>(v, lane);
  return (((lane & J) == 0) == ((lane & K) == 0)) ? max(v, u) : min(v, u);
}

// One value per lane sorted descending over lanes 0..63 (bitonic network,
// 21 compare-exchange steps).
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t v, int lane) {
  v = bitonic_step<2, 1>(v, lane);
  v = bitonic_step<4, 2>(v, lane);
  v = bitonic_step<4, 1>(v, lane);
  v = bitonic_step<8, 4>(v, lane);
  v = bitonic_step<8, 2>(v, lane);
  v = bitonic_step<8, 1>(v, lane);
  v = bitonic_step<16, 8>(v, lane);
  v = bitonic_step<16, 4>(v, lane);
  v = bitonic_step<16, 2>(v, lane);
  v = bitonic_step<16, 1>(v, lane);
  v = bitonic_step<32, 16>(v, lane);
  v = bitonic_step<32, 8>(v, lane);
  v = bitonic_step<32, 4>(v, lane);
  v = bitonic_step<32, 2>(v, lane);
  v = bitonic_step<32, 1>(v, lane);
  v = bitonic_step<64, 32>(v, lane);
  v = bitonic_step<64, 16>(v, lane);
  v = bitonic_step<64, 8>(v, lane);
  v = bitonic_step<64, 4>(v, lane);
  v = bitonic_step<64, 2>(v, lane);
  v = bitonic_step<64, 1>(v, lane);
  return v;
}

// LDS of the threshold selection: compacted candidates, then the weights
// by slot.
struct TopkScratch {
  uint32_t key[64];
  uint32_t id[64];
  float sig[64];
  float w[kMaxTopK];
};

// The selection of wave_topk_words, found without sequential picks: the
// top_k-th largest of the 64 lane heads (each lane's largest key, after a
// bitonic sort) bounds the top_k-th largest key from below, so every entry
// that can be picked has key >= that bound.  Those candidates (at least
// top_k, usually few) are compacted into LDS and each one's slot is its rank
// under (key desc, expert id asc); more than 64 candidates (ties at the
// bound) fall back to the sequential picks.  Same ids, weights and FP32
// summation order as wave_topk_words.  (A single wavefront issues about one
// dependent instruction per ~12 cycles here, so the sort, the compaction,
// the rank loop and the slot sum each take ~0.3-0.5 us.)
template <int PER_LANE>
__device__ __forceinline__ void wave_topk_words_sorted(const unsigned long long (&wd)[PER_LANE], int top_k,
                                                       float scaling, int norm, int lane, int32_t* ids_dst,
                                                       float* w_dst, TopkScratch& s, GroupLimit gl = {},
                                                       int64_t experts = 0) {
  uint32_t key[PER_LANE];
  float sig[PER_LANE];
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    key[i] = static_cast<uint32_t>(wd[i]);
    sig[i] = __uint_as_float(static_cast<uint32_t>(wd[i] >> 32));
  }
  if (gl.n_group > 1) group_limit_keys<PER_LANE>(key, experts, gl, lane);
  uint32_t head = 0;
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) head = max(head, key[i]);
  const uint32_t bound = __builtin_amdgcn_readlane(wave_sort_desc(head, lane), top_k - 1);
  unsigned long long mask[PER_LANE];
  int count = 0;
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    mask[i] = __ballot(key[i] >= bound && key[i] != 0u);
    count += __popcll(mask[i]);
  }
  if (count > 64) {
    wave_topk_words<PER_LANE>(wd, top_k, scaling, norm, lane, ids_dst, w_dst, gl, experts);
    return;
  }
  int base = 0;
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    if ((mask[i] >> lane) & 1ull) {
      const int pos = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                 static_cast<uint32_t>(mask[i] >> 32),
                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask[i]), 0u)));
      s.key[pos] = key[i];
      s.id[pos] = static_cast<uint32_t>(lane + 64 * i);
      s.sig[pos] = sig[i];
    }
    base += __popcll(mask[i]);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (lane < count) {
    const uint32_t k = s.key[lane], id = s.id[lane];
    int rank = 0;
    for (int m = 0; m < count; ++m) {
      const uint32_t km = s.key[m], im = s.id[m];
      rank += (km > k || (km == k && im < id)) ? 1 : 0;
    }
    if (rank < top_k) {
      ids_dst[rank] = static_cast<int32_t>(id);
      s.w[rank] = s.sig[lane];
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  float total = 0.0f;
  for (int sl = 0; sl < top_k; ++sl) total = __fadd_rn(total, s.w[sl]);
  if (lane < top_k) {
    float v = s.w[lane];
    if (top_k > 1 && norm) v = v / total;
    w_dst[lane] = __fmul_rn(v, scaling);
  }
}

template <int PER_LANE>
__device__ __forceinline__ void wave_topk_emit(const float* __restrict__ logits, const float* __restrict__ bias,
                                               int64_t experts, int top_k, float scaling, int norm, int lane,
                                               int32_t* ids_dst, float* w_dst, GroupLimit gl) {
  float lg[PER_LANE];
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    const int64_t c = lane + 64 * i;
    lg[i] = c < experts ? logits[c] : 0.0f;
  }
  wave_topk_regs<PER_LANE>(lg, bias, experts, top_k, scaling, norm, lane, ids_dst, w_dst, gl);
}

__device__ __forceinline__ void wave_topk(const float* __restrict__ logits, const float* __restrict__ bias,
                                          int64_t experts, int top_k, float scaling, int norm, int lane,
                                          int32_t* ids_dst, float* w_dst, GroupLimit gl) {
  if (experts <= 128) wave_topk_emit<2>(logits, bias, experts, top_k, scaling, norm, lane, ids_dst, w_dst, gl);
  else if (experts <= 320) wave_topk_emit<5>(logits, bias, experts, top_k, scaling, norm, lane, ids_dst, w_dst, gl);
  else wave_topk_emit<kMaxRouterExperts / 64>(logits, bias, experts, top_k, scaling, norm, lane, ids_dst, w_dst, gl);
}

// Narrow form for the gate/up prologue (experts <= 320; wider routers select
// in topk_kernel first), so the selection never raises the streaming kernel's
// register count.
__device__ __forceinline__ void wave_topk_narrow(const float* __restrict__ logits, const float* __restrict__ bias,
                                                 int64_t experts, int top_k, float scaling, int norm, int lane,
                                                 int32_t* ids_dst, float* w_dst, GroupLimit gl) {
  if (experts <= 128) wave_topk_emit<2>(logits, bias, experts, top_k, scaling, norm, lane, ids_dst, w_dst, gl);
  else wave_topk_emit<5>(logits, bias, experts, top_k, scaling, norm, lane, ids_dst, w_dst, gl);
}

}  // namespace glm53
