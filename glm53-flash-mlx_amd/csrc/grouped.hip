// Sorted grouped-expert prefill for the FP8 block-scaled MoE layer.
//
//  * Route plan (grouped_fp8.py:157-203; native_indexer_plan.metal:1878-1982):
//    per-block expert histograms, one scan workgroup (expert offsets, tile
//    offsets, expert-aligned descriptors, invalid-route count), and a stable
//    scatter that ranks each route among same-expert routes of its block.
//    No sorted-activation copy is made: the GEMM gathers token rows through
//    the sorted token index.
//  * Activation split (this build's MFMA operand format): every (row,
//    128-column block) gets a power-of-two scale s with amax/s <= 448, and
//    x/s is written as hi + lo/16 with hi, lo both E4M3.  A BF16 value has 8
//    significant bits: hi keeps 4 and lo the remaining 4, so the split is
//    exact whenever lo stays in E4M3's normal range, i.e. for every element
//    with |x/s| >= 2^-6 (|x| >= amax / 28672).  Smaller elements are rounded
//    on E4M3's subnormal grid, an absolute error of at most 2^-14 * s
//    (< 2.8e-7 * amax of the row block); the MFMA then multiplies these
//    operands by the raw weight codes with no further rounding of products.
//  * Grouped GEMM (grouped_fp8.py:30-140): gfx950 v_mfma_f32_16x16x128 with
//    E4M3 weights fed raw from HBM as the B operand (no decode, no LDS) and
//    the hi/lo activation rows as the A operand.  One MFMA covers exactly
//    one 128-deep scale block; its result is scaled by the weight block scale
//    and the activation scale and accumulated in FP32 registers.
//  * Reductions: grouped FP32 slot-order restore (grouped_fp8.py:273-276) or
//    the exact Direct ascending-expert BF16 order
//    (native_indexer_plan.metal:2174-2207), each with the shared-expert add.
#include "common.h"
#include "grouped.h"

namespace glm53 {

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ route plan --

__global__ __launch_bounds__(256) void route_count_kernel(RoutePlanArgs a) {
  __shared__ unsigned hist[kPlanMaxExperts];
  __shared__ unsigned bad;
  for (int e = threadIdx.x; e < a.experts; e += 256) hist[e] = 0;
  if (threadIdx.x == 0) bad = 0;
  __syncthreads();
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < a.routes) {
    int32_t e = a.expert_ids[i];
    if (e >= 0 && e < a.experts) atomicAdd(&hist[e], 1u);
    else atomicAdd(&bad, 1u);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < a.experts; e += 256) a.block_counts[static_cast<int64_t>(blockIdx.x) * a.experts + e] = hist[e];
  if (threadIdx.x == 0) a.block_invalid[blockIdx.x] = bad;
}

// Inclusive Hillis-Steele scan of buf[0..n) in LDS (n <= 1024, 1024 threads).
__device__ void block_scan_inclusive(unsigned* buf, int n) {
  for (int off = 1; off < n; off <<= 1) {
    unsigned v = 0;
    if (threadIdx.x < n && threadIdx.x >= off) v = buf[threadIdx.x - off];
    __syncthreads();
    if (threadIdx.x < n) buf[threadIdx.x] += v;
    __syncthreads();
  }
}

__global__ __launch_bounds__(1024) void route_scan_kernel(RoutePlanArgs a) {
  __shared__ unsigned route_cum[kPlanMaxExperts];
  __shared__ unsigned tile_cum[kPlanMaxExperts];
  __shared__ unsigned invalid_total;
  const int t = threadIdx.x;
  if (t == 0) invalid_total = 0;
  __syncthreads();
  // per-expert running base over blocks (exclusive), totals per expert
  if (t < a.experts) {
    unsigned run = 0;
    for (int64_t b = 0; b < a.blocks; ++b) {
      unsigned c = a.block_counts[b * a.experts + t];
      a.block_counts[b * a.experts + t] = run;
      run += c;
    }
    route_cum[t] = run;
    tile_cum[t] = (run + a.tile_rows - 1) / a.tile_rows;
  }
  for (int64_t b = t; b < a.blocks; b += 1024) atomicAdd(&invalid_total, a.block_invalid[b]);
  __syncthreads();
  block_scan_inclusive(route_cum, a.experts);
  block_scan_inclusive(tile_cum, a.experts);
  if (t < a.experts) {
    a.route_offsets[t + 1] = route_cum[t];
    a.tile_offsets[t + 1] = tile_cum[t];
  }
  if (t == 0) {
    a.route_offsets[0] = 0;
    a.tile_offsets[0] = 0;
    a.status[0] = invalid_total;                       // invalid route count
    a.status[1] = tile_cum[a.experts - 1];             // valid descriptors
  }
  // descriptors: owner by binary search over the inclusive tile scan
  const unsigned total_tiles = tile_cum[a.experts - 1];
  for (int64_t d = t; d < a.capacity; d += 1024) {
    if (d >= total_tiles) {
      a.tile_expert[d] = 0;
      a.tile_start[d] = static_cast<int32_t>(a.routes);
      a.tile_len[d] = 0;
      continue;
    }
    int lo = 0, hi = a.experts - 1;
    while (lo < hi) {  // first e with tile_cum[e] > d
      int mid = (lo + hi) >> 1;
      if (tile_cum[mid] > d) hi = mid; else lo = mid + 1;
    }
    const unsigned first_tile = lo == 0 ? 0 : tile_cum[lo - 1];
    const unsigned first_route = lo == 0 ? 0 : route_cum[lo - 1];
    const unsigned start = first_route + (static_cast<unsigned>(d) - first_tile) * a.tile_rows;
    const unsigned end = route_cum[lo];
    a.tile_expert[d] = lo;
    a.tile_start[d] = static_cast<int32_t>(start);
    a.tile_len[d] = static_cast<int32_t>(end - start < static_cast<unsigned>(a.tile_rows) ? end - start : a.tile_rows);
  }
}

__global__ __launch_bounds__(256) void route_scatter_kernel(RoutePlanArgs a) {
  __shared__ int32_t ids[256];
  const int t = threadIdx.x;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + t;
  ids[t] = i < a.routes ? a.expert_ids[i] : -1;
  __syncthreads();
  if (i >= a.routes) return;
  const int32_t e = ids[t];
  if (e < 0 || e >= a.experts) {
    a.inverse[i] = -1;
    return;
  }
  int rank = 0;
  for (int j = 0; j < t; ++j) rank += ids[j] == e;
  const int64_t pos = static_cast<int64_t>(a.route_offsets[e]) +
                      a.block_counts[static_cast<int64_t>(blockIdx.x) * a.experts + e] + rank;
  a.sorted_route[pos] = static_cast<int32_t>(i);
  a.inverse[i] = static_cast<int32_t>(pos);
  a.sorted_expert[pos] = e;
  a.sorted_token[pos] = static_cast<int32_t>(i / a.top_k);
  if (a.scores != nullptr) a.sorted_score[pos] = a.scores[i];
}

// ------------------------------------------------ activation hi/lo split --

// RNE to the E4M3 grid, saturating at +-448 (never the 0x7F/0xFF codes).
__device__ __forceinline__ uint32_t encode_e4m3(float v) {
  uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
  float a = fabsf(v);
  if (!(a < 448.0f)) return sign | 0x7Eu;
  if (a < 0.015625f) {  // below 2^-6: subnormal grid of 2^-9
    return sign | static_cast<uint32_t>(rintf(a * 512.0f));
  }
  int e = ilogbf(a);
  float m = rintf(ldexpf(a, 3 - e));  // in [8, 16]
  if (m >= 16.0f) {
    e += 1;
    m = 8.0f;
  }
  if (e > 8 || (e == 8 && m > 14.0f)) return sign | 0x7Eu;
  return sign | (static_cast<uint32_t>(e + 7) << 3) | (static_cast<uint32_t>(m) - 8u);
}

__device__ __forceinline__ float e4m3_value(uint32_t code) {
  uint16_t h = static_cast<uint16_t>(((code & 0x7Fu) << 7) | ((code & 0x80u) << 8));
  return static_cast<float>(__builtin_bit_cast(_Float16, h)) * 256.0f;
}

// One wavefront per (row, 128-column block): two elements per lane.
__global__ __launch_bounds__(256) void split_activations_kernel(SplitArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t blocks_per_row = a.cols / kBlock;
  if (unit >= a.rows * blocks_per_row) return;
  const int64_t row = unit / blocks_per_row;
  const int64_t blk = unit % blocks_per_row;
  const uint16_t* src = a.x + row * a.x_row_stride + blk * kBlock + 2 * lane;
  uint32_t pair = *reinterpret_cast<const uint32_t*>(src);
  float v0 = __uint_as_float(pair << 16);
  float v1 = __uint_as_float(pair & 0xffff0000u);
  float amax = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
  // s = 2^ceil(log2(amax / 448)): amax / s lies in (224, 448].
  float s = 1.0f;
  if (amax > 0.0f && isfinite(amax)) {
    int e = ilogbf(amax / 448.0f);
    if (e < -126) e = -126;
    s = ldexpf(1.0f, e);
    if (amax / s > 448.0f) s = ldexpf(1.0f, e + 1);
  }
  const float inv = 1.0f / s;
  float q0 = v0 * inv, q1 = v1 * inv;
  uint32_t h0 = encode_e4m3(q0), h1 = encode_e4m3(q1);
  uint32_t l0 = encode_e4m3((q0 - e4m3_value(h0)) * 16.0f);
  uint32_t l1 = encode_e4m3((q1 - e4m3_value(h1)) * 16.0f);
  const int64_t off = row * a.cols + blk * kBlock + 2 * lane;
  *reinterpret_cast<uint16_t*>(a.hi + off) = static_cast<uint16_t>(h0 | (h1 << 8));
  *reinterpret_cast<uint16_t*>(a.lo + off) = static_cast<uint16_t>(l0 | (l1 << 8));
  if (lane == 0) a.scale[row * blocks_per_row + blk] = s;
}

// --------------------------------------------------------- grouped GEMM --
//
// Workgroup = 4 wavefronts on one descriptor (<= 32 routes of one expert,
// four groups of 8) and one column tile.  Per 128-deep K block each wave
// loads its 16 weight rows (32 bytes per lane, straight into the MFMA B
// registers) and, for each 8-route group, the 16 A rows
// [hi(t0), lo(t0), hi(t1), lo(t1), ...] so that lane l's four accumulator
// rows are hi/lo of routes 2(l/16) and 2(l/16)+1 of the group.
//
// mode GEMM_PLAIN : wave w owns output columns [64*tile + 16w, +16).
// mode GEMM_SWIGLU: wave w owns intermediate columns j in [32*tile + 8w, +8):
//   B rows 0-7 are gate rows j, rows 8-15 the matching up rows; after the K
//   loop lane n<8 fetches its up partner from lane n+8 (DPP row_ror:8) and
//   stores h = SwiGLU(T(gate), T(up)).
//
// E4M3 codes 0x7F / 0xFF decode to +-480 in the reference's table but are
// NaN in the OCP E4M3 format the MFMA consumes.  Checkpoint quantisation
// never emits them (it saturates at +-448), so weights are scanned once and
// only a flagged matrix takes the FIX variant: such bytes are fed as
// 0x7E / 0xFE (+-448) and a second, chained MFMA adds +-32 at exactly those
// positions, reproducing +-480 without leaving the FP8 path.
__device__ __forceinline__ void split_480(uint32_t w, uint32_t& fixed, uint32_t& corr) {
  const uint32_t t = (w & 0x7F7F7F7Fu) ^ 0x7F7F7F7Fu;          // zero byte where |code| == 0x7F
  const uint32_t z = ~((t | 0x80808080u) - 0x01010101u) & 0x80808080u;  // exact per-byte zero test
  const uint32_t m = z >> 7;
  fixed = w ^ m;                                               // 0x7F -> 0x7E, 0xFF -> 0xFE
  corr = (m * 0x60u) | (w & z);                                // +-32 (code 0x60) where fixed
}

template <int MODE, bool FIX>
__device__ __forceinline__ void grouped_gemm_body(const GroupedGemmArgs& a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t d = blockIdx.y;
  int32_t expert, start, len;
  if (a.tile_expert != nullptr) {
    expert = a.tile_expert[d];
    start = a.tile_start[d];
    len = a.tile_len[d];
    if (start >= a.routes || len <= 0) return;
    if (expert < 0 || expert >= a.experts) return;
  } else {
    expert = 0;
    start = static_cast<int32_t>(d * kGroupedTileRows);
    len = static_cast<int32_t>(a.routes - start < kGroupedTileRows ? a.routes - start : kGroupedTileRows);
    if (len <= 0) return;
  }
  const int64_t K = a.K;
  const int64_t KB = K / kBlock;
  const int n16 = lane & 15;
  const int kq = lane >> 4;  // which 32-byte quarter of the 128-deep block

  // B row owned by this lane and the output column it lands on
  int64_t brow;
  int64_t col;
  const uint8_t* wbase;
  const float* sbase;
  if (MODE == GEMM_PLAIN) {
    col = static_cast<int64_t>(blockIdx.x) * 64 + wave * 16 + n16;
    if (static_cast<int64_t>(blockIdx.x) * 64 + wave * 16 >= a.N) return;
    brow = col;
    wbase = a.weight + static_cast<int64_t>(expert) * a.w_expert_stride;
    sbase = a.scale + static_cast<int64_t>(expert) * a.s_expert_stride;
  } else {
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) * 32 + wave * 8;
    if (j0 >= a.N) return;
    col = j0 + (n16 & 7);
    brow = col;
    if (n16 < 8) {
      wbase = a.weight + static_cast<int64_t>(expert) * a.w_expert_stride;
      sbase = a.scale + static_cast<int64_t>(expert) * a.s_expert_stride;
    } else {
      wbase = a.weight_up + static_cast<int64_t>(expert) * a.w_expert_stride;
      sbase = a.scale_up + static_cast<int64_t>(expert) * a.s_expert_stride;
    }
  }
  const bool col_ok = col < a.N;
  const uint8_t* bptr = wbase + (col_ok ? brow : 0) * K + kq * 32;
  const float* srow = sbase + ((col_ok ? brow : 0) >> 7) * a.s_cols;

  // A rows: lane's A row rho = n16 -> route 2*(rho/4) + ((rho>>1)&1) of each
  // 8-route group, hi if rho even else lo.
  const int tok_in_group = 2 * (n16 >> 2) + ((n16 >> 1) & 1);
  const uint8_t* aplane = (n16 & 1) ? a.a_lo : a.a_hi;
  const int groups = (len + 7) >> 3;
  int64_t arow[kGroupedTileRows / 8];
  bool aok[kGroupedTileRows / 8];
#pragma unroll
  for (int g = 0; g < kGroupedTileRows / 8; ++g) {
    const int tt = g * 8 + tok_in_group;
    aok[g] = g < groups && tt < len;
    const int64_t route = start + (aok[g] ? tt : 0);
    arow[g] = a.a_row_index != nullptr ? a.a_row_index[route] : route;
  }
  // activation rows of the two routes whose hi/lo rows land in this lane's
  // accumulator (routes 2kq and 2kq+1 of each group)
  int64_t srow0[kGroupedTileRows / 8], srow1[kGroupedTileRows / 8];
#pragma unroll
  for (int g = 0; g < kGroupedTileRows / 8; ++g) {
    const int t0 = g * 8 + 2 * kq, t1 = t0 + 1;
    const int64_t r0 = start + (t0 < len ? t0 : 0);
    const int64_t r1 = start + (t1 < len ? t1 : 0);
    srow0[g] = (a.a_row_index != nullptr ? a.a_row_index[r0] : r0) * KB;
    srow1[g] = (a.a_row_index != nullptr ? a.a_row_index[r1] : r1) * KB;
  }

  float acc[kGroupedTileRows / 8][2];
#pragma unroll
  for (int g = 0; g < kGroupedTileRows / 8; ++g) acc[g][0] = acc[g][1] = 0.0f;

  for (int64_t kb = 0; kb < KB; ++kb) {
    i32x8 b;
    if (col_ok) {
      u32x4 b0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bptr + kb * kBlock));
      u32x4 b1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bptr + kb * kBlock + 16));
      b = (i32x8){(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    } else {
      b = (i32x8){0, 0, 0, 0, 0, 0, 0, 0};
    }
    i32x8 bc = (i32x8){0, 0, 0, 0, 0, 0, 0, 0};
    if (FIX) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t f, c;
        split_480(static_cast<uint32_t>(b[i]), f, c);
        b[i] = static_cast<int>(f);
        bc[i] = static_cast<int>(c);
      }
    }
    const float sw = col_ok ? srow[kb] : 0.0f;
#pragma unroll
    for (int g = 0; g < kGroupedTileRows / 8; ++g) {
      if (g >= groups) break;  // uniform across the wave
      i32x8 av = (i32x8){0, 0, 0, 0, 0, 0, 0, 0};
      if (aok[g]) {
        const uint8_t* p = aplane + arow[g] * K + kb * kBlock + kq * 32;
        u32x4 a0 = *reinterpret_cast<const u32x4*>(p);
        u32x4 a1 = *reinterpret_cast<const u32x4*>(p + 16);
        av = (i32x8){(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
      }
      f32x4 c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0,
                                                                  127, 0, 127);
      if (FIX) c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bc, c, 0, 0, 0, 127, 0, 127);
      // rows of c: hi(t0), lo(t0), hi(t1), lo(t1) for t0 = 2kq, t1 = 2kq+1
      const float sa0 = a.a_scale[srow0[g] + kb];
      const float sa1 = a.a_scale[srow1[g] + kb];
      acc[g][0] = fmaf(fmaf(c[1], 0.0625f, c[0]), sa0 * sw, acc[g][0]);
      acc[g][1] = fmaf(fmaf(c[3], 0.0625f, c[2]), sa1 * sw, acc[g][1]);
    }
  }

#pragma unroll
  for (int g = 0; g < kGroupedTileRows / 8; ++g) {
    if (g >= groups) break;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int tt = g * 8 + 2 * kq + h;
      if (MODE == GEMM_PLAIN) {
        if (col_ok && tt < len) a.out[(start + tt) * a.out_row_stride + col] = f32_to_bf16(acc[g][h]);
      } else {
        // row_ror:8 within each 16-lane row: lane n gets lane (n+8)&15
        float up = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[g][h]), 0x128, 0xF, 0xF, true));
        if (n16 < 8 && col_ok && tt < len)
          a.out[(start + tt) * a.out_row_stride + col] = swiglu_mlx(acc[g][h], up, a.limit);
      }
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GroupedGemmArgs a) {
  if (a.fixup != nullptr && *a.fixup != 0) grouped_gemm_body<MODE, true>(a);
  else grouped_gemm_body<MODE, false>(a);
}

// Sets *flag (pre-cleared by clear_flag_kernel) when any byte of codes is
// 0x7F or 0xFF.
__global__ void clear_flag_kernel(int32_t* flag) { *flag = 0; }

__global__ void or_flags_kernel(int32_t* dst, const int32_t* a, const int32_t* b) { *dst = (*a != 0) | (*b != 0); }

__global__ __launch_bounds__(256) void scan_480_kernel(const uint8_t* codes, int64_t n, int32_t* flag) {
  const int64_t words = n / 16;
  bool hit = false;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < words;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes) + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t t = (q[j] & 0x7F7F7F7Fu) ^ 0x7F7F7F7Fu;
      hit |= (~((t | 0x80808080u) - 0x01010101u) & 0x80808080u) != 0u;
    }
  }
  if (blockIdx.x == 0) {
    for (int64_t i = words * 16 + threadIdx.x; i < n; i += 256) hit |= (codes[i] & 0x7Fu) == 0x7Fu;
  }
  if (hit) atomicOr(flag, 1);
}

// ------------------------------------------------------------ reductions --

// grouped_fp8.py:273-276: y[t] = T(sum_slot float(down[inv[t*k+slot]]) *
// score), FP32 products summed in slot order, optional BF16 shared add.
__global__ __launch_bounds__(256) void restore_reduce_kernel(ReduceArgs a) {
  const int64_t t = blockIdx.y;
  const int64_t h = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (h >= a.H) return;
  float total = 0.0f;
  for (int s = 0; s < a.top_k; ++s) {
    const int32_t pos = a.inverse[t * a.top_k + s];
    const float v = pos < 0 ? __builtin_nanf("") : bf16_to_f32(a.route_out[static_cast<int64_t>(pos) * a.H + h]);
    total = __fadd_rn(total, __fmul_rn(v, a.sorted_score[pos < 0 ? 0 : pos]));
  }
  float r = bf16_round(total);
  if (a.shared != nullptr) r = __fadd_rn(r, bf16_to_f32(a.shared[t * a.H + h]));
  a.out[t * a.H + h] = f32_to_bf16(r);
}

// native_indexer_plan.metal:2174-2207 (fp8.py:384-397 order): per token,
// ascending expert id; contribution = T(down * score); total = T(total + c).
__global__ __launch_bounds__(256) void direct_order_reduce_kernel(ReduceArgs a) {
  const int64_t t = blockIdx.y;
  const int64_t h = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (h >= a.H) return;
  int32_t slot_ids[kMaxReduceTopK];
  int order[kMaxReduceTopK];
  for (int s = 0; s < a.top_k; ++s) {
    slot_ids[s] = a.expert_ids[t * a.top_k + s];
    order[s] = s;
  }
  for (int i = 1; i < a.top_k; ++i) {  // stable insertion sort by expert id
    int v = order[i];
    int j = i - 1;
    while (j >= 0 && slot_ids[order[j]] > slot_ids[v]) {
      order[j + 1] = order[j];
      --j;
    }
    order[j + 1] = v;
  }
  float total = 0.0f;
  for (int r = 0; r < a.top_k; ++r) {
    const int64_t route = t * a.top_k + order[r];
    const int32_t pos = a.inverse[route];
    const float v = pos < 0 ? __builtin_nanf("") : bf16_to_f32(a.route_out[static_cast<int64_t>(pos) * a.H + h]);
    const float c = bf16_round(__fmul_rn(v, a.route_score[route]));
    total = bf16_round(__fadd_rn(total, c));
  }
  float r = total;
  if (a.shared != nullptr) r = __fadd_rn(r, bf16_to_f32(a.shared[t * a.H + h]));
  a.out[t * a.H + h] = f32_to_bf16(r);
}

// ------------------------------------------------------------- launchers --

hipError_t launch_route_plan(const RoutePlanArgs& a, hipStream_t st) {
  if (a.blocks > 0) {
    hipLaunchKernelGGL(route_count_kernel, dim3(static_cast<unsigned>(a.blocks)), dim3(256), 0, st, a);
  }
  hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(1024), 0, st, a);
  if (a.blocks > 0) {
    hipLaunchKernelGGL(route_scatter_kernel, dim3(static_cast<unsigned>(a.blocks)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_split_activations(const SplitArgs& a, hipStream_t st) {
  const int64_t units = a.rows * (a.cols / kBlock);
  if (units == 0) return hipSuccess;
  hipLaunchKernelGGL(split_activations_kernel, dim3(static_cast<unsigned>((units + 3) / 4)), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_grouped_gemm(const GroupedGemmArgs& a, int mode, int64_t descriptors, hipStream_t st) {
  if (descriptors == 0) return hipSuccess;
  if (mode == GEMM_PLAIN) {
    dim3 grid(static_cast<unsigned>((a.N + 63) / 64), static_cast<unsigned>(descriptors));
    hipLaunchKernelGGL(grouped_gemm_kernel<GEMM_PLAIN>, grid, dim3(256), 0, st, a);
  } else {
    dim3 grid(static_cast<unsigned>((a.N + 31) / 32), static_cast<unsigned>(descriptors));
    hipLaunchKernelGGL(grouped_gemm_kernel<GEMM_SWIGLU>, grid, dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_scan_480(const uint8_t* codes, int64_t n, int32_t* flag, bool clear, hipStream_t st) {
  if (clear) hipLaunchKernelGGL(clear_flag_kernel, dim3(1), dim3(1), 0, st, flag);
  if (n > 0) {
    int64_t blocks = (n / 16 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL(scan_480_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, codes, n, flag);
  }
  return hipGetLastError();
}

hipError_t launch_or_flags(int32_t* dst, const int32_t* a, const int32_t* b, hipStream_t st) {
  hipLaunchKernelGGL(or_flags_kernel, dim3(1), dim3(1), 0, st, dst, a, b);
  return hipGetLastError();
}

hipError_t launch_reduce(const ReduceArgs& a, bool direct_order, hipStream_t st) {
  if (a.tokens == 0) return hipSuccess;
  dim3 grid(static_cast<unsigned>((a.H + 255) / 256), static_cast<unsigned>(a.tokens));
  if (direct_order) hipLaunchKernelGGL(direct_order_reduce_kernel, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(restore_reduce_kernel, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace glm53
