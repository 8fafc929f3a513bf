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
//  * Grouped GEMM (grouped_fp8.py:30-140): gfx950 v_mfma_scale_f32_16x16x128
//    with raw E4M3 weight codes as the B operand (no decode) and the hi/lo
//    activation rows as the A operand, both streamed from HBM into an LDS
//    ring by direct global->LDS loads.  Two chained MFMAs (hi rows, then lo
//    rows) cover one 128-deep scale block, the activation scale riding as
//    the MFMA's E8M0 row scale; their result, times the weight block scale,
//    accumulates in FP32 registers.
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

// Inclusive scans of a[0..n) and b[0..n) in LDS (n <= 1024, 1024 threads,
// all of them calling): a shuffle scan inside each wavefront, then each
// thread adds the totals of the wavefronts before it.
__device__ void block_scan2_inclusive(unsigned* a, unsigned* b, int n) {
  __shared__ unsigned wave_a[16], wave_b[16];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  unsigned x = t < n ? a[t] : 0u, y = t < n ? b[t] : 0u;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned xo = __shfl_up(x, off), yo = __shfl_up(y, off);
    if (lane >= off) {
      x += xo;
      y += yo;
    }
  }
  if (lane == 63) {
    wave_a[w] = x;
    wave_b[w] = y;
  }
  __syncthreads();
  for (int i = 0; i < w; ++i) {
    x += wave_a[i];
    y += wave_b[i];
  }
  if (t < n) {
    a[t] = x;
    b[t] = y;
  }
  __syncthreads();
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
    int64_t b = 0;
    for (; b + 32 <= a.blocks; b += 32) {  // 32 loads in flight per round trip
      unsigned c[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) c[j] = a.block_counts[(b + j) * a.experts + t];
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        a.block_counts[(b + j) * a.experts + t] = run;
        run += c[j];
      }
    }
    for (; b + 8 <= a.blocks; b += 8) {
      unsigned c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = a.block_counts[(b + j) * a.experts + t];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a.block_counts[(b + j) * a.experts + t] = run;
        run += c[j];
      }
    }
    for (; b < a.blocks; ++b) {
      unsigned c = a.block_counts[b * a.experts + t];
      a.block_counts[b * a.experts + t] = run;
      run += c;
    }
    route_cum[t] = run;
    tile_cum[t] = (run + a.tile_rows - 1) / a.tile_rows;
  }
  for (int64_t b = t; b < a.blocks; b += 1024) atomicAdd(&invalid_total, a.block_invalid[b]);
  __syncthreads();
  block_scan2_inclusive(route_cum, tile_cum, a.experts);
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

// Hardware E4M3 conversion of a pair (q0, q1), both |q| <= 448, into bytes
// 0-1 (kUpper false) or 2-3 of hi_word, and of their residuals 16 (q - hi)
// into the same bytes of lo_word; the other bytes are kept.
template <bool kUpper>
__device__ __forceinline__ void encode_pair_e4m3(float q0, float q1, uint32_t& hi_word, uint32_t& lo_word) {
  const int h = __builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, static_cast<int>(hi_word), kUpper);
  hi_word = static_cast<uint32_t>(h);
  const float r0 = (q0 - __builtin_amdgcn_cvt_f32_fp8(h, kUpper ? 2 : 0)) * 16.0f;
  const float r1 = (q1 - __builtin_amdgcn_cvt_f32_fp8(h, kUpper ? 3 : 1)) * 16.0f;
  lo_word = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(r0, r1, static_cast<int>(lo_word), kUpper));
}

// V consecutive BF16 values as raw words: V = 8 is one 16-byte load (the
// pointer 16-byte aligned), V = 1 or 2 are 2-byte loads.
template <int V>
struct Bf16Run {
  uint32_t w[(V + 1) / 2];
  __device__ __forceinline__ void load(const uint16_t* p) {
    if constexpr (V == 8) {
      const uint4 r = *reinterpret_cast<const uint4*>(p);
      w[0] = r.x, w[1] = r.y, w[2] = r.z, w[3] = r.w;
    } else {
#pragma unroll
      for (int i = 0; i < (V + 1) / 2; ++i) w[i] = 0u;
#pragma unroll
      for (int i = 0; i < V; ++i) w[i >> 1] |= static_cast<uint32_t>(p[i]) << (16 * (i & 1));
    }
  }
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int i = 0; i < (V + 1) / 2; ++i) w[i] = 0u;
  }
  __device__ __forceinline__ float get(int i) const {
    return __uint_as_float(i & 1 ? (w[i >> 1] & 0xffff0000u) : (w[i >> 1] << 16));
  }
};

// Rounds V floats to BF16 and stores them (one 16-byte store for V = 8).
template <int V>
__device__ __forceinline__ void store_bf16_run(uint16_t* p, const float* v) {
  if constexpr (V == 8) {
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = static_cast<uint32_t>(f32_to_bf16(v[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(v[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(o[0], o[1], o[2], o[3]);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) p[i] = f32_to_bf16(v[i]);
  }
}

// Wavefront = one row x (V / 2) consecutive 128-column blocks; lane l holds
// V columns of block l / (128 / V).  V = 8 (16-byte loads, each block's amax
// a reduction over one 16-lane DPP row) when the rows are 16-byte aligned,
// V = 2 (one block per wavefront) otherwise.
template <int V>
__global__ __launch_bounds__(256) void split_activations_kernel(SplitArgs a) {
  constexpr int kLanesPerBlock = kBlock / V;
  constexpr int kBlocksPerWave = 64 / kLanesPerBlock;
  const int lane = threadIdx.x & 63;
  const int64_t blocks_per_row = a.cols / kBlock;
  const int64_t groups = (blocks_per_row + kBlocksPerWave - 1) / kBlocksPerWave;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (unit >= a.rows * groups) return;
  const int64_t row = unit / groups;
  const int64_t blk = (unit % groups) * kBlocksPerWave + lane / kLanesPerBlock;
  const bool valid = blk < blocks_per_row;
  const int64_t col = blk * kBlock + V * (lane % kLanesPerBlock);
  Bf16Run<V> x;
  x.clear();
  if (valid) x.load(a.x + row * a.x_row_stride + col);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) amax = fmaxf(amax, fabsf(x.get(i)));
  if constexpr (kLanesPerBlock == 64) {
    amax = wave_max(amax);
  } else {
    static_assert(kLanesPerBlock == 16, "a block spans one DPP row or the whole wavefront");
    amax = fmaxf(amax, dpp_f32<0xB1>(amax));   // quad_perm [1,0,3,2]
    amax = fmaxf(amax, dpp_f32<0x4E>(amax));   // quad_perm [2,3,0,1]
    amax = fmaxf(amax, dpp_f32<0x141>(amax));  // row_half_mirror
    amax = fmaxf(amax, dpp_f32<0x140>(amax));  // row_mirror: the block's amax in all 16 lanes
  }
  // s = 2^ceil(log2(amax / 448)): amax / s lies in (224, 448].
  float s = 1.0f;
  if (amax > 0.0f && isfinite(amax)) {
    int e = ilogbf(amax / 448.0f);
    if (e < -126) e = -126;
    s = ldexpf(1.0f, e);
    if (amax / s > 448.0f) s = ldexpf(1.0f, e + 1);
  }
  const float inv = 1.0f / s;
  float q[V];
  bool in_range = true;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    q[i] = x.get(i) * inv;
    in_range = in_range && fabsf(q[i]) <= 448.0f;
  }
  uint32_t hi[(V + 3) / 4] = {}, lo[(V + 3) / 4] = {};
  if (in_range) {
    // Every |q| <= 448 is on the E4M3 range, where the hardware conversion
    // (OCP E4M3, round to nearest even) is encode_e4m3; the residual
    // |q - hi| <= 16 makes 16 (q - hi) lie within +-256.
#pragma unroll
    for (int w = 0; w < (V + 3) / 4; ++w) {
      encode_pair_e4m3<false>(q[4 * w], q[4 * w + 1], hi[w], lo[w]);
      if constexpr (V >= 4) encode_pair_e4m3<true>(q[4 * w + 2], q[4 * w + 3], hi[w], lo[w]);
    }
  } else {  // a non-finite or saturating value in this lane
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const uint32_t h = encode_e4m3(q[i]);
      const uint32_t l = encode_e4m3((q[i] - e4m3_value(h)) * 16.0f);
      hi[i >> 2] |= h << (8 * (i & 3));
      lo[i >> 2] |= l << (8 * (i & 3));
    }
  }
  if (!valid) return;
  const int64_t off = row * a.cols + col;
  if constexpr (V == 8) {
    *reinterpret_cast<uint2*>(a.hi + off) = make_uint2(hi[0], hi[1]);
    *reinterpret_cast<uint2*>(a.lo + off) = make_uint2(lo[0], lo[1]);
  } else {
    static_assert(V == 2, "narrow split handles two columns per lane");
    *reinterpret_cast<uint16_t*>(a.hi + off) = static_cast<uint16_t>(hi[0]);
    *reinterpret_cast<uint16_t*>(a.lo + off) = static_cast<uint16_t>(lo[0]);
  }
  if (lane % kLanesPerBlock == 0) a.scale[row * blocks_per_row + blk] = s;
}

// --------------------------------------------------------- grouped GEMM --
//
// Workgroup = 4 wavefronts on one work item: one descriptor (32 GPW routes
// of one expert, 2 GPW pairs of 16) times one 128-row weight tile.  Per
// 128-deep K block (a "stage"):
//   * B: the tile's 128 weight rows of raw E4M3 codes (16 KB),
//   * A: per 16-route pair, one 16-row operand tile of the routes' hi rows
//     and one of their lo rows, gathered through the sorted token index
//     (2 x 2 KB),
// both brought straight from global memory into an LDS ring by direct loads
// (global_load_lds_dwordx4: lane l's 16 bytes land at base + 16 l), so no
// registers hold data in flight and the ring's other stages stream while
// one is multiplied.  Each direct load reads 8 rows as whole 128-byte lines
// (a 16-row operand tile takes two); in LDS a row's 16-byte pieces are
// permuted by an XOR of the row index, so the MFMA lane (r = l % 16, q =
// l / 16) reads its 32 operand bytes (row r, bytes 32 q .. 32 q + 31) as two
// conflict-free 16-byte LDS reads (operand_slots).  Whole lines per load
// stream weight tiles about 14% faster than 64 bytes of 16 rows per load.
// Per (pair, weight tile) two chained v_mfma_scale_f32_16x16x128_f8f6f4
// (pair_pass): hi rows x tile, then lo rows x tile added into the same
// result, with the route's activation block scale (a power of two) as the A
// rows' E8M0 scale and the lo pass's 1/16 as the B scale; the result, times
// the tile's weight block scale, accumulates in FP32 (one FMA per element).
// Lane l holds routes 4 (l / 16) .. 4 (l / 16) + 3 of the pair in column
// l % 16 of the tile.  Two shapes: GPW = 2 (64-route descriptors, 2-stage
// ring; wavefront w multiplies pair w against the 8 tiles) for many routes
// per expert, GPW = 1 (32 routes, 3-stage ring; wavefront w multiplies pair
// w / 2 against half of the tiles) otherwise.  Every shape computes each
// output element by the same sequence of operations, so all give the same
// bits.
//
// mode GEMM_PLAIN : the tile is output columns [128 tile, +128).
// mode GEMM_SWIGLU: the tile is gate rows j in [64 tile, +64) (tiles 0-3)
//   and the matching up rows (tiles 4-7), so h = SwiGLU(T(gate), T(up))
//   forms in registers.
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

namespace {

constexpr int kTileRows = 128;                     // weight rows per work item
constexpr int kOperand = 2048;                     // one 16-row x 128-byte operand tile in LDS
constexpr int kStageB = (kTileRows / 16) * kOperand;  // 16 KB
// LDS ring depth of each shape: two slots (48 KB for 32-route
// descriptors, whose stages stream through registers kRegAhead stages
// ahead; 64 KB for 64-route descriptors, whose direct loads keep one stage
// in flight); two workgroups per CU either way.
template <int GPW>
constexpr int ring_stages() {
  return 2;
}
// Stages the register-staged shape (GPW = 1) keeps in flight in registers
constexpr int kRegAhead = 2;
// Descriptors of 32 GPW routes: 2 GPW pairs of 16, i.e. 4 GPW activation
// operand tiles (hi and lo rows of each pair) per stage
template <int GPW>
constexpr int stage_bytes() {
  return kStageB + 4 * GPW * kOperand;
}
static_assert(kGemmTileRows == 64 && kGemmMinTileRows == 32, "descriptor sizes of the two GEMM shapes");

// Direct global -> LDS load of 16 bytes per lane; lane l writes lds_base +
// 16 l (lds_base wave-uniform).  Written as inline assembly so that the only
// wait on it is the counted one in stage_barrier: the compiler otherwise
// drains every direct load before any LDS read it cannot prove disjoint.
__device__ __forceinline__ void lds_direct16(const uint8_t* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_base) : "memory", "m0");
}

// The same load addressed as base + off: base wave-uniform (held in SGPRs),
// off a per-lane unsigned 32-bit offset, so a loop-invariant source costs
// one VGPR instead of a 64-bit address pair.
__device__ __forceinline__ void lds_direct16_at(const uint8_t* base, uint32_t off, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_base)
               : "memory", "m0");
}

// Waits until at most N of this wavefront's vector-memory loads are in
// flight and its LDS reads have returned, then joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// LDS layout of one 16-row x 128-byte operand tile: row r's 16-byte piece p
// sits in slot p ^ (r % 8) ^ (r / 8) of the row's 128 bytes, so the two
// direct loads that fill a tile each read 8 rows as whole 128-byte lines
// (lane l: row l / 8, slot l % 8).  The MFMA reads below (lane l: row
// l % 16, pieces 2 (l / 16) and 2 (l / 16) + 1) run at the LDS's full
// 16-byte read rate with this permutation: a read probe of the operand
// pattern measured ~210 bytes per clock per CU, the rate of 64 consecutive
// 16-byte reads, against ~120 for slot p ^ ((r / 2) % 8), though both give
// every 16 consecutive lanes distinct banks.
struct OperandSlots {
  uint32_t lo, hi;  // byte offsets of the lane's two pieces in a tile
};
__device__ __forceinline__ OperandSlots operand_slots(int lane) {
  const int r = lane & 15, kq = lane >> 4, g = (r & 7) ^ (r >> 3);
  return {static_cast<uint32_t>(128 * r + 16 * ((2 * kq) ^ g)), static_cast<uint32_t>(128 * r + 16 * ((2 * kq + 1) ^ g))};
}
// Byte offset, within its row's 128-byte K block, of the piece lane l loads
// in load h (0: rows 0-7, 1: rows 8-15) of a tile; its row is 8 h + l / 8,
// its slot l % 8, so the piece is (l % 8) ^ (l / 8) ^ h: load 1's offset is
// load 0's with bit 4 flipped.
__device__ __forceinline__ int load_piece_offset(int lane, int h) {
  return 16 * ((lane & 7) ^ (lane >> 3) ^ h);
}

__device__ __forceinline__ i32x8 lds_operand(const uint8_t* tile, OperandSlots o) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(tile + o.lo);
  const u32x4 hi = *reinterpret_cast<const u32x4*>(tile + o.hi);
  return (i32x8){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// E8M0 code of an activation block scale: the split's scales are powers of
// two 2^e, -126 <= e <= 127, whose FP32 exponent field e + 127 is the code.
__device__ __forceinline__ uint32_t scale_e8m0(float s) { return (__float_as_uint(s) >> 23) & 0xFFu; }

// A weight tile's B operand as the MFMA takes it: FIX feeds codes 0x7F /
// 0xFF as 0x7E / 0xFE and returns the +-32 corrections in bc.
template <bool FIX>
__device__ __forceinline__ void weight_operand(i32x8& b, i32x8& bc) {
  bc = (i32x8){0, 0, 0, 0, 0, 0, 0, 0};
  if (FIX) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t f, cr;
      split_480(static_cast<uint32_t>(b[i]), f, cr);
      b[i] = static_cast<int>(f);
      bc[i] = static_cast<int>(cr);
    }
  }
}

// One pass of a 16-route pair over a weight tile: rows a (the pair's hi or
// lo rows) times b (FIX: plus the corrections bc) added into c.  The A rows'
// E8M0 scale is byte OPSEL of se (the lane's route), the B scale SB (127:
// 1 for the hi rows, 123: 1/16 for the lo rows).
template <bool FIX, int OPSEL, int SB>
__device__ __forceinline__ f32x4 pair_pass(const i32x8& a, const i32x8& b, const i32x8& bc, f32x4 c, int se) {
  c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, OPSEL, se, 0, SB);
  if (FIX) c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, bc, c, 0, 0, OPSEL, se, 0, SB);
  return c;
}
// pair_pass with the scale byte chosen by a value that unrolling makes constant
template <bool FIX, int SB>
__device__ __forceinline__ f32x4 pair_pass_byte(int byte, const i32x8& a, const i32x8& b, const i32x8& bc, f32x4 c,
                                                int se) {
  switch (byte) {
    case 0: return pair_pass<FIX, 0, SB>(a, b, bc, c, se);
    case 1: return pair_pass<FIX, 1, SB>(a, b, bc, c, se);
    case 2: return pair_pass<FIX, 2, SB>(a, b, bc, c, se);
    default: return pair_pass<FIX, 3, SB>(a, b, bc, c, se);
  }
}

}  // namespace

// What a work item reads and writes: the routed problem's operands or the
// dense problem's (GroupedGemmArgs.x_*), chosen per item.
struct ItemSource {
  const uint8_t* a_hi;
  const uint8_t* a_lo;
  const float* a_scale;
  const int32_t* a_row_index;
  int64_t routes;
  const int32_t* tile_expert;
  const int32_t* tile_start;
  const int32_t* tile_len;
  int64_t experts;
  const uint8_t* weight;
  const uint8_t* weight_up;
  int wg;  // row groups of the weight matrices (common.h)
  const float* scale;
  const float* scale_up;
  uint16_t* out;
  int64_t out_row_stride;
};

// Stores a wavefront's BF16 results: v[j][t][i / 2] holds, in its low half
// for even i and its high half for odd i, route 16 (p0 + pstep j) + 4 (l /
// 16) + i of the item and output column c0 + 16 t + l % 16.  Buffer stores
// against a record that ends after the item's len rows: a route past len
// lies outside it, a column past N is given an offset outside it, and the
// hardware drops both, so the stores need no branches.  (The host keeps
// out_row_stride below 2^22, so every offset fits 32 bits.)
template <int NP, int T>
__device__ __forceinline__ void store_item_rows(const ItemSource& src, int32_t start, int32_t len, int p0, int pstep,
                                                int64_t c0, int64_t N, const uint32_t (&v)[NP > 0 ? NP : 1][T][2],
                                                int lane) {
  const int n16 = lane & 15, kq = lane >> 4;
  const uint32_t stride2 = 2u * static_cast<uint32_t>(src.out_row_stride);
  const __amdgpu_buffer_rsrc_t rec = __builtin_amdgcn_make_buffer_rsrc(
      src.out + static_cast<int64_t>(start) * src.out_row_stride, 0, static_cast<int>(stride2 * len), 0x00020000);
  uint32_t coff[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t c = c0 + 16 * t + n16;
    coff[t] = c < N ? 2u * static_cast<uint32_t>(c) : 0x80000000u;
  }
#pragma unroll
  for (int j = 0; j < NP; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t roff = stride2 * static_cast<uint32_t>(16 * (p0 + pstep * j) + 4 * kq + i);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint16_t bits = static_cast<uint16_t>(i & 1 ? v[j][t][i >> 1] >> 16 : v[j][t][i >> 1]);
        __builtin_amdgcn_raw_buffer_store_b16(bits, rec, static_cast<int>(roff + coff[t]), 0, 0);
      }
    }
}

// SWIGLU epilogue of a wavefront: pair j of the wavefront is descriptor
// pair p0 + pstep j; lane l holds, for its routes 16 p + 4 (l / 16) + i,
// gate tiles 0 .. T - 1 in acc[j][t] and the matching up tiles in
// acc[j][t + T]; output column c0 + 16 t + l % 16.  Every value takes the
// straight-line form, two at a time; a wavefront with a value outside its
// range (|T(g)| > 87, NaN or T(g) = 0xC0DB: rare) recomputes all of its
// values with swiglu_mlx.
template <int NP, int T>
__device__ __forceinline__ void swiglu_epilogue(const GroupedGemmArgs& a, const ItemSource& src, int32_t start,
                                                int32_t len, int p0, int pstep, int64_t c0,
                                                const float (&acc)[NP > 0 ? NP : 1][2 * T][4], int lane) {
  uint32_t h[NP > 0 ? NP : 1][T][2];
  SwigluCheck check;
#pragma unroll
  for (int j = 0; j < NP; ++j)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int q = 0; q < 2; ++q)
        h[j][t][q] = swiglu_mlx_straight2(acc[j][t][2 * q], acc[j][t + T][2 * q], acc[j][t][2 * q + 1],
                                          acc[j][t + T][2 * q + 1], a.limit, check);
  if (__builtin_amdgcn_ballot_w64(!swiglu_straight_ok(check, a.limit)) != 0) {
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          h[j][t][q] = swiglu_mlx(acc[j][t][2 * q], acc[j][t + T][2 * q], a.limit) |
                       static_cast<uint32_t>(swiglu_mlx(acc[j][t][2 * q + 1], acc[j][t + T][2 * q + 1], a.limit)) << 16;
  }
  store_item_rows<NP, T>(src, start, len, p0, pstep, c0, a.N, h, lane);
}

// PLAIN epilogue of a wavefront: acc[j][t] holds output columns c0 + 16 t
// + l % 16 of routes 16 (p0 + pstep j) + 4 (l / 16) + i, stored as BF16.
template <int NP, int T>
__device__ __forceinline__ void plain_epilogue(const GroupedGemmArgs& a, const ItemSource& src, int32_t start,
                                               int32_t len, int p0, int pstep, int64_t c0,
                                               const float (&acc)[NP > 0 ? NP : 1][T][4], int lane) {
  uint32_t h[NP > 0 ? NP : 1][T][2];
#pragma unroll
  for (int j = 0; j < NP; ++j)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int q = 0; q < 2; ++q) h[j][t][q] = f32x2_to_bf16x2(acc[j][t][2 * q], acc[j][t][2 * q + 1]);
  store_item_rows<NP, T>(src, start, len, p0, pstep, c0, a.N, h, lane);
}

// Wavefront w's share of a work item: it loads weight tiles 2 w, 2 w + 1 and
// activation tiles GPW w .. GPW w + GPW - 1 of every stage (NL of them: none
// when their pair has no routes), and multiplies one pair (NP = 1; NP = 0
// when the pair has no routes) against T weight tiles: GPW = 2 pair w
// against all 8 tiles, GPW = 1 pair w / 2 against the tiles of half h =
// w % 2 (PLAIN: tiles 4 h .. 4 h + 3; SWIGLU: gate tiles 2 h, 2 h + 1 and
// the matching up tiles).
template <int MODE, bool FIX, int GPW, int NP>
__device__ __forceinline__ void grouped_gemm_loop(const GroupedGemmArgs& a, const ItemSource src, int64_t ntile,
                                                  int32_t start, int32_t len, int64_t KB,
                                                  const uint8_t* const (&gb)[2][2], const uint8_t* const (&ga)[GPW][2],
                                                  uint8_t* lds, uint32_t lds_addr, const uint8_t* lds_se,
                                                  const float* lds_sw, int wave, int lane) {
  constexpr int kStage = stage_bytes<GPW>();
  constexpr int kRoutes = 32 * GPW;
  constexpr int NL = GPW == 2 ? 2 * NP : NP;  // activation tiles this wavefront loads per stage
  constexpr int P = 4 + 2 * NL;               // its direct loads per stage
  constexpr int T = GPW == 2 ? 8 : 4;         // weight tiles it multiplies
  const int pair = GPW == 2 ? wave : wave >> 1;
  const int half = wave & 1;
  const OperandSlots slots = operand_slots(lane);
  auto issue = [&](int64_t kb, int slot) {
    const int64_t ko = kb * kBlock;        // activation rows: row-major
    const int64_t kw = kb << (7 + src.wg);  // weight rows: K block kb of the row group
    const uint32_t sb = lds_addr + slot * kStage + 2 * wave * kOperand;
    lds_direct16(gb[0][0] + kw, sb);
    lds_direct16(gb[0][1] + kw, sb + 1024);
    lds_direct16(gb[1][0] + kw, sb + kOperand);
    lds_direct16(gb[1][1] + kw, sb + kOperand + 1024);
    const uint32_t sa = lds_addr + slot * kStage + kStageB + GPW * wave * kOperand;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      lds_direct16(ga[j][0] + ko, sa + j * kOperand);
      lds_direct16(ga[j][1] + ko, sa + j * kOperand + 1024);
    }
  };
  // the LDS weight tile of local tile tt, and whether it holds up rows
  auto tile_of = [&](int tt) {
    if (GPW == 2) return tt;
    return MODE == GEMM_PLAIN ? 4 * half + tt : (tt < 2 ? 2 * half + tt : 4 + 2 * half + tt - 2);
  };
  auto up_tile = [&](int tt) { return MODE == GEMM_SWIGLU && tt >= T / 2; };

  float acc[NP > 0 ? NP : 1][T][4];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[0][t][i] = 0.0f;

  // one stage's MFMAs on the operands in LDS slot `slot`
  auto compute = [&](int64_t kb, int slot) {
    if (NP > 0) {
      const uint8_t* st = lds + slot * kStage;
      const i32x8 ahi = lds_operand(st + kStageB + (2 * pair) * kOperand, slots);
      const i32x8 alo = lds_operand(st + kStageB + (2 * pair + 1) * kOperand, slots);
      const int se = lds_se[kb * kRoutes + 16 * pair + (lane & 15)];
      const float sw_lo = lds_sw[kb];
      const float sw_hi = MODE == GEMM_SWIGLU ? lds_sw[KB + kb] : sw_lo;
      i32x8 bq[T], bc[T];  // every weight tile read ahead: one LDS wait per stage
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        bq[tt] = lds_operand(st + tile_of(tt) * kOperand, slots);
        weight_operand<FIX>(bq[tt], bc[tt]);
      }
      // Each tile's hi pass issues T MFMAs before its lo pass reads the
      // result, and tile tt is folded into the accumulators after tile
      // tt + 1's lo pass is issued: the MFMAs of a stage issue back to back
      // while the folding runs beside them.
      f32x4 c[T];
#pragma unroll
      for (int tt = 0; tt < T; ++tt)
        c[tt] = pair_pass<FIX, 0, 127>(ahi, bq[tt], bc[tt], (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, se);
      auto fold = [&](int tt) {
        const float sw = up_tile(tt) ? sw_hi : sw_lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[0][tt][i] = fmaf(c[tt][i], sw, acc[0][tt][i]);
      };
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        c[tt] = pair_pass<FIX, 0, 123>(alo, bq[tt], bc[tt], c[tt], se);
        if (tt > 0) fold(tt - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      fold(T - 1);
    }
  };

  constexpr int kStages = ring_stages<GPW>();
  if constexpr (GPW == 1) {
    // Register-staged stream: each stage's operand bytes come with plain
    // 16-byte loads (the same 8 rows x 128 bytes per instruction as the
    // direct loads) kRegAhead stages ahead into registers and are written to
    // the LDS slot at the positions the direct loads would fill; a 2-slot
    // ring, one barrier per stage.  Every load is compiler-visible, so each
    // wait is the exact one.  A weight-streaming read probe moved 6.4-6.5
    // TB/s this way against 5.6-5.8 TB/s with direct loads.
    static_assert(kStages == 2, "the register-staged shape double-buffers its LDS");
    struct Staged {
      u32x4 b[4];
      u32x4 a[NL > 0 ? 2 * NL : 1];
    };
    auto load = [&](int64_t kb, Staged& r) {
      const int64_t ko = kb * kBlock;
      const int64_t kw = kb << (7 + src.wg);
      r.b[0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gb[0][0] + kw));
      r.b[1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gb[0][1] + kw));
      r.b[2] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gb[1][0] + kw));
      r.b[3] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gb[1][1] + kw));
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        r.a[2 * j] = *reinterpret_cast<const u32x4*>(ga[j][0] + ko);
        r.a[2 * j + 1] = *reinterpret_cast<const u32x4*>(ga[j][1] + ko);
      }
    };
    auto store = [&](int slot, const Staged& r) {
      uint8_t* sb = lds + slot * kStage + 2 * wave * kOperand + 16 * lane;
      *reinterpret_cast<u32x4*>(sb) = r.b[0];
      *reinterpret_cast<u32x4*>(sb + 1024) = r.b[1];
      *reinterpret_cast<u32x4*>(sb + kOperand) = r.b[2];
      *reinterpret_cast<u32x4*>(sb + kOperand + 1024) = r.b[3];
      uint8_t* sa = lds + slot * kStage + kStageB + GPW * wave * kOperand + 16 * lane;
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        *reinterpret_cast<u32x4*>(sa + j * kOperand) = r.a[2 * j];
        *reinterpret_cast<u32x4*>(sa + j * kOperand + 1024) = r.a[2 * j + 1];
      }
    };
    // stage kb's bytes sit in r[kb % kRegAhead] until written to slot kb % 2;
    // stages past the last K block are never loaded or written
    // prologue loads are unconditional too: a block index past the last
    // K block re-reads the last one (only when KB <= kRegAhead), never stored
    auto clamp_kb = [&](int64_t kb) { return kb < KB ? kb : KB - 1; };
    Staged r[kRegAhead];
#pragma unroll
    for (int q = 0; q < kRegAhead; ++q) load(clamp_kb(q), r[q]);
    store(0, r[0]);
    load(clamp_kb(kRegAhead), r[0]);
    // Each stage: wait at the barrier (slot kb % 2 written by every
    // wavefront, all done reading slot (kb + 1) % 2, stage kb - 1), write
    // stage kb + 1 into that slot, load stage kb + 1 + kRegAhead into the
    // registers it leaves, multiply stage kb.  The main loop's loads are
    // unconditional, so the compiler's count of the loads in flight stays
    // exact (a conditional load made it wait for all of them).
    int64_t kb0 = 0;
    for (; kb0 + 2 * kRegAhead < KB; kb0 += kRegAhead) {
#pragma unroll
      for (int q = 0; q < kRegAhead; ++q) {
        const int64_t kb = kb0 + q;
        const int qn = (q + 1) % kRegAhead;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        store(static_cast<int>((kb + 1) & 1), r[qn]);
        load(kb + 1 + kRegAhead, r[qn]);
        compute(kb, static_cast<int>(kb & 1));
      }
    }
    for (; kb0 < KB; kb0 += kRegAhead) {
#pragma unroll
      for (int q = 0; q < kRegAhead; ++q) {
        const int64_t kb = kb0 + q;
        if (kb >= KB) break;
        const int qn = (q + 1) % kRegAhead;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (kb + 1 < KB) {
          store(static_cast<int>((kb + 1) & 1), r[qn]);
          if (kb + 1 + kRegAhead < KB) load(kb + 1 + kRegAhead, r[qn]);
        }
        compute(kb, static_cast<int>(kb & 1));
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
      if (s < KB) issue(s, s);
    int slot = 0;
    for (int64_t kb = 0; kb < KB; ++kb) {
      if (kb + kStages - 2 < KB) stage_barrier<P * (kStages - 2)>();
      else stage_barrier<0>();
      if (kb + kStages - 1 < KB) issue(kb + kStages - 1, slot == 0 ? kStages - 1 : slot - 1);
      compute(kb, slot);
      slot = slot == kStages - 1 ? 0 : slot + 1;
    }
  }

  // epilogue: lane holds routes 16 pair + 4 kq + i, column 16 tile + l % 16
  // (PLAIN: the wavefront's tiles tile_of(tt) are contiguous from tile_of(0))
  if (MODE == GEMM_PLAIN)
    plain_epilogue<NP, T>(a, src, start, len, pair, 1, ntile * kTileRows + tile_of(0) * 16, acc, lane);
  if (MODE == GEMM_SWIGLU)
    swiglu_epilogue<NP, T / 2>(a, src, start, len, pair, 1, ntile * (kTileRows / 2) + (GPW == 2 ? 0 : 32 * half), acc,
                               lane);
}

// Activation block scales of a work item's ROUTES routes into LDS as E8M0
// codes, K-block-major: [kb][r], or for the wide shape (WIDE)
// [kb][r % 16][r / 16], so that a lane reads the codes of its row in all
// eight pairs as one 8-byte word.  THREADS / ROUTES
// threads per route, each with its route's token row, eight loads in
// flight per thread, then the stores; indices past the last K block are
// clamped to it, so every load and store is unconditional (a clamped store
// writes the code that block's store writes) and the compiler's wait
// tracking sees every load consumed before the K loop.  Routes past the
// descriptor's end repeat its last route.
template <int ROUTES, int THREADS, bool WIDE>
__device__ __forceinline__ void load_activation_scales(const ItemSource& src, int32_t start, int32_t len,
                                                       int64_t KB, uint8_t* lds_se) {
  constexpr int TPR = THREADS / ROUTES;
  static_assert(TPR * ROUTES == THREADS, "threads split evenly over the routes");
  const int r = static_cast<int>(threadIdx.x) / TPR, sub = static_cast<int>(threadIdx.x) % TPR;
  const int64_t route = start + (r < len ? r : len - 1);
  const int64_t token = src.a_row_index != nullptr ? src.a_row_index[route] : route;
  const float* row = src.a_scale + token * KB;
  const int64_t pos = WIDE ? ((r & 15) * 8 + (r >> 4)) : r;
  constexpr int64_t kStride = WIDE ? 128 : ROUTES;  // bytes per K block
  for (int64_t kb0 = sub; kb0 < KB; kb0 += 8 * TPR) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t kb = kb0 + u * TPR;
      v[u] = row[kb < KB ? kb : KB - 1];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t kb = kb0 + u * TPR;
      lds_se[(kb < KB ? kb : KB - 1) * kStride + pos] = static_cast<uint8_t>(scale_e8m0(v[u]));
    }
  }
}

template <int MODE, bool FIX, int GPW>
__device__ __forceinline__ void grouped_gemm_body(const GroupedGemmArgs& a, const ItemSource src, int64_t ntile, int64_t d,
                                                  uint8_t* lds) {
  constexpr int kRoutes = 32 * GPW;  // routes per descriptor
  constexpr int kStage = stage_bytes<GPW>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  int32_t expert, start, len;
  if (!item_routes<kRoutes>(src, d, expert, start, len)) return;
  const int64_t K = a.K;
  const int64_t KB = K / kBlock;
  const int pairs = (len + 15) >> 4;
  uint8_t* lds_se = lds + ring_stages<GPW>() * kStage;                    // [KB][kRoutes]
  float* lds_sw = reinterpret_cast<float*>(lds_se + kRoutes * KB);        // [2][KB]

  // ---- block scales of the work item: activations of every route, weights
  // of the tile (one 128-row scale block: PLAIN tiles are 128-aligned, SWIGLU
  // tiles 64-aligned within one block)
  auto token_of = [&](int r) -> int64_t {
    const int64_t route = start + (r < len ? r : len - 1);
    return src.a_row_index != nullptr ? src.a_row_index[route] : route;
  };
  load_activation_scales<kRoutes, 256, false>(src, start, len, KB, lds_se);
  const int64_t srow = MODE == GEMM_PLAIN ? ntile : (ntile >> 1);
  const int64_t soff = static_cast<int64_t>(expert) * a.s_expert_stride + srow * a.s_cols;
  for (int64_t i = threadIdx.x; i < (MODE == GEMM_SWIGLU ? 2 : 1) * KB; i += 256)
    lds_sw[i] = i < KB ? src.scale[soff + i] : src.scale_up[soff + i - KB];
  __syncthreads();

  // ---- per-lane global sources of the direct loads: load h of a tile
  // fills its rows 8 h .. 8 h + 7, lane l reading row 8 h + l / 8
  auto b_row = [&](int t, int h) -> const uint8_t* {
    const int rr = 8 * h + (lane >> 3);
    int64_t row;
    const uint8_t* w;
    if (MODE == GEMM_PLAIN) {
      row = ntile * kTileRows + t * 16 + rr;
      w = src.weight;
    } else {
      row = ntile * (kTileRows / 2) + (t & 3) * 16 + rr;
      w = t < 4 ? src.weight : src.weight_up;
    }
    if (row >= a.N) row = a.N - 1;  // rows past the matrix: valid bytes, results never stored
    return w + static_cast<int64_t>(expert) * a.w_expert_stride + group_row_base(row, K, src.wg) +
           load_piece_offset(lane, h);
  };
  const uint8_t* gb[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h) gb[t][h] = b_row(2 * wave + t, h);
  // activation operand tile g: the hi rows (g even) or lo rows (g odd) of
  // pair g / 2; its row rho is route 16 (g / 2) + rho
  const uint8_t* ga[GPW][2];
#pragma unroll
  for (int j = 0; j < GPW; ++j) {
    const int g = GPW * wave + j;
    const uint8_t* plane = (g & 1) ? src.a_lo : src.a_hi;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      ga[j][h] = plane + token_of(16 * (g >> 1) + 8 * h + (lane >> 3)) * K + load_piece_offset(lane, h);
  }
  const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const bool active = (GPW == 2 ? wave : wave >> 1) < pairs;  // wave-uniform: this wavefront's pair holds routes
#define GLM53_LOOP(n) \
  grouped_gemm_loop<MODE, FIX, GPW, n>(a, src, ntile, start, len, KB, gb, ga, lds, lds_addr, lds_se, lds_sw, wave, lane)
  if (active) GLM53_LOOP(1);
  else GLM53_LOOP(0);
#undef GLM53_LOOP
}

template <int GPW>
size_t gemm_lds_bytes(int64_t K) {
  // ring, activation scale codes [KB][32 GPW], weight scales [2][KB]
  return static_cast<size_t>(ring_stages<GPW>()) * stage_bytes<GPW>() +
         (32 * GPW + 2 * sizeof(float)) * static_cast<size_t>(K / kBlock);
}

// The work item w of a launch: its column tile, its descriptor (of the
// routed problem or, past the routed descriptors, of the dense one), the
// operands it reads and whether its weights hold 0x7F/0xFF codes.
__device__ __forceinline__ ItemSource item_source(const GroupedGemmArgs& a, int64_t used, int64_t w, bool desc_major,
                                                  int64_t& ntile, int64_t& d, bool& fix) {
  const int64_t D = used + a.x_descriptors;
  ntile = desc_major ? w % a.n_tiles : w / D;
  d = desc_major ? w / a.n_tiles : w % D;
  const bool dense = d >= used;  // an item of the dense problem
  if (dense) d -= used;
  ItemSource src;
  src.a_hi = dense ? a.x_a_hi : a.a_hi;
  src.a_lo = dense ? a.x_a_lo : a.a_lo;
  src.a_scale = dense ? a.x_a_scale : a.a_scale;
  src.a_row_index = dense ? nullptr : a.a_row_index;
  src.routes = dense ? a.x_routes : a.routes;
  src.tile_expert = dense ? nullptr : a.tile_expert;
  src.tile_start = a.tile_start;
  src.tile_len = a.tile_len;
  src.experts = dense ? 1 : a.experts;
  src.weight = dense ? a.x_weight : a.weight;
  src.weight_up = dense ? a.x_weight_up : a.weight_up;
  src.wg = dense ? a.x_w_group_log2 : a.w_group_log2;
  src.scale = dense ? a.x_scale : a.scale;
  src.scale_up = dense ? a.x_scale_up : a.scale_up;
  src.out = dense ? a.x_out : a.out;
  src.out_row_stride = dense ? a.x_out_row_stride : a.out_row_stride;
  auto set = [](const int32_t* flag) { return flag != nullptr && *flag != 0; };
  fix = dense ? set(a.x_fixup) || set(a.x_fixup_up) : set(a.fixup) || set(a.fixup_up);
  return src;
}

// The descriptor's expert, first route and route count (at most R routes);
// false for an unused descriptor.
template <int R>
__device__ __forceinline__ bool item_routes(const ItemSource& src, int64_t d, int32_t& expert, int32_t& start,
                                            int32_t& len) {
  if (src.tile_expert != nullptr) {
    expert = src.tile_expert[d];
    start = src.tile_start[d];
    len = src.tile_len[d];
    if (start >= src.routes || len <= 0) return false;
    if (expert < 0 || expert >= src.experts) return false;
    if (len > R) len = R;
    if (start + len > src.routes) len = static_cast<int32_t>(src.routes - start);
  } else {
    expert = 0;
    start = static_cast<int32_t>(d * R);
    len = static_cast<int32_t>(src.routes - start < R ? src.routes - start : R);
    if (len <= 0) return false;
  }
  return true;
}

// The routed descriptors in use: the route plan's device count when given
// (clamped to the capacity), else all of them.
__device__ __forceinline__ int64_t used_descriptors(const GroupedGemmArgs& a) {
  if (a.used_descriptors == nullptr) return a.descriptors;
  const int64_t u = static_cast<int64_t>(*a.used_descriptors);
  return u < a.descriptors ? u : a.descriptors;
}

// Work items (column tile, descriptor in use) are dealt to the XCDs in
// contiguous runs: workgroup i runs on XCD i % 8, and item w = (i % 8) *
// ceil(W / 8) + i / 8 keeps neighbouring items on one XCD and its L2.  W
// counts the items of descriptors in use, so every XCD gets the same share
// of real work; the grid is sized for the capacity and its surplus
// workgroups exit at once.  This shape orders items descriptor-major (all
// column tiles of a descriptor, i.e. one expert's whole matrix, in a row:
// its weight rows stream in address order and its activation rows stay in
// L2; config 4 -9%); the wide shape tile-major (descriptors of one heavy
// expert side by side share each weight tile; descriptor-major was 4%
// slower there).
template <int MODE, int GPW>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GroupedGemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];
  const int64_t used = used_descriptors(a);
  const int64_t items = a.n_tiles * (used + a.x_descriptors);
  const int64_t per_xcd = (items + 7) / 8;
  if (static_cast<int64_t>(blockIdx.x / 8) >= per_xcd) return;
  const int64_t w = static_cast<int64_t>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (w >= items) return;
  int64_t ntile, d;
  bool fix;
  const ItemSource src = item_source(a, used, w, true, ntile, d, fix);
  if (fix) grouped_gemm_body<MODE, true, GPW>(a, src, ntile, d, lds_dyn);
  else grouped_gemm_body<MODE, false, GPW>(a, src, ntile, d, lds_dyn);
}

// ------------------------------------------ grouped GEMM, wide shape --
//
// For plans whose experts carry many routes: work item = one 128-route
// descriptor (8 pairs of 16 routes) x 512 weight rows (PLAIN: 512 output
// columns; SWIGLU: 256 gate rows and the matching 256 up rows), one
// 512-thread workgroup per CU (8 wavefronts, two per SIMD).  Wavefront w
// multiplies every pair of the descriptor against its own four 16-row
// weight tiles (PLAIN: output columns 64 w .. 64 w + 63 of the item;
// SWIGLU: gate rows 32 w .. 32 w + 31 and the matching up rows), so all
// wavefronts carry the same work whatever the descriptor's route count.
// The wavefront loads its four tiles itself (direct loads into its own
// 8 KB of a single-buffered 64 KB B stage) and reads them into registers
// during the previous stage's last pair; once those reads have returned it
// issues the next stage's tiles into the same bytes, so the weight stream
// needs no workgroup barrier and runs a stage ahead.  The activations come
// through a 2-stage ring of 32 KB stages (wavefront w loads pair w's hi and
// lo tiles).  One barrier per stage, after each wavefront's last
// activation read of the stage and before its last pair's MFMAs, makes the
// next stage's activation tiles visible and frees this stage's slot; the
// wavefronts leave it with that pair's MFMAs in hand, so the MFMA pipes
// have work while the next stage starts (3-4% faster than a barrier at the
// stage start).  Per stage 8 KB of B and 32 KB of A operand reads for 64
// MFMAs per wavefront.  The arithmetic per output
// element is that of the narrower shapes, so every shape gives the same
// bits.
namespace {
constexpr int kWidePairs = kGemmWideRows / 16;            // 8
constexpr int kWideTilesPerWave = 4;                      // weight tiles per wavefront
constexpr int kWideBTiles = 8 * kWideTilesPerWave;        // 32 tiles: 512 rows
constexpr int kWideBBytes = kWideBTiles * kOperand;       // 64 KB
constexpr int kWideABytes = 2 * kWidePairs * kOperand;    // 32 KB per A stage
constexpr int kWidePlainRows = kWideBTiles * 16;          // 512
constexpr int kWideGateRows = kWidePlainRows / 2;         // 256
}  // namespace

size_t gemm_wide_lds_bytes(int64_t K) {
  // B stage, 2-stage A ring, activation scale codes [KB][128 routes],
  // weight scales [4][KB]
  return static_cast<size_t>(kWideBBytes + 2 * kWideABytes) +
         (kGemmWideRows + 4 * sizeof(float)) * static_cast<size_t>(K / kBlock);
}

// Direct-load sources of a wavefront.  Load h of its tile q covers rows U +
// 0 .. 7 with U = (q < 2 ? rlo : rhi) + 16 (q % 2) + 8 h (a multiple of 8,
// clamped to rows - 8, rows being a multiple of 8); lane l reads row U + l /
// 8 at its piece, and since U is a multiple of 8, group_row_base(U + l / 8)
// = group_row_base(U) + group_row_base(l / 8).  So the wave-uniform part
// wrow[2 q + h] = group_row_base(U) (+ (kb << (7 + wg)) for stage kb) goes
// into the SGPR base and the lane adds woff (h = 0; h = 1 flips bit 4 of the
// piece: woff ^ 16).  Load h of its pair's hi / lo rows reads a_hi / a_lo at
// aoff[h] (token row tok[h] at the lane's piece) + 128 kb.
struct WideSources {
  const uint8_t* wlo;      // PLAIN: the expert's matrix; SWIGLU: its gate rows
  const uint8_t* whi;      // PLAIN: the same matrix; SWIGLU: its up rows
  const uint8_t* a_hi;
  const uint8_t* a_lo;
  int32_t wg;              // row groups of the matrices (common.h)
  int64_t wrow[2 * kWideTilesPerWave];
  uint32_t woff;
  uint32_t aoff[2];
};

// A wave-uniform pointer as the compiler can prove it uniform (so that it
// lives in SGPRs).
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint8_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <int MODE, bool FIX, int NP>
__device__ __forceinline__ void wide_gemm_loop(const GroupedGemmArgs& a, const ItemSource src, int64_t ntile,
                                                int32_t start, int32_t len, int64_t KB, const WideSources& ls,
                                                bool loads_pair, uint8_t* lds, uint32_t lds_addr, const uint8_t* lds_se,
                                                const float* lds_sw, int wave, int lane) {
  constexpr int T = kWideTilesPerWave;
  const OperandSlots slots = operand_slots(lane);
  const uint32_t b_own = static_cast<uint32_t>(wave) * T * kOperand;  // this wavefront's tiles in the B stage
  auto issue_b = [&](int64_t kb) {
    const uint8_t* mlo = ls.wlo + (kb << (7 + ls.wg));
    const uint8_t* mhi = ls.whi + (kb << (7 + ls.wg));
#pragma unroll
    for (int q = 0; q < T; ++q)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        lds_direct16_at((q < 2 ? mlo : mhi) + ls.wrow[2 * q + h], ls.woff ^ (16 * h),
                        lds_addr + b_own + q * kOperand + 1024 * h);
  };
  auto issue_b_tile = [&](int64_t kb, int q) {
    const uint8_t* m = (q < 2 ? ls.wlo : ls.whi) + (kb << (7 + ls.wg));
#pragma unroll
    for (int h = 0; h < 2; ++h)
      lds_direct16_at(m + ls.wrow[2 * q + h], ls.woff ^ (16 * h), lds_addr + b_own + q * kOperand + 1024 * h);
  };
  auto issue_a = [&](int64_t kb, int slot) {
    if (loads_pair) {
      const uint32_t sa = lds_addr + kWideBBytes + slot * kWideABytes + 2 * wave * kOperand;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        lds_direct16_at(ls.a_hi + kb * kBlock, ls.aoff[h], sa + 1024 * h);
        lds_direct16_at(ls.a_lo + kb * kBlock, ls.aoff[h], sa + kOperand + 1024 * h);
      }
    }
  };
  // weight scale row (of lds_sw) of the wavefront's tile q: PLAIN its
  // 64 rows lie in block (64 w) / 128 of the item; SWIGLU gate tiles in
  // gate block (32 w) / 128, up tiles in the same up block
  const int sw_lo = MODE == GEMM_PLAIN ? (64 * wave) >> 7 : (32 * wave) >> 7;
  const int sw_hi = MODE == GEMM_PLAIN ? sw_lo : 2 + sw_lo;

  float acc[NP][T][4];
#pragma unroll
  for (int j = 0; j < NP; ++j)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][t][i] = 0.0f;

  // Stage 0 (B and A) was issued by wide_gemm_body, before the block
  // scales, and has landed in every wavefront (the body waited for its own
  // loads before the barrier that published the scales).  The wavefront's
  // B tiles of a stage are read into registers during the previous stage's
  // last pair, each as soon as that pair's last MFMA on the tile has
  // issued (its own direct loads waited for; no barrier: no other
  // wavefront reads them), so a stage starts on its MFMAs at once and its
  // B bytes take the next stage.
  i32x8 bq[T];
#pragma unroll
  for (int q = 0; q < T; ++q) bq[q] = lds_operand(lds + b_own + q * kOperand, slots);
  i32x8 ahi_next = lds_operand(lds + kWideBBytes, slots);
  i32x8 alo_next = lds_operand(lds + kWideBBytes + kOperand, slots);
  int slot = 0;
  for (int64_t kb = 0; kb < KB; ++kb) {
    // the other slot's stage (kb - 1) was read out by every wavefront before
    // the barrier in its last pair, and this wavefront's B tiles of stage kb
    // are in registers: stage kb + 1 goes in, A first (the barrier's count
    // leaves B's 2 T loads in flight).  With more than T pairs the B tiles
    // go out one per pair instead, each after the pair's hi pass: twelve
    // direct loads at a stage start had the wavefronts stall on the vector
    // memory queue (gate/up -3%, down -4%).  Those issues are unconditional
    // (a branch in the pair loop made the compiler spill), so the last stage
    // reloads its own tiles, unused.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (kb + 1 < KB) {
      issue_a(kb + 1, slot ^ 1);
      if constexpr (NP <= T) issue_b(kb + 1);
    }
    const int64_t kb_next = kb + 1 < KB ? kb + 1 : kb;
    const float w_lo = lds_sw[sw_lo * KB + kb], w_hi = lds_sw[sw_hi * KB + kb];
    // bytes j: the E8M0 scales of this lane's route in pairs j (lo word) and 4 + j (hi word)
    const uint2 se2 = *reinterpret_cast<const uint2*>(lds_se + kb * kGemmWideRows + (lane & 15) * 8);
    const uint8_t* st = lds + kWideBBytes + slot * kWideABytes;
    f32x4 c[T];
    auto fold = [&](int j, int q) {
      const float sw = q < 2 ? w_lo : w_hi;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][q][i] = fmaf(c[q][i], sw, acc[j][q][i]);
    };
    const uint8_t* st_next = lds + kWideBBytes + (slot ^ 1) * kWideABytes;
    // A operands a whole pair ahead: pair j + 1's hi and lo rows (after the
    // last pair: the next stage's first) are read as pair j's lo pass
    // starts, so each pair's operands have had a whole pair's MFMAs to
    // arrive (8 VGPRs more than reading the lo rows at the pair's own start:
    // gate/up -3%, down -3.5%)
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int se = static_cast<int>(j < 4 ? se2.x : se2.y);
      const i32x8 ahi = ahi_next;
      const i32x8 alo = alo_next;
      // Issue priority falls as a wavefront gets ahead in its stage, so of
      // the two on a SIMD the one behind gets the MFMA pipe and they reach
      // the barrier closer together (gate/up -2%).
      if (j == 0) __builtin_amdgcn_s_setprio(3);
      else if (j == 2) __builtin_amdgcn_s_setprio(2);
      else if (j == 4) __builtin_amdgcn_s_setprio(1);
      else if (j == 6) __builtin_amdgcn_s_setprio(0);
      // Every wavefront has read this stage's A and its own share of the
      // next stage's A has landed: the next stage's A is complete, and this
      // stage's slot is free for the stage after.  Each wavefront still
      // holds its last pair's MFMAs, so the pipes have work at the release.
      if (j == NP - 1) stage_barrier<2 * T>();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < T; ++q) {
        if (j > 0) fold(j - 1, q);
        i32x8 b = bq[q], bc;
        weight_operand<FIX>(b, bc);
        c[q] = pair_pass_byte<FIX, 127>(j & 3, ahi, b, bc, (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, se);
      }
      if constexpr (!FIX) {
        // each tile's fold right before its first MFMA (the fold of tile q
        // waits only for tile q's last MFMA of the previous pair, not for
        // tile T - 1's)
        if (j > 0) {
#pragma unroll
          for (int q = 0; q < T; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU: fold(j - 1, q)
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA: tile q's hi pass
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NP > T) {  // tiles 0 .. T - 1 at pairs 0 .. T - 1: all before the last pair's barrier
        if (j < T) issue_b_tile(kb_next, j);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (j + 1 < NP) {
        ahi_next = lds_operand(st + (2 * j + 2) * kOperand, slots);
        alo_next = lds_operand(st + (2 * j + 3) * kOperand, slots);
      } else {  // unused after the last stage
        ahi_next = lds_operand(st_next, slots);
        alo_next = lds_operand(st_next + kOperand, slots);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < T; ++q) {
        i32x8 b = bq[q], bc;
        weight_operand<FIX>(b, bc);
        c[q] = pair_pass_byte<FIX, 123>(j & 3, alo, b, bc, c[q], se);
        if (j == NP - 1) {
          // unconditional (the last stage rereads its own tiles, unused),
          // so that no tile stays live beside its successor
          if (q == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the next stage's B landed
          bq[q] = lds_operand(lds + b_own + q * kOperand, slots);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = 0; q < T; ++q) fold(NP - 1, q);
    slot ^= 1;
  }

  // epilogue: lane holds columns 16 tile + l % 16 of routes 16 j + 4 kq + i
  if (MODE == GEMM_PLAIN) {
    plain_epilogue<NP, T>(a, src, start, len, 0, 1, ntile * kWidePlainRows + 64 * wave, acc, lane);
  } else {
    swiglu_epilogue<NP, T / 2>(a, src, start, len, 0, 1, ntile * kWideGateRows + 32 * wave, acc, lane);
  }
}

template <int MODE, bool FIX>
__device__ __forceinline__ void wide_gemm_body(const GroupedGemmArgs& a, const ItemSource src, int64_t ntile,
                                                int64_t d, uint8_t* lds) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  int32_t expert, start, len;
  if (!item_routes<kGemmWideRows>(src, d, expert, start, len)) return;
  const int64_t K = a.K;
  const int64_t KB = K / kBlock;
  const int pairs = (len + 15) >> 4;
  uint8_t* lds_se = lds + kWideBBytes + 2 * kWideABytes;                    // [KB][128]
  float* lds_sw = reinterpret_cast<float*>(lds_se + kGemmWideRows * KB);    // [4][KB]
  auto token_of = [&](int r) -> int64_t {
    const int64_t route = start + (r < len ? r : len - 1);
    return src.a_row_index != nullptr ? src.a_row_index[route] : route;
  };
  // direct-load sources: load h of a weight tile fills its rows 8 h .. 8 h
  // + 7, lane l reading row r = 8 h + l / 8 at piece (l % 8) ^ (l / 8) ^ h,
  // i.e. the h = 0 offset with bit 0 of the piece flipped for h = 1.  The
  // offsets fit 32 bits: the launcher takes this shape only for matrices
  // and activation planes under 2 GiB (and rows a multiple of 8).
  WideSources ls;
  {
    const uint8_t* e0 = src.weight + static_cast<int64_t>(expert) * a.w_expert_stride;
    ls.wlo = uniform_ptr(e0);
    ls.whi = MODE == GEMM_SWIGLU ? uniform_ptr(src.weight_up + static_cast<int64_t>(expert) * a.w_expert_stride)
                                 : ls.wlo;
    ls.a_hi = uniform_ptr(src.a_hi);
    ls.a_lo = uniform_ptr(src.a_lo);
    ls.wg = src.wg;
    const int64_t rows = a.N;
    const int32_t piece = load_piece_offset(lane, 0);
    const int64_t rlo = MODE == GEMM_PLAIN ? ntile * kWidePlainRows + 64 * wave : ntile * kWideGateRows + 32 * wave;
    const int64_t rhi = MODE == GEMM_PLAIN ? rlo + 32 : rlo;
#pragma unroll
    for (int q = 0; q < kWideTilesPerWave; ++q)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int64_t u = (q < 2 ? rlo : rhi) + 16 * (q & 1) + 8 * h;
        u = u < rows - 8 ? u : rows - 8;
        ls.wrow[2 * q + h] = group_row_base(u, K, ls.wg);
      }
    ls.woff = static_cast<uint32_t>(group_row_base(lane >> 3, K, ls.wg) + piece);
#pragma unroll
    for (int h = 0; h < 2; ++h)
      ls.aoff[h] = static_cast<uint32_t>(token_of(16 * wave + 8 * h + (lane >> 3)) * K + (piece ^ (16 * h)));
  }
  const bool loads_pair = wave < pairs;  // wave-uniform
  const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  // stage 0's direct loads fly while the block scales are gathered
  {
    const uint32_t b_own = static_cast<uint32_t>(wave) * kWideTilesPerWave * kOperand;
#pragma unroll
    for (int q = 0; q < kWideTilesPerWave; ++q)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        lds_direct16_at((q < 2 ? ls.wlo : ls.whi) + ls.wrow[2 * q + h], ls.woff ^ (16 * h),
                        lds_addr + b_own + q * kOperand + 1024 * h);
    if (loads_pair) {
      const uint32_t sa = lds_addr + kWideBBytes + 2 * wave * kOperand;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        lds_direct16_at(ls.a_hi, ls.aoff[h], sa + 1024 * h);
        lds_direct16_at(ls.a_lo, ls.aoff[h], sa + kOperand + 1024 * h);
      }
    }
  }
  load_activation_scales<kGemmWideRows, 512, true>(src, start, len, KB, lds_se);
  // weight scale rows: PLAIN the item's four 128-row blocks; SWIGLU the two
  // blocks its 256 gate rows span, then the same up blocks
  const int64_t srows = (a.N + 127) / 128;
  const int64_t b0 = MODE == GEMM_PLAIN ? 4 * ntile : 2 * ntile;
  for (int64_t i = threadIdx.x; i < 4 * KB; i += 512) {
    const int64_t r = i / KB, k = i - r * KB;
    int64_t blk = b0 + (MODE == GEMM_PLAIN ? r : (r & 1));
    blk = blk < srows ? blk : srows - 1;
    const float* sc = (MODE == GEMM_SWIGLU && r >= 2) ? src.scale_up : src.scale;
    lds_sw[i] = sc[static_cast<int64_t>(expert) * a.s_expert_stride + blk * a.s_cols + k];
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wavefront's stage-0 loads landed
  __syncthreads();

#define GLM53_WIDE(n) \
  wide_gemm_loop<MODE, FIX, n>(a, src, ntile, start, len, KB, ls, loads_pair, lds, lds_addr, lds_se, lds_sw, wave, lane)
  // rows past the descriptor's routes (in its last pair) hold stale
  // activations: their products are never stored
  switch (pairs) {
    case 1: GLM53_WIDE(1); break;
    case 2: GLM53_WIDE(2); break;
    case 3: GLM53_WIDE(3); break;
    case 4: GLM53_WIDE(4); break;
    case 5: GLM53_WIDE(5); break;
    case 6: GLM53_WIDE(6); break;
    case 7: GLM53_WIDE(7); break;
    default: GLM53_WIDE(8); break;
  }
#undef GLM53_WIDE
}

template <int MODE>
__global__ __launch_bounds__(512) void grouped_gemm_wide_kernel(GroupedGemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];
  const int64_t used = used_descriptors(a);
  const int64_t items = a.n_tiles * (used + a.x_descriptors);
  const int64_t per_xcd = (items + 7) / 8;
  if (static_cast<int64_t>(blockIdx.x / 8) >= per_xcd) return;
  const int64_t w = static_cast<int64_t>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (w >= items) return;
  int64_t ntile, d;
  bool fix;
  const ItemSource src = item_source(a, used, w, false, ntile, d, fix);
  if (fix) wide_gemm_body<MODE, true>(a, src, ntile, d, lds_dyn);
  else wide_gemm_body<MODE, false>(a, src, ntile, d, lds_dyn);
}

// Sets *flag (pre-cleared by clear_flag_kernel) when any byte of codes is
// 0x7F or 0xFF.
__global__ void clear_flag_kernel(int32_t* flag) { *flag = 0; }


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
// Stores one thread's V MoE outputs (FP32 values already BF16-exact): the
// plain row, or the kHcBranches hyper-connection streams built from them
// (native_indexer_plan.metal:2362-2388: mixed = fma(comb[s][b], residual[s],
// mixed) over s in order from 0, then T(post[b] * moe + mixed)).
template <int V>
__device__ __forceinline__ void store_moe_row(const ReduceArgs& a, int64_t t, int64_t h0, const float (&moe)[V]) {
  if (a.hc_out == nullptr) {
    store_bf16_run<V>(a.out + t * a.H + h0, moe);
    return;
  }
  Bf16Run<V> res[kHcBranches];
#pragma unroll
  for (int s = 0; s < kHcBranches; ++s) res[s].load(a.hc_residual + (t * kHcBranches + s) * a.H + h0);
#pragma unroll
  for (int b = 0; b < kHcBranches; ++b) {
    const float post = a.hc_post[t * kHcBranches + b];
    float y[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
      float mixed = 0.0f;
#pragma unroll
      for (int s = 0; s < kHcBranches; ++s)
        mixed = __builtin_fmaf(a.hc_comb[(t * kHcBranches + s) * kHcBranches + b], res[s].get(i), mixed);
      y[i] = __fadd_rn(__fmul_rn(post, moe[i]), mixed);
    }
    store_bf16_run<V>(a.hc_out + (t * kHcBranches + b) * a.H + h0, y);
  }
}

// Thread = V consecutive columns of one token (V = 8: 16-byte loads and
// stores, when H and the row pointers allow it; V = 1 otherwise).  The
// token's positions and scores are read first (uniform across the
// workgroup), then every slot's row is requested before the first is summed,
// so the row loads overlap instead of each waiting behind the last.
template <int V, int K>
__global__ __launch_bounds__(256) void restore_reduce_kernel(ReduceArgs a) {
  constexpr int kSlots = K > 0 ? K : kMaxReduceTopK;  // K = 0: top_k known only at run time
  const int k = K > 0 ? K : a.top_k;
  const int64_t t = blockIdx.y;
  const int64_t h0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * V;
  if (h0 >= a.H) return;
  int32_t pos[kSlots];
  float score[kSlots];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) pos[s] = s < k ? a.inverse[t * k + s] : 0;
#pragma unroll
  for (int s = 0; s < kSlots; ++s) score[s] = s < k ? a.sorted_score[pos[s] < 0 ? 0 : pos[s]] : 0.0f;
  Bf16Run<V> row[kSlots];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {  // a missing route (pos < 0) reads row 0 and sums NaN
    row[s].clear();
    if (s < k) row[s].load(a.route_out + static_cast<int64_t>(pos[s] < 0 ? 0 : pos[s]) * a.H + h0);
  }
  float total[V];
#pragma unroll
  for (int i = 0; i < V; ++i) total[i] = 0.0f;
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    if (s >= k) continue;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float v = pos[s] < 0 ? __builtin_nanf("") : row[s].get(i);
      total[i] = __fadd_rn(total[i], __fmul_rn(v, score[s]));
    }
  }
  Bf16Run<V> sh;
  sh.clear();
  if (a.shared != nullptr) sh.load(a.shared + t * a.H + h0);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    total[i] = bf16_round(total[i]);
    if (a.shared != nullptr) total[i] = bf16_round(__fadd_rn(total[i], sh.get(i)));
  }
  store_moe_row<V>(a, t, h0, total);
}

// native_indexer_plan.metal:2174-2207 (fp8.py:384-397 order): per token,
// ascending expert id; contribution = T(down * score); total = T(total + c).
// Thread = V consecutive columns; loads are issued as above, in sorted order.
template <int V>
__global__ __launch_bounds__(256) void direct_order_reduce_kernel(ReduceArgs a) {
  const int64_t t = blockIdx.y;
  const int64_t h0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * V;
  if (h0 >= a.H) return;
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
  int32_t pos[kMaxReduceTopK];
  float score[kMaxReduceTopK];
#pragma unroll
  for (int r = 0; r < kMaxReduceTopK; ++r) pos[r] = a.inverse[t * a.top_k + (r < a.top_k ? order[r] : 0)];
#pragma unroll
  for (int r = 0; r < kMaxReduceTopK; ++r) score[r] = a.route_score[t * a.top_k + (r < a.top_k ? order[r] : 0)];
  Bf16Run<V> row[kMaxReduceTopK];
#pragma unroll
  for (int r = 0; r < kMaxReduceTopK; ++r) {
    row[r].clear();
    if (r < a.top_k) row[r].load(a.route_out + static_cast<int64_t>(pos[r] < 0 ? 0 : pos[r]) * a.H + h0);
  }
  float total[V];
#pragma unroll
  for (int i = 0; i < V; ++i) total[i] = 0.0f;
#pragma unroll
  for (int r = 0; r < kMaxReduceTopK; ++r) {
    if (r >= a.top_k) continue;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float v = pos[r] < 0 ? __builtin_nanf("") : row[r].get(i);
      const float c = bf16_round(__fmul_rn(v, score[r]));
      total[i] = bf16_round(__fadd_rn(total[i], c));
    }
  }
  Bf16Run<V> sh;
  sh.clear();
  if (a.shared != nullptr) sh.load(a.shared + t * a.H + h0);
#pragma unroll
  for (int i = 0; i < V; ++i)
    if (a.shared != nullptr) total[i] = bf16_round(__fadd_rn(total[i], sh.get(i)));
  store_moe_row<V>(a, t, h0, total);
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
  if (a.rows == 0) return hipSuccess;
  if (a.cols % kBlock != 0) return hipErrorInvalidValue;
  const bool wide = a.x_row_stride % 8 == 0 && reinterpret_cast<uintptr_t>(a.x) % 16 == 0;
  const int64_t blocks_per_row = a.cols / kBlock;
  const int64_t units = a.rows * (wide ? (blocks_per_row + 3) / 4 : blocks_per_row);  // wavefronts
  const dim3 grid(static_cast<unsigned>((units + 3) / 4));
  if (wide) hipLaunchKernelGGL(split_activations_kernel<8>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(split_activations_kernel<2>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_grouped_gemm(const GroupedGemmArgs& a, int mode, int64_t descriptors, hipStream_t st) {
  if (descriptors == 0 && a.x_descriptors == 0) return hipSuccess;
  // the epilogues' buffer stores take 32-bit offsets of up to 128 rows
  if (a.out_row_stride < a.N || a.out_row_stride >= (int64_t{1} << 22) ||
      (a.x_descriptors > 0 && (a.x_out_row_stride < a.N || a.x_out_row_stride >= (int64_t{1} << 22))))
    return hipErrorInvalidValue;
  if (a.tile_rows == kGemmWideRows) {
    GroupedGemmArgs g = a;
    g.n_tiles = mode == GEMM_PLAIN ? (a.N + kWidePlainRows - 1) / kWidePlainRows : (a.N + kWideGateRows - 1) / kWideGateRows;
    g.descriptors = descriptors;
    const int64_t items = g.n_tiles * (descriptors + g.x_descriptors);
    const unsigned grid = static_cast<unsigned>(8 * ((items + 7) / 8));
    const size_t lds = gemm_wide_lds_bytes(a.K);
    if (a.K % kBlock != 0 || a.K <= 0 || lds > 160 * 1024) return hipErrorInvalidValue;
    // its direct loads take 32-bit offsets into each matrix and activation plane
    if (!wide_offsets_fit(a.N, a.K, a.routes > a.x_routes ? a.routes : a.x_routes)) return hipErrorInvalidValue;
    if (mode == GEMM_PLAIN) hipLaunchKernelGGL(grouped_gemm_wide_kernel<GEMM_PLAIN>, dim3(grid), dim3(512), lds, st, g);
    else hipLaunchKernelGGL(grouped_gemm_wide_kernel<GEMM_SWIGLU>, dim3(grid), dim3(512), lds, st, g);
    return hipGetLastError();
  }
  GroupedGemmArgs g = a;
  g.n_tiles = mode == GEMM_PLAIN ? (a.N + 127) / 128 : (a.N + 63) / 64;
  g.descriptors = descriptors;
  const int64_t items = g.n_tiles * (descriptors + g.x_descriptors);
  const unsigned grid = static_cast<unsigned>(8 * ((items + 7) / 8));
  if (a.tile_rows != 0 && a.tile_rows != kGemmMinTileRows && a.tile_rows != kGemmTileRows)
    return hipErrorInvalidValue;
  const bool narrow = a.tile_rows == kGemmMinTileRows;
  const size_t lds = narrow ? gemm_lds_bytes<1>(a.K) : gemm_lds_bytes<2>(a.K);
  if (a.K % kBlock != 0 || a.K <= 0 || lds > 160 * 1024) return hipErrorInvalidValue;
#define GLM53_GEMM(m, w) hipLaunchKernelGGL((grouped_gemm_kernel<m, w>), dim3(grid), dim3(256), lds, st, g)
  if (mode == GEMM_PLAIN) {
    if (narrow) GLM53_GEMM(GEMM_PLAIN, 1);
    else GLM53_GEMM(GEMM_PLAIN, 2);
  } else {
    if (narrow) GLM53_GEMM(GEMM_SWIGLU, 1);
    else GLM53_GEMM(GEMM_SWIGLU, 2);
  }
#undef GLM53_GEMM
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

hipError_t launch_reduce(const ReduceArgs& a, bool direct_order, hipStream_t st) {
  if (a.tokens == 0) return hipSuccess;
  if (a.top_k > kMaxReduceTopK) return hipErrorInvalidValue;
  auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool wide = a.H % 8 == 0 && a16(a.route_out) && a16(a.out) && a16(a.shared) && a16(a.hc_residual) &&
                    a16(a.hc_out);
  const int64_t per_thread = wide ? 8 : 1;
  const dim3 grid(static_cast<unsigned>((a.H / per_thread + 255) / 256), static_cast<unsigned>(a.tokens));
  if (wide) {
    if (direct_order) hipLaunchKernelGGL(direct_order_reduce_kernel<8>, grid, dim3(256), 0, st, a);
    else if (a.top_k == 8) hipLaunchKernelGGL((restore_reduce_kernel<8, 8>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((restore_reduce_kernel<8, 0>), grid, dim3(256), 0, st, a);
  } else {
    if (direct_order) hipLaunchKernelGGL(direct_order_reduce_kernel<1>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((restore_reduce_kernel<1, 0>), grid, dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace glm53
