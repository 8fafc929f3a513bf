// FP32 router logits for many tokens (patch.py:131-134 of the reference:
// logits = x.astype(float32) @ W.T, W FP32 [experts, hidden]) on BF16 MFMA.
//
// Every FP32 weight w is split exactly into three BF16 parts by truncation:
// hi = w with its low 16 bits cleared, mid = (w - hi) truncated the same
// way, lo = w - hi - mid (at most 8 significant bits, so exact in BF16);
// w = hi + mid + lo.  A BF16 activation times a BF16 part is exact in FP32,
// so three v_mfma_f32_16x16x32_bf16 per operand pair accumulate x . w in
// FP32 like an FP32 GEMM; only the order of the FP32 additions differs.
// router_planes_kernel writes the three parts once per call as BF16 planes
// [3][experts][hidden]; the GEMM then only loads and multiplies.
//
// GEMM work item = 64 tokens (four 16-row MFMA tiles) x 4 NT expert tiles of
// 16 x one K chunk; wavefront w owns expert tiles w, w + 4, ... of the item.
// Each lane reads its operands straight from global memory as 16-byte BF16
// runs (row lane % 16, K run 8 (lane / 16) of each 32-deep step; any K
// order works as long as both operands use the same one), double-buffered
// one step ahead.  K chunks ("splits") write FP32 partial sums [split]
// [token][expert]; topk_kernel adds them in split order.  Items run
// split-major in contiguous runs per XCD, so the items of one split share
// that chunk's weight planes in one L2.

#include "common.h"
#include "kernels.h"

namespace glm53 {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kRouterTileTokens = 64;
constexpr int kRouterTilesPerWave = 2;  // NT: 8 expert tiles (128 experts) per work item

// Thread = 8 consecutive weights: two 16-byte FP32 loads, three 16-byte BF16 stores.
__global__ __launch_bounds__(256) void router_planes_kernel(const float* w, uint16_t* planes, int64_t n) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (i >= n) return;
  const float4 a = *reinterpret_cast<const float4*>(w + i);
  const float4 b = *reinterpret_cast<const float4*>(w + i + 4);
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[4], m[4], l[4];
#pragma unroll
  for (int k = 0; k < 8; k += 2) {
    uint32_t hb[2], mb[2], lb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t b0 = __float_as_uint(v[k + j]) & 0xffff0000u;
      const float r1 = v[k + j] - __uint_as_float(b0);
      const uint32_t b1 = __float_as_uint(r1) & 0xffff0000u;
      const float r2 = r1 - __uint_as_float(b1);
      hb[j] = b0;
      mb[j] = b1;
      lb[j] = __float_as_uint(r2) & 0xffff0000u;  // r2 already fits in BF16
    }
    h[k >> 1] = (hb[0] >> 16) | hb[1];
    m[k >> 1] = (mb[0] >> 16) | mb[1];
    l[k >> 1] = (lb[0] >> 16) | lb[1];
  }
  *reinterpret_cast<uint4*>(planes + i) = make_uint4(h[0], h[1], h[2], h[3]);
  *reinterpret_cast<uint4*>(planes + n + i) = make_uint4(m[0], m[1], m[2], m[3]);
  *reinterpret_cast<uint4*>(planes + 2 * n + i) = make_uint4(l[0], l[1], l[2], l[3]);
}

template <int NT>
struct Fragments {
  uint4 x[4];      // 4 token tiles
  uint4 w[NT][3];  // NT expert tiles x (hi, mid, lo)
};

template <int NT>
__device__ __forceinline__ void load_fragments(Fragments<NT>& f, const uint16_t* const (&xrow)[4],
                                               const uint16_t* const (&wrow)[NT], int64_t plane, int64_t k) {
#pragma unroll
  for (int m = 0; m < 4; ++m) f.x[m] = *reinterpret_cast<const uint4*>(xrow[m] + k);
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int p = 0; p < 3; ++p) f.w[j][p] = *reinterpret_cast<const uint4*>(wrow[j] + p * plane + k);
}

template <int NT>
__device__ __forceinline__ void multiply(f32x4_t (&acc)[4][NT], const Fragments<NT>& f, const bool (&live)[NT]) {
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    if (!live[j]) continue;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bf16x8_t xa = __builtin_bit_cast(bf16x8_t, f.x[m]);
#pragma unroll
      for (int p = 0; p < 3; ++p)
        acc[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(bf16x8_t, f.w[j][p]), acc[m][j],
                                                            0, 0, 0);
    }
  }
}

template <int NT>
__global__ __launch_bounds__(256) void router_gemm_kernel(RouterGemmArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: tile tests branch on scalars
  const int64_t groups = a.token_groups * a.expert_groups;
  const int64_t items = groups * a.splits;
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t item = static_cast<int64_t>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (item >= items) return;
  const int64_t split = item / groups;
  const int64_t t0 = (item % groups / a.expert_groups) * kRouterTileTokens;
  const int64_t tile0 = (item % a.expert_groups) * 4 * NT;
  const int64_t k_begin = split * a.k_chunk;
  const int64_t k_end = k_begin + a.k_chunk < a.hidden ? k_begin + a.k_chunk : a.hidden;
  const int64_t tiles = (a.experts + 15) / 16;
  const int64_t plane = a.experts * a.hidden;
  const int r = lane & 15;
  const int q = lane >> 4;
  // Rows past the last token or expert read the last one; their sums are dropped.
  const uint16_t* xrow[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int64_t t = t0 + 16 * m + r;
    xrow[m] = a.x + (t < a.tokens ? t : a.tokens - 1) * a.hidden + 8 * q;
  }
  const uint16_t* wrow[NT];
  bool live[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int64_t tile = tile0 + wave + 4 * j;
    const int64_t e = 16 * tile + r;
    live[j] = tile < tiles;
    wrow[j] = a.planes + (e < a.experts ? e : a.experts - 1) * a.hidden + 8 * q;
  }
  f32x4_t acc[4][NT];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[m][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // The chunk holds an even number of 32-deep steps (K chunks are multiples
  // of 128).  Loads are never conditional (the last prefetch re-reads the
  // first step and is not used), so the compiler's counted waits keep the
  // next step's loads in flight across each step's MFMAs.
  Fragments<NT> f0, f1;
  load_fragments(f0, xrow, wrow, plane, k_begin);
  for (int64_t k = k_begin; k < k_end; k += 64) {
    load_fragments(f1, xrow, wrow, plane, k + 32);
    multiply(acc, f0, live);
    load_fragments(f0, xrow, wrow, plane, k + 64 < k_end ? k + 64 : k_begin);
    multiply(acc, f1, live);
  }
  // D layout of the 16x16 MFMA: lane holds rows 4 (lane / 16) + i, column lane % 16.
  float* out = a.partial + split * a.tokens * a.experts;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int64_t e = 16 * (tile0 + wave + 4 * j) + r;
    if (!live[j] || e >= a.experts) continue;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t t = t0 + 16 * m + 4 * q + i;
        if (t < a.tokens) out[t * a.experts + e] = acc[m][j][i];
      }
  }
}

}  // namespace

bool router_gemm_supported(int64_t hidden, int64_t experts, const void* x, const void* weight) {
  return hidden > 0 && hidden % 128 == 0 && experts > 0 && experts <= kMaxRouterExperts &&
         reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0;
}

RouterGemmShape router_gemm_shape(int64_t tokens, int64_t hidden, int64_t experts) {
  RouterGemmShape s{};
  s.token_groups = (tokens + kRouterTileTokens - 1) / kRouterTileTokens;
  const int64_t tiles = (experts + 15) / 16;
  s.expert_groups = (tiles + 4 * kRouterTilesPerWave - 1) / (4 * kRouterTilesPerWave);
  const int64_t groups = s.token_groups * s.expert_groups;
  const int64_t blocks = hidden / 128;
  // Two work items per CU where K allows, at most kMaxRouterSplits partial planes.
  int64_t want = (512 + groups - 1) / groups;
  if (want > kMaxRouterSplits) want = kMaxRouterSplits;
  if (want > blocks) want = blocks;
  if (want < 1) want = 1;
  const int64_t chunk_blocks = (blocks + want - 1) / want;
  s.k_chunk = chunk_blocks * 128;
  s.splits = (blocks + chunk_blocks - 1) / chunk_blocks;
  return s;
}

size_t router_planes_bytes(int64_t hidden, int64_t experts) {
  return static_cast<size_t>(3 * 2) * static_cast<size_t>(hidden * experts);
}

hipError_t launch_router_logits(const RouterGemmArgs& a, const float* weight, hipStream_t st) {
  if (a.tokens == 0) return hipSuccess;
  if (!router_gemm_supported(a.hidden, a.experts, a.x, weight) || a.k_chunk % 128 != 0 || a.splits < 1 ||
      a.splits > kMaxRouterSplits || reinterpret_cast<uintptr_t>(a.planes) % 16 != 0)
    return hipErrorInvalidValue;
  const int64_t n = a.experts * a.hidden;
  hipLaunchKernelGGL(router_planes_kernel, dim3(static_cast<unsigned>((n / 8 + 255) / 256)), dim3(256), 0, st, weight,
                     a.planes, n);
  // item(b) = (b % 8) * ceil(items / 8) + b / 8 covers every item only over 8 * ceil(items / 8) workgroups
  const int64_t items = a.token_groups * a.expert_groups * a.splits;
  hipLaunchKernelGGL(router_gemm_kernel<kRouterTilesPerWave>, dim3(static_cast<unsigned>((items + 7) / 8 * 8)),
                     dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace glm53
