// FP32 router logits for many tokens (patch.py:131-134 of the reference:
// logits = x.astype(float32) @ W.T, W FP32 [experts, hidden]) on BF16 MFMA.
//
// Every FP32 weight w is split exactly into three BF16 parts by truncation:
// hi = w with its low 16 bits cleared, mid = (w - hi) truncated the same
// way, lo = w - hi - mid (at most 8 significant bits, so exact in BF16);
// w = hi + mid + lo.  A BF16 activation times a BF16 part is exact in FP32,
// so three v_mfma_f32_16x16x32_bf16 per operand pair accumulate x . w in
// FP32 like an FP32 GEMM; only the order of the FP32 additions differs.
//
// Work item = 128 tokens x 96 experts x one K chunk, 4 wavefronts in a 2 x 2
// grid (64 tokens x 48 experts each: 4 x 3 MFMA tiles).  Per 32-deep K step
// the workgroup loads the tokens' BF16 rows (8 KB) and the experts' FP32 rows
// (12 KB) once from global memory into registers, kAhead steps ahead, splits
// the weights into their three BF16 parts on the way into LDS (18 KB), and
// every wavefront reads its MFMA operands from LDS: each operand byte leaves
// L2 once per workgroup (the register-operand form read the token rows once
// per wavefront).  K chunks ("splits") write FP32 partial sums
// [split][token][expert]; topk_kernel adds them in split order.  Items run
// split-major in contiguous runs per XCD, so the items of one split share
// that chunk's weight rows in one L2.

#include "common.h"
#include "kernels.h"

namespace glm53 {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTileTokens = 128;
constexpr int kTileExperts = 96;
constexpr int kStep = 32;                       // K per step: one v_mfma_f32_16x16x32_bf16
constexpr int kRowBytes = kStep * 2;            // 64 B: one BF16 row of a step in LDS
constexpr int kXBytes = kTileTokens * kRowBytes;   // 8 KB
constexpr int kPlaneBytes = kTileExperts * kRowBytes;  // 6 KB per BF16 part
constexpr int kStageBytes = kXBytes + 3 * kPlaneBytes;  // 26 KB
#ifndef GLM53_ROUTER_AHEAD
#define GLM53_ROUTER_AHEAD 3
#endif
constexpr int kAhead = GLM53_ROUTER_AHEAD;       // steps of global loads in flight

// Octet q (8 BF16 = 16 B) of LDS row r sits at slot q ^ ((r >> 2) & 3): the
// 16 lanes reading octet q of rows r .. r + 15 then spread over all banks.
__device__ __forceinline__ int slot_offset(int r, int q) { return r * kRowBytes + 16 * (q ^ ((r >> 2) & 3)); }

// The three BF16 parts of four FP32 weights, packed two per word.
__device__ __forceinline__ void split3(const f32x4_t& v, uint2& hi, uint2& mid, uint2& lo) {
  const float in[4] = {v[0], v[1], v[2], v[3]};
  uint32_t h[4], m[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t b0 = __float_as_uint(in[j]) & 0xffff0000u;
    const float r1 = in[j] - __uint_as_float(b0);
    const uint32_t b1 = __float_as_uint(r1) & 0xffff0000u;
    const float r2 = r1 - __uint_as_float(b1);
    h[j] = b0;
    m[j] = b1;
    l[j] = __float_as_uint(r2) & 0xffff0000u;  // r2 already fits in BF16
  }
  hi = make_uint2((h[0] >> 16) | h[1], (h[2] >> 16) | h[3]);
  mid = make_uint2((m[0] >> 16) | m[1], (m[2] >> 16) | m[3]);
  lo = make_uint2((l[0] >> 16) | l[1], (l[2] >> 16) | l[3]);
}

// One step's global operands held by a thread: token rows (two 16-byte BF16
// octets) and expert rows (three 16-byte FP32 quads).
// ext_vector_type members: with HIP's uint4 / float4 the register copies
// became memcpy's that kept the prefetched activations in scratch memory,
// each written there right after its load was issued (that is, after
// waiting for it), and the many-token router ran ~10% longer.
struct StepRegs {
  u32x4_t x[2];
  f32x4_t w[3];
};

__global__ __launch_bounds__(256, 2) void router_tile_kernel(RouterGemmArgs a, const float* __restrict__ weight) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // 2 stages
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t groups = a.token_groups * a.expert_groups;
  const int64_t items = groups * a.splits;
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t item = static_cast<int64_t>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (item >= items) return;
  const int64_t split = item / groups;
  const int64_t t0 = (item % groups / a.expert_groups) * kTileTokens;
  const int64_t e0 = (item % a.expert_groups) * kTileExperts;
  const int64_t k_begin = split * a.k_chunk;
  const int64_t k_end = k_begin + a.k_chunk < a.hidden ? k_begin + a.k_chunk : a.hidden;
  const int64_t H = a.hidden;

  // ---- global load assignment (rows past the last token / expert re-read
  // the last one; their sums are never stored)
  // tokens: thread t loads octets 2 (t % 2) and 2 (t % 2) + 1 of row t / 2
  const int xr = t >> 1, xq = 2 * (t & 1);
  const uint16_t* xsrc = a.x + (t0 + xr < a.tokens ? t0 + xr : a.tokens - 1) * H + 8 * xq;
  // experts: 96 rows x 8 quads of 4 FP32 = 768 quads, quad i = t + 256 j -> row i / 8, quad i % 8
  const float* wsrc[3];
  int wr[3], wq[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int i = t + 256 * j;
    wr[j] = i >> 3;
    wq[j] = i & 7;
    const int64_t e = e0 + wr[j];
    wsrc[j] = weight + (e < a.experts ? e : a.experts - 1) * H + 4 * wq[j];
  }
  auto load = [&](StepRegs& r, int64_t k) {
    r.x[0] = *reinterpret_cast<const u32x4_t*>(xsrc + k);
    r.x[1] = *reinterpret_cast<const u32x4_t*>(xsrc + k + 8);
#pragma unroll
    for (int j = 0; j < 3; ++j) r.w[j] = *reinterpret_cast<const f32x4_t*>(wsrc[j] + k);
  };
  auto store = [&](const StepRegs& r, uint8_t* stage) {
    *reinterpret_cast<u32x4_t*>(stage + slot_offset(xr, xq)) = r.x[0];
    *reinterpret_cast<u32x4_t*>(stage + slot_offset(xr, xq + 1)) = r.x[1];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      uint2 hi, mid, lo;
      split3(r.w[j], hi, mid, lo);
      // quad wq holds K 4 wq .. 4 wq + 3: half (wq & 1) of octet wq / 2
      const int off = slot_offset(wr[j], wq[j] >> 1) + 8 * (wq[j] & 1);
      uint8_t* planes = stage + kXBytes;
      *reinterpret_cast<uint2*>(planes + off) = hi;
      *reinterpret_cast<uint2*>(planes + kPlaneBytes + off) = mid;
      *reinterpret_cast<uint2*>(planes + 2 * kPlaneBytes + off) = lo;
    }
  };

  // ---- MFMA operand reads: lane reads row 16 tile + lane % 16, octet lane / 16
  const int wm = wave >> 1, wn = wave & 1;  // 64-token half, 48-expert half
  const int r16 = lane & 15, q = lane >> 4;
  f32x4_t acc[4][3];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < 3; ++n) acc[m][n] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // kAhead register sets: step k's global loads are issued kAhead steps
  // before its operands go into LDS, so several steps' loads are in flight
  // behind each step's MFMAs (one step of 32 is too short to cover them).
  StepRegs regs[kAhead];
#pragma unroll
  for (int d = 0; d < kAhead; ++d)
    if (k_begin + d * kStep < k_end) load(regs[d], k_begin + d * kStep);
  int s = 0;
  for (int64_t k0 = k_begin; k0 < k_end; k0 += kAhead * kStep) {
#pragma unroll
    for (int d = 0; d < kAhead; ++d) {
      const int64_t k = k0 + d * kStep;
      if (k >= k_end) break;
      uint8_t* stage = lds + s * kStageBytes;
      store(regs[d], stage);
      __syncthreads();  // the stage is complete; the other stage's readers are done
      if (k + kAhead * kStep < k_end) load(regs[d], k + kAhead * kStep);
      bf16x8_t xa[4];
#pragma unroll
      for (int m = 0; m < 4; ++m)
        xa[m] = __builtin_bit_cast(bf16x8_t,
                                   *reinterpret_cast<const uint4*>(stage + slot_offset(64 * wm + 16 * m + r16, q)));
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        const int row = 48 * wn + 16 * n + r16;
        bf16x8_t wb[3];
#pragma unroll
        for (int p = 0; p < 3; ++p)
          wb[p] = __builtin_bit_cast(
              bf16x8_t, *reinterpret_cast<const uint4*>(stage + kXBytes + p * kPlaneBytes + slot_offset(row, q)));
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int p = 0; p < 3; ++p)
            acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[m], wb[p], acc[m][n], 0, 0, 0);
      }
      s ^= 1;
    }
  }
  // D layout of the 16x16 MFMA: lane holds rows 4 (lane / 16) + i, column lane % 16.
  float* out = a.partial + split * a.tokens * a.experts;
#pragma unroll
  for (int n = 0; n < 3; ++n) {
    const int64_t e = e0 + 48 * wn + 16 * n + r16;
    if (e >= a.experts) continue;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t tok = t0 + 64 * wm + 16 * m + 4 * q + i;
        if (tok < a.tokens) out[tok * a.experts + e] = acc[m][n][i];
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
  s.token_groups = (tokens + kTileTokens - 1) / kTileTokens;
  s.expert_groups = (experts + kTileExperts - 1) / kTileExperts;
  const int64_t groups = s.token_groups * s.expert_groups;
  const int64_t blocks = hidden / 128;
  // At most 512 work items (two per CU, one round) where K allows: a 513th
  // item would cost a whole second round (e.g. 2,048 tokens x 288 experts,
  // 48 groups over K = 4,096: 11 planes were 528 items, 8 planes are 384),
  // and at most kMaxRouterSplits partial planes.
  int64_t want = 512 / groups;
  if (want > kMaxRouterSplits) want = kMaxRouterSplits;
  if (want > blocks) want = blocks;
  if (want < 1) want = 1;
  const int64_t chunk_blocks = (blocks + want - 1) / want;
  s.k_chunk = chunk_blocks * 128;
  s.splits = (blocks + chunk_blocks - 1) / chunk_blocks;
  return s;
}

hipError_t launch_router_logits(const RouterGemmArgs& a, const float* weight, hipStream_t st) {
  if (a.tokens == 0) return hipSuccess;
  if (!router_gemm_supported(a.hidden, a.experts, a.x, weight) || a.k_chunk % 128 != 0 || a.splits < 1 ||
      a.splits > kMaxRouterSplits)
    return hipErrorInvalidValue;
  // item(b) = (b % 8) * ceil(items / 8) + b / 8 covers every item only over 8 * ceil(items / 8) workgroups
  const int64_t items = a.token_groups * a.expert_groups * a.splits;
  hipLaunchKernelGGL(router_tile_kernel, dim3(static_cast<unsigned>((items + 7) / 8 * 8)), dim3(256),
                     2 * kStageBytes, st, a, weight);
  return hipGetLastError();
}

}  // namespace glm53
