// Device helpers shared by every kernel of the FP8 block-scaled MoE path.
// gfx950 (CDNA4) only: 64-lane wavefronts, DPP cross-lane moves, f16 dot2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace glm53 {

constexpr int kBlock = 128;   // FP8 scale block edge (weight_scale_inv is per 128x128)
constexpr int kWave = 64;

// ------------------------------------------------------- weight layouts ---
//
// An E4M3 matrix [N, K] is stored either row-major (g = 0: the checkpoint
// layout, element (n, k) at n K + k) or in row groups (g = 1 .. 7, K a
// multiple of 128): the 2^g rows of group n >> g are stored together, their
// K span as K / 128 consecutive blocks of 2^g rows x 128 bytes, so that
//   (n, k) -> (n >> g) 2^g K + (k >> 7) 2^g 128 + (n mod 2^g) 128 + k mod 128.
// A 128-row MFMA weight stage then reads 128 / 2^g contiguous runs of
// 2^g x 128 bytes instead of 128 runs of 128 bytes, and a group's whole K
// span (2^g K bytes) is one contiguous run for the decode GEMV.  g = 0 is
// the same formula, so every kernel takes g as an argument.
constexpr int kMaxRowGroupLog2 = 7;

__host__ __device__ __forceinline__ int64_t group_row_base(int64_t n, int64_t K, int g) {
  return ((n >> g) << g) * K + ((n & ((int64_t{1} << g) - 1)) << 7);
}
__host__ __device__ __forceinline__ int64_t group_col(int64_t k, int g) {
  return ((k >> 7) << (7 + g)) | (k & 127);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------ BF16 ---

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even FP32 -> BF16 (the Metal/MLX bfloat conversion); a
// NaN keeps its upper bits and is made quiet.  gfx950's v_cvt_pk_bf16_f32
// (what the __bf16 conversion compiles to) gives exactly these bits: checked
// on the GPU against the integer form -- (u + 0x7fff + ((u >> 16) & 1)) >> 16,
// NaN -> (u >> 16) | 0x40 -- for all 2^32 FP32 patterns.  One instruction
// instead of a rounding sequence with a NaN select at every BF16 step.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ------------------------------------------------------------------ E4M3 ---
//
// Exact E4M3 -> FP16 decode of two bytes packed into one dword.  With the
// E4M3 exponent field e (bias 7) and mantissa m moved into FP16's exponent
// (bias 15) and mantissa fields, the FP16 value is exactly 2^-8 times the
// E4M3 value for every code, subnormals included (e=0 lands on FP16
// subnormals m*2^-17), and the 0x7F/0xFF codes decode to +-480/256 exactly as
// the reference's LUT does (no NaN code).  The 2^8 is folded into the block
// scale.  Three or four VALU ops per pair, no table.
//
// v = [b3 b2 b1 b0]:   odd pair -> (b1, b3)   even pair -> (b0, b2)
__device__ __forceinline__ uint32_t e4m3x2_odd_to_f16x2(uint32_t v) {
  return ((v >> 1) & 0x3F803F80u) | (v & 0x80008000u);
}
__device__ __forceinline__ uint32_t e4m3x2_even_to_f16x2(uint32_t v) {
  return ((v << 7) & 0x3F803F80u) | ((v << 8) & 0x80008000u);
}

__device__ __forceinline__ float dot2(uint32_t w_f16x2, uint32_t x_f16x2, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w_f16x2),
                                __builtin_bit_cast(half2_t, x_f16x2), acc, false);
}

// Partial dot product of 4 weight bytes with 4 activations held as the FP16
// pairs (x0, x2) and (x1, x3) (the same byte pairing as the decode above).
__device__ __forceinline__ float dot4_e4m3(uint32_t w4, uint32_t x02, uint32_t x13, float acc) {
  acc = dot2(e4m3x2_even_to_f16x2(w4), x02, acc);
  return dot2(e4m3x2_odd_to_f16x2(w4), x13, acc);
}

// Pack activations (already scaled into FP16 range) as (xa, xb) FP16 pair.
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  half2_t h = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(uint32_t, h);
}

// Power-of-two exponent that maps |x| <= amax into [2^14, 2^15): activations
// divided by 2^shift are exact in FP16 (BF16 has 8 significant bits, FP16 11)
// unless they sit more than 2^28 below the lane's maximum.
__device__ __forceinline__ int f16_shift_for(float amax) {
  if (!(amax > 0.0f) || !isfinite(amax)) return 0;
  int e = ilogbf(amax);
  return e - 14;
}

// ---------------------------------------------------------- reductions ---

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over all 64 lanes; every lane gets the total.  DPP within 16-lane
// rows, then the four row totals through readlane.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// ------------------------------------------------------------- SwiGLU ---
//
// MLX BF16 sigmoid as the reference evaluates it (every step rounded to
// BF16): tail = 1 / (1 + exp(|g|)); sigma = g < 0 ? tail : 1 - tail.  MLX's
// Metal fast::exp and the correctly rounded exponential agree, after BF16
// rounding, on every finite BF16 g in [-10, 10] except g = -6.84375
// (0xC0DB): exp(6.84375) = 938.0000478 lies 5e-5 above the BF16 midpoint
// 938, and fast::exp rounds to 936, giving sigma = 0x3A8C.  That point is
// reproduced explicitly; expf is accurate to well inside 5e-5 there.
__device__ __forceinline__ float sigmoid_mlx_bf16(uint16_t gbits) {
  if (gbits == 0xC0DBu) return bf16_to_f32(0x3A8Cu);
  float g = bf16_to_f32(gbits);
  float e = bf16_round(expf(fabsf(g)));
  float d = bf16_round(1.0f + e);
  float tail = bf16_round(1.0f / d);
  return g < 0.0f ? tail : bf16_round(1.0f - tail);
}

// The same function from the hardware exponential (v_exp_f32 through
// __expf) and reciprocal (v_rcp_f32): over all 65536 BF16 inputs its BF16
// steps round to the same bits as sigmoid_mlx_bf16's except where |g| > 87
// (exp(|g|) near FP32 overflow, 1/d near the subnormal range) and at the
// fast::exp point above; those inputs take sigmoid_mlx_bf16 itself.  The
// equality over all patterns is a GPU test (through glm53_sigmoid_bf16).
__device__ __forceinline__ float sigmoid_mlx_bf16_fast(uint16_t gbits) {
  const float g = bf16_to_f32(gbits);
  const float a = fabsf(g);
  const float e = bf16_round(__expf(a));
  const float d = bf16_round(1.0f + e);
  const float tail = bf16_round(__builtin_amdgcn_rcpf(d));
  const float upper = bf16_round(1.0f - tail);
  if (!(a <= 87.0f) || gbits == 0xC0DBu) return sigmoid_mlx_bf16(gbits);
  return g < 0.0f ? tail : upper;
}

// Clamped SwiGLU with the reference's exact rounding points:
// g' = T(min(T(g), L)); u' = T(clip(T(u), -L, L)); h = T(T(g' * s(g')) * u').
// Inputs are the FP32 accumulator values before the projection's BF16 store.
// swiglu_mlx_prepare gives g' (BF16 bits) and u'; swiglu_mlx_finish the
// output from them and s(g').
__device__ __forceinline__ void swiglu_mlx_prepare(float gate_acc, float up_acc, float limit, uint16_t& ga, float& ua) {
  float g = bf16_round(gate_acc);
  float u = bf16_round(up_acc);
  float gv = (g < limit) ? g : limit;
  if (isnan(g)) gv = g;
  float uv = fminf(fmaxf(u, -limit), limit);
  if (isnan(u)) uv = u;
  ga = f32_to_bf16(gv);
  ua = bf16_round(uv);
}

__device__ __forceinline__ uint16_t swiglu_mlx_finish(uint16_t ga, float ua, float sigma) {
  float silu = bf16_round(bf16_to_f32(ga) * sigma);
  return f32_to_bf16(silu * ua);
}

__device__ __forceinline__ uint16_t swiglu_mlx(float gate_acc, float up_acc, float limit) {
  uint16_t ga;
  float ua;
  swiglu_mlx_prepare(gate_acc, up_acc, limit, ga, ua);
  return swiglu_mlx_finish(ga, ua, sigmoid_mlx_bf16_fast(ga));
}

// swiglu_mlx as straight-line arithmetic on two values at once, for
// epilogues that hold many values per lane.  Every BF16 rounding converts
// both values with one v_cvt_pk_bf16_f32; the result holds value 0's bits
// in its low half and value 1's in its high half.  Same bits as swiglu_mlx
// for every input with 0 < L, |T(g)| <= 87, T(u) not NaN and T(g) != 0xC0DB:
// `check` keeps the largest BF16 magnitudes of T(g) and T(u) and the smallest
// XOR of T(g) with 0xC0DB, and when swiglu_straight_ok(check, L) is false the
// caller recomputes its values with swiglu_mlx.  For such inputs the clamps
// are v_min / v_med3 (no NaN operand; with 0 < L, +-0 stays itself), and the
// sign select is a bit select (g' = -0 gives tail = upper = 0.5).
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// Written as assembly: built as a two-element vector conversion, a pair of
// accumulator elements became one 8-byte load that kept the accumulators in
// scratch memory.  The compiler does not insert the wait state a VALU
// instruction needs before it reads the result of a transcendental one
// (v_exp_f32, v_rcp_f32) when the reader is inline assembly: the form for
// such operands carries it.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_after_trans(float a, float b) {
  uint32_t r;
  asm("s_nop 0\n\tv_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float bf16x2_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16x2_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

struct SwigluCheck {
  uint32_t mag = 0;           // max |T(g)| bits (low half), max |T(u)| bits (high half)
  uint32_t key = 0xFFFFFFFFu;  // min T(g) ^ 0xC0DB (low half)
};
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, a), __builtin_bit_cast(u16x2_t, b)));
}
__device__ __forceinline__ uint32_t min_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2_t, a), __builtin_bit_cast(u16x2_t, b)));
}

// Written as assembly: on operands it cannot prove canonical the compiler
// adds a canonicalising v_max before every min/max/med3, which these
// operands (non-NaN whenever the result is used) do not need.
__device__ __forceinline__ float min_f32(float a, float b) {
  float r;
  asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float med3_f32(float a, float b, float c) {
  float r;
  asm("v_med3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// bits of t where the sign bit of x is set, of u elsewhere
__device__ __forceinline__ float sign_select(float x, float t, float u) {
  const uint32_t neg = static_cast<uint32_t>(static_cast<int32_t>(__float_as_uint(x)) >> 31);
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(neg), "v"(__float_as_uint(t)), "v"(__float_as_uint(u)));
  return __uint_as_float(r);
}

__device__ __forceinline__ uint32_t swiglu_mlx_straight2(float gate0, float up0, float gate1, float up1, float limit,
                                                         SwigluCheck& check) {
  const uint32_t gu0 = f32x2_to_bf16x2(gate0, up0), gu1 = f32x2_to_bf16x2(gate1, up1);
  check.mag = max_u16x2(check.mag, max_u16x2(gu0 & 0x7FFF7FFFu, gu1 & 0x7FFF7FFFu));
  check.key = min_u16x2(check.key, min_u16x2(gu0 ^ 0xC0DBu, gu1 ^ 0xC0DBu));
  // g' = T(min(T(g), L)) and u' = T(clip(T(u), -L, L)) of each value
  const uint32_t p0 = f32x2_to_bf16x2(min_f32(bf16x2_lo(gu0), limit), med3_f32(bf16x2_hi(gu0), -limit, limit));
  const uint32_t p1 = f32x2_to_bf16x2(min_f32(bf16x2_lo(gu1), limit), med3_f32(bf16x2_hi(gu1), -limit, limit));
  const float g0 = bf16x2_lo(p0), u0 = bf16x2_hi(p0), g1 = bf16x2_lo(p1), u1 = bf16x2_hi(p1);
  const uint32_t e = f32x2_to_bf16x2_after_trans(__expf(fabsf(g0)), __expf(fabsf(g1)));
  const uint32_t d = f32x2_to_bf16x2(1.0f + bf16x2_lo(e), 1.0f + bf16x2_hi(e));
  const uint32_t tail =
      f32x2_to_bf16x2_after_trans(__builtin_amdgcn_rcpf(bf16x2_lo(d)), __builtin_amdgcn_rcpf(bf16x2_hi(d)));
  const float t0 = bf16x2_lo(tail), t1 = bf16x2_hi(tail);
  const uint32_t upper = f32x2_to_bf16x2(1.0f - t0, 1.0f - t1);
  const float s0 = sign_select(g0, t0, bf16x2_lo(upper)), s1 = sign_select(g1, t1, bf16x2_hi(upper));
  const uint32_t silu = f32x2_to_bf16x2(g0 * s0, g1 * s1);
  return f32x2_to_bf16x2(bf16x2_lo(silu) * u0, bf16x2_hi(silu) * u1);
}
__device__ __forceinline__ bool swiglu_straight_ok(const SwigluCheck& c, float limit) {
  // |T(g)| <= 87 (0x42AE), T(u) not NaN (<= 0x7F80), no 0xC0DB, 0 < L
  return (c.mag & 0xFFFFu) <= 0x42AEu && (c.mag >> 16) <= 0x7F80u && (c.key & 0xFFFFu) != 0 && limit > 0.0f;
}

}  // namespace glm53
