/*
 * glm53_oracle.c -- CPU restatement of the reference's Direct FP8 MoE
 * arithmetic.  TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load this library as the checker or as the CPU
 * comparator.  The product path (glm53-flash-mlx_amd/) never links or calls
 * it.
 *
 * Every function states the reference file:line whose semantics it restates
 * (paths relative to the kiojuvr/glm53-flash-mlx repository root).
 *
 * Numerical convention.  The reference accumulates FP32 products on Metal in
 * an order fixed by simd_sum, which cannot be reproduced here.  This oracle
 * instead evaluates each dot product in double precision (every product
 * x*lut*scale is exact in double, so the sum is the real-number value to
 * ~1e-16 relative) and rounds to FP32 and then BF16 exactly where the
 * reference rounds.  The result is the correctly rounded value of the
 * reference's formula; a Metal or HIP FP32 accumulation lands on the same BF16
 * value except for rare one-ulp rounding-boundary cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define GLM53O_BLOCK 128

/* ---------------------------------------------------------------- BF16 --- */

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even FP32 -> BF16 (MLX / Metal bfloat conversion). */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

uint16_t glm53o_f32_to_bf16(float f) { return f32_to_bf16(f); }
float glm53o_bf16_to_f32(uint16_t b) { return bf16_to_f32(b); }

/* ---------------------------------------------------------------- E4M3 --- */

/* fp8.py:22-27 `_e4m3_value`: sign * (m*2^-9 if e==0 else (1+m/8)*2^(e-7)).
 * Codes 0x7F / 0xFF decode to +-480 (the reference has no NaN code). */
double glm53o_e4m3_value(uint8_t byte) {
    double sign = (byte & 0x80) ? -1.0 : 1.0;
    int exponent = (byte >> 3) & 15;
    int mantissa = byte & 7;
    double value = exponent == 0 ? mantissa * ldexp(1.0, -9)
                                 : (1.0 + mantissa / 8.0) * ldexp(1.0, exponent - 7);
    return sign * value;
}

/* fp8.py:37-39 LUT (also native_indexer_plan.metal:19-35). */
void glm53o_e4m3_lut(float* out256) {
    for (int code = 0; code < 256; ++code) out256[code] = (float)glm53o_e4m3_value((uint8_t)code);
}

static double g_lut[256];
static int g_lut_ready = 0;
static void lut_init(void) {
    if (g_lut_ready) return;
    for (int code = 0; code < 256; ++code) g_lut[code] = glm53o_e4m3_value((uint8_t)code);
    g_lut_ready = 1;
}

/* ------------------------------------------------------ block FP8 linear --- */

/*
 * fp8.py:254-299 `block_fp8_linear` (GEMV 41-72 for one row, tiled-8 GEMM
 * 74-116 otherwise; packed.py:304-387 is the same contraction over one bank
 * expert):
 *     y[m, n] = T( sum_k float(x[m, k]) * LUT[w[n, k]] * s[n/128, k/128] )
 * x: bf16 [M, K] (row stride x_stride elements), w: u8 [N, K] row-major,
 * s: f32 [ceil(N/128), s_cols] row-major, y: bf16 [M, N] (row stride
 * y_stride).  Sum in double, then round to FP32 (the reference's accumulator
 * type) and to BF16 (T).
 */
void glm53o_fp8_linear(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride,
                       const uint8_t* w, int64_t N, const float* s, int64_t s_cols,
                       uint16_t* y, int64_t y_stride) {
    lut_init();
    double* xd = (double*)malloc(sizeof(double) * (size_t)(M * K > 0 ? M * K : 1));
    for (int64_t m = 0; m < M; ++m)
        for (int64_t k = 0; k < K; ++k) xd[m * K + k] = bf16_to_f32(x[m * x_stride + k]);
#pragma omp parallel
    {
        double* wd = (double*)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            const uint8_t* wr = w + n * K;
            const float* sr = s + (n / GLM53O_BLOCK) * s_cols;
            for (int64_t k = 0; k < K; ++k) wd[k] = g_lut[wr[k]] * (double)sr[k / GLM53O_BLOCK];
            for (int64_t m = 0; m < M; ++m) {
                const double* xr = xd + m * K;
                double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
                int64_t k = 0;
                for (; k + 4 <= K; k += 4) {
                    a0 += xr[k] * wd[k];
                    a1 += xr[k + 1] * wd[k + 1];
                    a2 += xr[k + 2] * wd[k + 2];
                    a3 += xr[k + 3] * wd[k + 3];
                }
                for (; k < K; ++k) a0 += xr[k] * wd[k];
                double total = (a0 + a1) + (a2 + a3);
                y[m * y_stride + n] = f32_to_bf16((float)total);
            }
        }
        free(wd);
    }
    free(xd);
}

/* Same contraction, FP32 output before the BF16 store (used by the router
 * restatement, which keeps FP32 logits: patch.py:131-142). x is FP32 here. */
void glm53o_f32_linear(const float* x, int64_t M, int64_t K, const float* w, int64_t N, float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        const float* wr = w + n * K;
        for (int64_t m = 0; m < M; ++m) {
            const float* xr = x + m * K;
            double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
            int64_t k = 0;
            for (; k + 4 <= K; k += 4) {
                a0 += (double)xr[k] * wr[k];
                a1 += (double)xr[k + 1] * wr[k + 1];
                a2 += (double)xr[k + 2] * wr[k + 2];
                a3 += (double)xr[k + 3] * wr[k + 3];
            }
            for (; k < K; ++k) a0 += (double)xr[k] * wr[k];
            y[m * N + n] = (float)((a0 + a1) + (a2 + a3));
        }
    }
}

/* -------------------------------------------------------------- SwiGLU --- */

/*
 * MLX BF16 sigmoid as the reference evaluates it (packed.py:155-160, the
 * mx.sigmoid / nn.silu it reproduces, native_indexer_plan.metal:216-223):
 *     tail = 1 / (1 + exp(|g|))   with every step rounded to BF16
 *     sigma = g < 0 ? tail : 1 - tail   (rounded to BF16)
 * MLX evaluates exp with Metal fast::exp.  The reference's exhaustive sweep
 * over all 33,346 finite BF16 values in [-10, 10]
 * (bench-results/m3ultra512-native-routed-sigmoid-formula-sweep-20260907.json)
 * shows fast::exp agrees with the correctly rounded exponential at every
 * point except g = -6.84375 (bits 0xC0DB), where exp(6.84375) =
 * 938.0000478... sits 5e-5 above the BF16 rounding midpoint 938 and
 * fast::exp lands at or below it: BF16 exp = 936, sigma bits 0x3A8C instead
 * of 0x3A8B.  The positive twin g = +6.84375 is unaffected (1 - tail rounds
 * to 1.0 either way).
 */
uint16_t glm53o_sigmoid_bf16(uint16_t gbits) {
    float g = bf16_to_f32(gbits);
    if (isnan(g)) return gbits;
    if (gbits == 0xC0DBu) return 0x3A8Cu;
    float e = bf16_round((float)exp(fabs((double)g)));
    float d = bf16_round(1.0f + e);
    float tail = bf16_round(1.0f / d);
    float sigma = g < 0.0f ? tail : bf16_round(1.0f - tail);
    return f32_to_bf16(sigma);
}

/*
 * Clamped SwiGLU rounding sequence (packed.py:146-163; patch.py:104-112;
 * fp8.py:337-340, 376-378; grouped_fp8.py:265-270):
 *     g' = T(min(g, limit)),  u' = T(clip(u, -limit, limit))
 *     h  = T( T(g' * sigma(g')) * u' )
 */
static inline uint16_t swiglu_one(uint16_t gbits, uint16_t ubits, float limit) {
    float g = bf16_to_f32(gbits);
    float u = bf16_to_f32(ubits);
    float gv = g < limit ? g : limit;
    if (isnan(g)) gv = g;
    float uv = u < -limit ? -limit : (u > limit ? limit : u);
    if (isnan(u)) uv = u;
    uint16_t ga = f32_to_bf16(gv);
    float gaf = bf16_to_f32(ga);
    float ua = bf16_round(uv);
    float sig = bf16_to_f32(glm53o_sigmoid_bf16(ga));
    float silu = bf16_round(gaf * sig);
    return f32_to_bf16(silu * ua);
}

void glm53o_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, float limit, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = swiglu_one(gate[i], up[i], limit);
}

/* ---------------------------------------------------------------- router --- */

/*
 * patch.py:131-142 `Float32Gate` + mlx-vlm 0.6.17 @ e82d557d
 * `dsv32.group_expert_select` (uv.lock:720-723), restated as the published
 * DeepSeek-V3 auxiliary-loss-free rule with n_group = 1
 * (scripts/sweep_grouped_fp8_suffix.py:84-91 restates the weighting half):
 *   logits = x_f32 @ W_f32^T           (FP32)
 *   sig    = sigmoid(logits)            (FP32)
 *   choice = sig + bias                 (FP32, used only for selection)
 *   ids    = top_k(choice), ordered by (choice desc, id asc)
 *   w      = sig[ids]; w /= sum(w) if norm; w *= routed_scaling_factor
 * The ordering rule is this build's documented tie policy; MLX argpartition
 * leaves slot order unspecified.  `choice_out` (optional, [T, E]) returns the
 * biased scores for near-tie analysis.
 */
/*
 * Group-limited selection (the DeepSeek-V3 rule of mlx-vlm
 * dsv32.group_expert_select for n_group > 1; patch.py:134-142 passes
 * n_group and topk_group): groups of E / n_group consecutive experts, group
 * score = FP32 sum of the group's two largest biased scores, and the biased
 * scores of every group outside the topk_group best (equal scores: the lower
 * group index ranks first) set to 0.0 before the top-k.
 */
static void group_limit(float* choice, int64_t E, int64_t n_group, int64_t topk_group) {
    if (n_group <= 1) return;
    const int64_t per = E / n_group;
    float gs[64];
    for (int64_t g = 0; g < n_group; ++g) {
        float m1 = -INFINITY, m2 = -INFINITY;
        for (int64_t e = g * per; e < (g + 1) * per; ++e) {
            const float v = choice[e];
            if (v > m1) {
                m2 = m1;
                m1 = v;
            } else if (v > m2) {
                m2 = v;
            }
        }
        gs[g] = m1 + m2;
    }
    for (int64_t g = 0; g < n_group; ++g) {
        int64_t rank = 0;
        for (int64_t h = 0; h < n_group; ++h)
            if (gs[h] > gs[g] || (gs[h] == gs[g] && h < g)) ++rank;
        if (rank >= topk_group)
            for (int64_t e = g * per; e < (g + 1) * per; ++e) choice[e] = 0.0f;
    }
}

void glm53o_router(const uint16_t* x, int64_t T, int64_t H, const float* w, const float* bias,
                   int64_t E, int64_t top_k, float scaling, int norm, int64_t n_group, int64_t topk_group,
                   int32_t* ids_out, float* scores_out, float* choice_out) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)(T * H));
    float* logits = (float*)malloc(sizeof(float) * (size_t)(T * E));
    for (int64_t i = 0; i < T * H; ++i) xf[i] = bf16_to_f32(x[i]);
    glm53o_f32_linear(xf, T, H, w, E, logits);
    float* sig = (float*)malloc(sizeof(float) * (size_t)E);
    float* choice = (float*)malloc(sizeof(float) * (size_t)E);
    unsigned char* taken = (unsigned char*)malloc((size_t)E);
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t e = 0; e < E; ++e) {
            double l = logits[t * E + e];
            sig[e] = (float)(1.0 / (1.0 + exp(-l)));
            choice[e] = sig[e] + bias[e];
            taken[e] = 0;
        }
        group_limit(choice, E, n_group, topk_group);
        if (choice_out)
            for (int64_t e = 0; e < E; ++e) choice_out[t * E + e] = choice[e];
        float total = 0.0f;
        for (int64_t slot = 0; slot < top_k; ++slot) {
            int64_t best = -1;
            for (int64_t e = 0; e < E; ++e) {
                if (taken[e]) continue;
                if (best < 0 || choice[e] > choice[best]) best = e;
            }
            taken[best] = 1;
            ids_out[t * top_k + slot] = (int32_t)best;
            scores_out[t * top_k + slot] = sig[best];
            total += sig[best];
        }
        for (int64_t slot = 0; slot < top_k; ++slot) {
            float v = scores_out[t * top_k + slot];
            if (top_k > 1 && norm) v = v / total;
            scores_out[t * top_k + slot] = v * scaling;
        }
    }
    free(taken);
    free(choice);
    free(sig);
    free(logits);
    free(xf);
}

/* ------------------------------------------------------- reductions ------ */

/*
 * packed.py:168-179 / 602-621 and fp8.py:457: ordered FP32 weighted top-k
 * reduction, out[h] = T( sum_{s=0..k-1} float(down[s, h]) * score[s] ) with
 * each product rounded to FP32 and summed sequentially in slot order.
 */
void glm53o_weighted_reduction(const uint16_t* down, const float* scores, int64_t k, int64_t H,
                               uint16_t* out) {
    for (int64_t h = 0; h < H; ++h) {
        float total = 0.0f;
        for (int64_t s = 0; s < k; ++s) {
            float contribution = bf16_to_f32(down[s * H + h]) * scores[s];
            total += contribution;
        }
        out[h] = f32_to_bf16(total);
    }
}

/* BF16 + BF16 -> BF16 (packed.py:922; native_indexer_plan.metal:525-535). */
/* native_indexer_plan.metal:2362-2388 (finish_hc of native_prefill_moe_plan.cpp:136-161):
 * out[r, b, d] = T(post[r, b] * moe[r, d] + mixed), mixed = fma chain over
 * s = 0..3 of comb[r, s, b] * residual[r, s, d] from 0 (4 streams). */
void glm53o_hc_expand(const uint16_t* moe, const uint16_t* residual, const float* post, const float* comb,
                      int64_t rows, int64_t hidden, uint16_t* out) {
    for (int64_t r = 0; r < rows; ++r)
        for (int b = 0; b < 4; ++b)
            for (int64_t d = 0; d < hidden; ++d) {
                float mixed = 0.0f;
                for (int src = 0; src < 4; ++src)
                    mixed = fmaf(comb[(r * 4 + src) * 4 + b], bf16_to_f32(residual[(r * 4 + src) * hidden + d]), mixed);
                const float branch = post[r * 4 + b] * bf16_to_f32(moe[r * hidden + d]);
                out[(r * 4 + b) * hidden + d] = f32_to_bf16(branch + mixed);
            }
}

void glm53o_add_bf16(const uint16_t* a, const uint16_t* b, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(bf16_to_f32(a[i]) + bf16_to_f32(b[i]));
}

/*
 * Direct prefill accumulation order (fp8.py:384-397; restated exactly by
 * native_indexer_plan.metal:2174-2207): per token, visit its k routes in
 * ascending expert id; contribution = T(float(route_out) * score);
 * total = T(total + contribution), starting from BF16 zero.
 * route_out is indexed by flat route t*k + slot ([T*k, H] bf16).
 */
void glm53o_direct_order_reduce(const uint16_t* route_out, const int32_t* ids, const float* scores,
                                int64_t T, int64_t k, int64_t H, uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        int32_t order[64];
        int64_t kk = k < 64 ? k : 64;
        for (int64_t s = 0; s < kk; ++s) order[s] = (int32_t)s;
        /* stable insertion sort of slots by expert id */
        for (int64_t a = 1; a < kk; ++a) {
            int32_t v = order[a];
            int64_t b = a - 1;
            while (b >= 0 && ids[t * k + order[b]] > ids[t * k + v]) {
                order[b + 1] = order[b];
                --b;
            }
            order[b + 1] = v;
        }
        for (int64_t h = 0; h < H; ++h) {
            float total = 0.0f;
            for (int64_t r = 0; r < kk; ++r) {
                int64_t route = t * k + order[r];
                float contribution = bf16_round(bf16_to_f32(route_out[route * H + h]) * scores[route]);
                total = bf16_round(total + contribution);
            }
            out[t * H + h] = f32_to_bf16(total);
        }
    }
}

/*
 * Grouped prefill reduction (grouped_fp8.py:273-276):
 *   weighted = sorted_output * sorted_scores[:, None]   (FP32 products)
 *   y[t] = T( sum_slot weighted[inverse[t*k + slot]] )  (FP32, slot order)
 */
void glm53o_restore_and_reduce(const uint16_t* sorted_out, const float* sorted_scores,
                               const int64_t* inverse, int64_t T, int64_t k, int64_t H, uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t h = 0; h < H; ++h) {
            float total = 0.0f;
            for (int64_t s = 0; s < k; ++s) {
                int64_t row = inverse[t * k + s];
                total += bf16_to_f32(sorted_out[row * H + h]) * sorted_scores[row];
            }
            out[t * H + h] = f32_to_bf16(total);
        }
    }
}

int glm53o_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void glm53o_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
