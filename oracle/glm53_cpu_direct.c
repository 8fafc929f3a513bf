/*
 * glm53_cpu_direct.c -- the benchmark's CPU comparator: the reference's
 * Direct FP8 MoE path evaluated with FP32 accumulation on the host cores
 * (OpenMP, AVX2 FMA), the role the task gives to MLX's CPU stream (the
 * reference itself has no CPU FP8 path: fp8.py:118-139, 256-257).
 * MEASUREMENT AND TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times
 * it and tests/ check it against the float64 oracle; the product path never
 * links or calls it.
 *
 * Semantics restated (paths relative to the kiojuvr/glm53-flash-mlx root):
 *   block_fp8_linear   fp8.py:41-116, 254-299: y = T(sum_k x_k * (LUT[w] * s))
 *   E4M3 table         fp8.py:22-39 (0x7F / 0xFF = +-480, no NaN code)
 *   FP32 router        patch.py:131-142: logits = x_f32 . W_f32^T, sigmoid,
 *                      top-k of sigmoid + bias (ties: lower id), weights =
 *                      sigmoid of the picks, normalised, x scaling factor
 *   SwiGLU             packed.py:146-163 / patch.py:104-112, MLX BF16 steps
 *   decode (T = 1)     fp8.py:372-383: FP32 slot-order sum of T(down_s) w_s
 *   prefill            fp8.py:384-397 (order restated at
 *                      native_indexer_plan.metal:2174-2207): experts in
 *                      ascending id, result = T(result + T(out * w)) in BF16
 *   shared add         packed.py:922: T(T(routed) + T(shared))
 * Dot products accumulate in FP32 in the order the vectorised loop takes
 * (8-wide partial sums), so outputs differ from the exactly rounded float64
 * oracle by an occasional BF16 ulp, as the reference's own Metal FP32 sums do.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define BLK 128

static inline float bf16f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float rbf(float f) { return bf16f(f2bf(f)); }

static float g_lut[256];
static int g_lut_ready = 0;

/* fp8.py:22-39: sign * (m 2^-9 if e == 0 else (1 + m / 8) 2^(e - 7)) for
 * every code (0x7F / 0xFF = +-480); a table lookup per weight byte is the
 * fastest host decode measured (a branch-free bit form ran 8x slower). */
static void lut_init(void) {
    if (g_lut_ready) return;
    for (int c = 0; c < 256; ++c) {
        const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
        const double v = e == 0 ? m * ldexp(1.0, -9) : (1.0 + m / 8.0) * ldexp(1.0, e - 7);
        g_lut[c] = (float)(s ? -v : v);
    }
    g_lut_ready = 1;
}

/* out[i] = the value of code c[i] (checked against the table in tests/). */
void glm53c_decode_codes(const uint8_t* c, int64_t n, float* out) {
    lut_init();
    for (int64_t i = 0; i < n; ++i) out[i] = g_lut[c[i]];
}

/* y[m, n] = T(sum_k x[m, k] * LUT[w[n, k]] * s[n / 128, k / 128]) with FP32
 * accumulation.  x bf16 [M, K] (row stride K), w u8 [N, K], s f32 [ceil(N /
 * 128), ceil(K / 128)], y bf16 [M, N] (row stride y_stride).  Threads take
 * blocks of 16 weight rows, dequantise them once (the tiled tree x . (LUT .
 * s), fp8.py:74-116) and reduce every activation row against them, four
 * weight rows per pass. */
void glm53c_linear(const uint16_t* x, int64_t M, int64_t K, const uint8_t* w, int64_t N, const float* s,
                   uint16_t* y, int64_t y_stride) {
    lut_init();
    const int64_t SC = (K + BLK - 1) / BLK;
    float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
    for (int64_t i = 0; i < M * K; ++i) xf[i] = bf16f(x[i]);
    const int64_t NB = 16;
#pragma omp parallel
    {
        float* wf = (float*)malloc(sizeof(float) * (size_t)(NB * K));
#pragma omp for schedule(dynamic, 1)
        for (int64_t n0 = 0; n0 < N; n0 += NB) {
            const int64_t nb = N - n0 < NB ? N - n0 : NB;
            for (int64_t j = 0; j < nb; ++j) {
                const uint8_t* wr = w + (n0 + j) * K;
                const float* sr = s + ((n0 + j) / BLK) * SC;
                float* dst = wf + j * K;
                for (int64_t k0 = 0; k0 < K; k0 += BLK) {
                    const int64_t k1 = k0 + BLK < K ? k0 + BLK : K;
                    const float sc = sr[k0 / BLK];
                    for (int64_t k = k0; k < k1; ++k) dst[k] = g_lut[wr[k]] * sc;
                }
            }
            for (int64_t m = 0; m < M; ++m) {
                const float* xr = xf + m * K;
                int64_t j = 0;
                for (; j + 4 <= nb; j += 4) {
                    const float *w0 = wf + j * K, *w1 = w0 + K, *w2 = w1 + K, *w3 = w2 + K;
                    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma omp simd reduction(+ : a0, a1, a2, a3)
                    for (int64_t k = 0; k < K; ++k) {
                        const float xv = xr[k];
                        a0 += xv * w0[k];
                        a1 += xv * w1[k];
                        a2 += xv * w2[k];
                        a3 += xv * w3[k];
                    }
                    uint16_t* yr = y + m * y_stride + n0 + j;
                    yr[0] = f2bf(a0);
                    yr[1] = f2bf(a1);
                    yr[2] = f2bf(a2);
                    yr[3] = f2bf(a3);
                }
                for (; j < nb; ++j) {
                    const float* w0 = wf + j * K;
                    float a0 = 0.0f;
#pragma omp simd reduction(+ : a0)
                    for (int64_t k = 0; k < K; ++k) a0 += xr[k] * w0[k];
                    y[m * y_stride + n0 + j] = f2bf(a0);
                }
            }
        }
        free(wf);
    }
    free(xf);
}

/* MLX BF16 sigmoid (packed.py:155-160): e = T(exp|g|), tail = T(1 / T(1 +
 * e)); sigma = tail for negative g, T(1 - tail) otherwise. */
static inline float sigmoid_bf16(float g) {
    if (isnan(g)) return g;
    const float tail = rbf(1.0f / rbf(1.0f + rbf(expf(fabsf(g)))));
    return g < 0.0f ? tail : rbf(1.0f - tail);
}

/* packed.py:146-163: h = T(T(g' * sigmoid(g')) * u'), g' = T(min(g, L)),
 * u' = T(clip(u, -L, L)), NaN passing through both clamps. */
static inline uint16_t swiglu1(uint16_t gb, uint16_t ub, float L) {
    const float g = bf16f(gb), u = bf16f(ub);
    const float gc = isnan(g) ? g : rbf(g < L ? g : L);
    const float uc = isnan(u) ? u : rbf(u < -L ? -L : (u > L ? L : u));
    return f2bf(rbf(gc * sigmoid_bf16(gc)) * uc);
}

/* patch.py:131-142 for T tokens: FP32 logits, then top_k of sigmoid + bias
 * ordered (value desc, id asc), weights = sigmoid of the picks normalised
 * (norm != 0) times the scaling factor. */
void glm53c_router(const uint16_t* x, int64_t T, int64_t H, const float* w, const float* bias, int64_t E,
                   int64_t top_k, float scaling, int norm, int32_t* ids, float* scores) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        float* xf = (float*)malloc(sizeof(float) * (size_t)H);
        float* sig = (float*)malloc(sizeof(float) * (size_t)E);
        for (int64_t h = 0; h < H; ++h) xf[h] = bf16f(x[t * H + h]);
        for (int64_t e = 0; e < E; ++e) {
            const float* wr = w + e * H;
            float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
            for (int64_t h = 0; h < H; ++h) acc += xf[h] * wr[h];
            sig[e] = 1.0f / (1.0f + expf(-acc));
        }
        float total = 0.0f;
        for (int64_t j = 0; j < top_k; ++j) {
            int64_t best = -1;
            float bv = 0.0f;
            for (int64_t e = 0; e < E; ++e) {
                int taken = 0;
                for (int64_t i = 0; i < j; ++i) taken |= ids[t * top_k + i] == e;
                if (taken) continue;
                const float v = sig[e] + bias[e];
                if (best < 0 || v > bv) {
                    best = e;
                    bv = v;
                }
            }
            ids[t * top_k + j] = (int32_t)best;
            scores[t * top_k + j] = sig[best];
            total += sig[best];
        }
        for (int64_t j = 0; j < top_k; ++j)
            scores[t * top_k + j] = (norm ? scores[t * top_k + j] / total : scores[t * top_k + j]) * scaling;
        free(xf);
        free(sig);
    }
}

/* One expert (fp8.py:329-340) over rows x [R, H] -> out [R, H]:
 * down(swiglu(T(x . Wg), T(x . Wu))). gate rows and up rows are I x H
 * matrices, down is H x I. */
static void expert_forward(const uint16_t* x, int64_t R, int64_t H, int64_t I, const uint8_t* gw, const float* gs,
                           const uint8_t* uw, const float* us, const uint8_t* dw, const float* ds, float L,
                           uint16_t* out) {
    uint16_t* g = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(R * I));
    uint16_t* u = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(R * I));
    glm53c_linear(x, R, H, gw, I, gs, g, I);
    glm53c_linear(x, R, H, uw, I, us, u, I);
    for (int64_t i = 0; i < R * I; ++i) g[i] = swiglu1(g[i], u[i], L);
    glm53c_linear(g, R, I, dw, H, ds, out, H);
    free(g);
    free(u);
}

/* DirectFP8MoE.__call__ (fp8.py:343-400) on the routes ids / scores [T, k]
 * (from glm53c_router or the caller) over a bank in the reference layout
 * (packed.py:782-850: gate_up [E, 2I, H], scales [E, 2 ceil(I/128),
 * ceil(H/128)], down [E, H, I], scales [E, ceil(H/128), ceil(I/128)]) and an
 * optional shared expert of width Is (sg / su [Is, H], sd [H, Is]; sg NULL:
 * none).  out bf16 [T, H]. */
void glm53c_direct_moe(const uint16_t* x, int64_t T, int64_t H, int64_t I, int64_t k, const int32_t* ids,
                       const float* scores, const uint8_t* gate_up, const float* gate_up_s, const uint8_t* down,
                       const float* down_s, const uint8_t* sg, const float* sgs, const uint8_t* su,
                       const float* sus, const uint8_t* sd, const float* sds, int64_t Is, float L, uint16_t* out) {
    const int64_t SR = (I + BLK - 1) / BLK, SH = (H + BLK - 1) / BLK;
    const int64_t E_stride_gu = 2 * I * H, E_stride_gus = 2 * SR * SH, E_stride_d = H * I, E_stride_ds = SH * SR;
    uint16_t* route_out = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * k * H));
    /* buckets in ascending expert id (fp8.py:384-397) */
    int32_t emax = 0;
    for (int64_t r = 0; r < T * k; ++r) emax = ids[r] > emax ? ids[r] : emax;
    int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)(T * k));
    uint16_t* xb = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * k * H));
    uint16_t* ob = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * k * H));
    for (int32_t e = 0; e <= emax; ++e) {
        int64_t n = 0;
        for (int64_t r = 0; r < T * k; ++r)
            if (ids[r] == e) rows[n++] = r;
        if (n == 0) continue;
        for (int64_t i = 0; i < n; ++i) memcpy(xb + i * H, x + (rows[i] / k) * H, sizeof(uint16_t) * (size_t)H);
        const uint8_t* gw = gate_up + e * E_stride_gu;
        const float* gsc = gate_up_s + e * E_stride_gus;
        expert_forward(xb, n, H, I, gw, gsc, gw + I * H, gsc + SR * SH, down + e * E_stride_d,
                       down_s + e * E_stride_ds, L, ob);
        for (int64_t i = 0; i < n; ++i) memcpy(route_out + rows[i] * H, ob + i * H, sizeof(uint16_t) * (size_t)H);
    }
    if (T == 1) {
        /* decode: FP32 slot-order weighted sum (fp8.py:372-383) */
        for (int64_t h = 0; h < H; ++h) {
            float acc = 0.0f;
            for (int64_t s = 0; s < k; ++s) acc += bf16f(route_out[s * H + h]) * scores[s];
            out[h] = f2bf(acc);
        }
    } else {
        /* prefill: ascending expert, BF16 accumulation of T(out * w) */
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < T; ++t) {
            int order[64];
            for (int64_t s = 0; s < k; ++s) order[s] = (int)s;
            for (int64_t a = 1; a < k; ++a)
                for (int64_t b = a; b > 0 && ids[t * k + order[b]] < ids[t * k + order[b - 1]]; --b) {
                    const int tmp = order[b];
                    order[b] = order[b - 1];
                    order[b - 1] = tmp;
                }
            for (int64_t h = 0; h < H; ++h) {
                float total = 0.0f;
                for (int64_t j = 0; j < k; ++j) {
                    const int64_t s = order[j];
                    total = rbf(total + rbf(bf16f(route_out[(t * k + s) * H + h]) * scores[t * k + s]));
                }
                out[t * H + h] = f2bf(total);
            }
        }
    }
    if (sg != NULL) {
        uint16_t* sh = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(T * H));
        expert_forward(x, T, H, Is, sg, sgs, su, sus, sd, sds, L, sh);
        for (int64_t i = 0; i < T * H; ++i) out[i] = f2bf(bf16f(out[i]) + bf16f(sh[i]));
        free(sh);
    }
    free(rows);
    free(xb);
    free(ob);
    free(route_out);
}

int glm53c_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
