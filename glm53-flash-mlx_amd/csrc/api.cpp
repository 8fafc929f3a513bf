// C ABI of libglm53_moe.so (declared in include/glm53_moe.h).
//
// Host-side validation, plan objects with fixed device scratch, and the
// launch schedules of the decode and prefill paths.  No C++ exception
// crosses the boundary: every entry point returns a status code and leaves a
// thread-local message for glm53_last_error().
#include <glm53_moe.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "grouped.h"
#include "kernels.h"
#include "layout.h"
#include "synth.h"

using namespace glm53;

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(GLM53_DEVICE_ERROR, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                      \
  do {                                           \
    hipError_t _e = (expr);                      \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

#define CHECK_ARG(cond, ...)                                        \
  do {                                                              \
    if (!(cond)) return fail(GLM53_INVALID_ARGUMENT, __VA_ARGS__);  \
  } while (0)

inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline size_t round_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// Bytes of the hi/lo/scale split of a [rows, cols] activation matrix.
size_t split_bytes(int64_t rows, int64_t cols) {
  return 2 * round_up(static_cast<size_t>(rows * cols)) + round_up(sizeof(float) * static_cast<size_t>(rows * (cols / 128)));
}

struct SplitBuf {
  uint8_t* hi;
  uint8_t* lo;
  float* scale;
};

SplitBuf carve_split(void* base, int64_t rows, int64_t cols) {
  uint8_t* p = static_cast<uint8_t*>(base);
  SplitBuf b;
  b.hi = p;
  p += round_up(static_cast<size_t>(rows * cols));
  b.lo = p;
  p += round_up(static_cast<size_t>(rows * cols));
  b.scale = reinterpret_cast<float*>(p);
  return b;
}

hipError_t split(const void* x, int64_t rows, int64_t cols, const SplitBuf& b, hipStream_t st) {
  SplitArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_row_stride = cols;
  a.rows = rows;
  a.cols = cols;
  a.hi = b.hi;
  a.lo = b.lo;
  a.scale = b.scale;
  return launch_split_activations(a, st);
}

int check_linear(const glm53_linear& l, int64_t out, int64_t in, const char* name) {
  CHECK_ARG(l.weight != nullptr && l.scale_inv != nullptr, "%s: null weight or scale", name);
  CHECK_ARG(l.out_features == out && l.in_features == in, "%s: shape [%lld, %lld] != expected [%lld, %lld]", name,
            (long long)l.out_features, (long long)l.in_features, (long long)out, (long long)in);
  return GLM53_OK;
}

int check_bank(const glm53_bank* b, int64_t H, int64_t I, int64_t E) {
  CHECK_ARG(b != nullptr, "bank is null");
  CHECK_ARG(b->gate_up_weight && b->gate_up_scale_inv && b->down_weight && b->down_scale_inv,
            "bank has a null buffer");
  CHECK_ARG(b->hidden == H && b->intermediate == I && b->experts == E,
            "bank shape (E=%lld, H=%lld, I=%lld) != plan (E=%lld, H=%lld, I=%lld)", (long long)b->experts,
            (long long)b->hidden, (long long)b->intermediate, (long long)E, (long long)H, (long long)I);
  CHECK_ARG(b->row_group_log2 >= 0 && b->row_group_log2 <= GLM53_MAX_ROW_GROUP_LOG2,
            "bank row_group_log2 %d outside [0, %d]", (int)b->row_group_log2, GLM53_MAX_ROW_GROUP_LOG2);
  CHECK_ARG(b->row_group_log2 == 0 || (H % 128 == 0 && I % 128 == 0),
            "a row-group bank needs hidden and intermediate multiples of 128 (H=%lld, I=%lld)", (long long)H,
            (long long)I);
  return GLM53_OK;
}

// A bank handle: the descriptor handed out (first, so the pointer returned
// is the handle's) and the device buffers the handle owns -- the code flag,
// and for an imported bank the re-laid weights and the copied scales.
struct BankHandle {
  glm53_bank pub;
  void* owned[5];
};

int check_layout_args(int64_t matrices, int64_t rows, int64_t cols, int32_t from_log2, int32_t to_log2) {
  CHECK_ARG(matrices >= 0 && rows >= 0 && cols >= 0, "invalid dimensions");
  CHECK_ARG(from_log2 >= 0 && from_log2 <= GLM53_MAX_ROW_GROUP_LOG2 && to_log2 >= 0 &&
                to_log2 <= GLM53_MAX_ROW_GROUP_LOG2,
            "row_group_log2 must lie in [0, %d]", GLM53_MAX_ROW_GROUP_LOG2);
  CHECK_ARG((rows * cols) % 16 == 0, "rows * cols must be a multiple of 16");
  if (from_log2 > 0 || to_log2 > 0) {
    const int64_t group = int64_t{1} << std::max(from_log2, to_log2);
    CHECK_ARG(cols % 128 == 0, "a row-group layout needs cols % 128 == 0 (cols=%lld)", (long long)cols);
    CHECK_ARG(rows % group == 0, "rows (%lld) must be a multiple of the row group (%lld)", (long long)rows,
              (long long)group);
  } else {
    CHECK_ARG(cols % 16 == 0, "cols must be a multiple of 16");
  }
  return GLM53_OK;
}

// Group-limited selection of a router (0 in either field reads as 1, the
// ungrouped selection).
int router_groups(const glm53_router* r) { return r->n_group > 0 ? r->n_group : 1; }
int router_topk_groups(const glm53_router* r) { return r->topk_group > 0 ? r->topk_group : 1; }

int check_groups(const glm53_router* r) {
  const int64_t n = router_groups(r), t = router_topk_groups(r), E = r->experts;
  CHECK_ARG(n <= 64, "n_group must be at most 64");
  CHECK_ARG(t <= n, "topk_group %lld exceeds n_group %lld", (long long)t, (long long)n);
  if (n > 1) {
    CHECK_ARG(E % n == 0 && E / n >= 2, "n_group %lld must divide %lld experts into groups of two or more",
              (long long)n, (long long)E);
    CHECK_ARG(r->top_k <= t * (E / n), "top_k %lld exceeds the %lld experts of %lld kept groups", (long long)r->top_k,
              (long long)(t * (E / n)), (long long)t);
  }
  return GLM53_OK;
}

int check_router(const glm53_router* r, int64_t H, int64_t E, int64_t k) {
  CHECK_ARG(r != nullptr && r->weight != nullptr && r->bias != nullptr, "router weight/bias is null");
  CHECK_ARG(E <= kMaxRouterExperts, "router experts must be at most %d", kMaxRouterExperts);
  CHECK_ARG(r->hidden == H && r->experts == E, "router shape [%lld, %lld] != [%lld, %lld]", (long long)r->experts,
            (long long)r->hidden, (long long)E, (long long)H);
  CHECK_ARG(r->top_k == k, "router top_k %lld != plan top_k %lld", (long long)r->top_k, (long long)k);
  return check_groups(r);
}

int topk(const float* logits, const glm53_router* r, int64_t T, int32_t* ids, float* scores, hipStream_t st,
         int splits = 1, int64_t split_stride = 0) {
  TopkArgs a{};
  a.logits = logits;
  a.splits = splits;
  a.split_stride = split_stride;
  a.bias = r->bias;
  a.tokens = T;
  a.experts = r->experts;
  a.top_k = static_cast<int>(r->top_k);
  a.routed_scaling_factor = r->routed_scaling_factor;
  a.norm_topk_prob = r->norm_topk_prob;
  a.n_group = router_groups(r);
  a.topk_group = router_topk_groups(r);
  a.ids_out = ids;
  a.scores_out = scores;
  HIP_TRY(launch_topk(a, st), "topk launch");
  return GLM53_OK;
}

// Router logits and selection for T > 1 tokens.  Where the shape allows
// (hidden % 128 == 0, 16-byte aligned rows) the BF16-MFMA tile kernel writes
// FP32 partial sums per K chunk (up to kMaxRouterSplits planes of T x E) to
// `space` and the selection adds them in chunk order; other shapes compute
// the FP32 logits per (expert, token) into `logits`.
size_t router_space_bytes(int64_t T, int64_t E) {
  return sizeof(float) * static_cast<size_t>(T) * static_cast<size_t>(kMaxRouterSplits * E);
}

int route_tokens(const glm53_router* r, const void* x, int64_t T, float* space, float* logits, int32_t* ids,
                 float* scores, hipStream_t st) {
  const int64_t H = r->hidden, E = r->experts;
  if (router_gemm_supported(H, E, x, r->weight)) {
    const RouterGemmShape shape = router_gemm_shape(T, H, E);
    RouterGemmArgs g{};
    g.x = static_cast<const uint16_t*>(x);
    g.partial = space;
    g.tokens = T;
    g.hidden = H;
    g.experts = E;
    g.token_groups = shape.token_groups;
    g.expert_groups = shape.expert_groups;
    g.k_chunk = shape.k_chunk;
    g.splits = shape.splits;
    HIP_TRY(launch_router_logits(g, r->weight, st), "router logits launch");
    return topk(g.partial, r, T, ids, scores, st, static_cast<int>(shape.splits), T * E);
  }
  RouterArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.weight = r->weight;
  a.experts = E;
  a.hidden = H;
  a.tokens = T;
  a.logits_out = logits;
  HIP_TRY(launch_router(a, st), "router launch");
  return topk(logits, r, T, ids, scores, st);
}

}  // namespace

extern "C" {

const char* glm53_last_error(void) { return g_error.c_str(); }
int glm53_abi_version(void) { return GLM53_ABI_VERSION; }

// ------------------------------------------------------------ linear ------

size_t glm53_fp8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 1 || K <= 0 || K % 128 != 0 || N % 16 != 0) return 0;
  return split_bytes(M, K) + 256;  // + the 0x7F/0xFF code flag
}

int glm53_e4m3_scan_codes(const uint8_t* codes, int64_t n, int32_t* flag, void* stream) {
  CHECK_ARG(n >= 0 && flag != nullptr && (n == 0 || codes != nullptr), "invalid arguments");
  CHECK_ARG(aligned(codes, 16) || n < 16, "codes must be 16-byte aligned");
  HIP_TRY(launch_scan_480(codes, n, flag, true, S(stream)), "scan launch");
  return GLM53_OK;
}

int glm53_relayout_weights(const uint8_t* src, uint8_t* dst, int64_t matrices, int64_t rows, int64_t cols,
                           int32_t from_log2, int32_t to_log2, void* stream) {
  int rc = check_layout_args(matrices, rows, cols, from_log2, to_log2);
  if (rc) return rc;
  const int64_t bytes = matrices * rows * cols;
  if (bytes == 0) return GLM53_OK;
  CHECK_ARG(src && dst, "null pointer argument");
  CHECK_ARG(aligned(src, 16) && aligned(dst, 16), "weights must be 16-byte aligned");
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
  CHECK_ARG(s0 + static_cast<uintptr_t>(bytes) <= d0 || d0 + static_cast<uintptr_t>(bytes) <= s0,
            "source and destination overlap (the re-lay is out of place)");
  RelayoutArgs a{src, dst, rows, cols, matrices, rows * cols, from_log2, to_log2};
  HIP_TRY(launch_relayout(a, S(stream)), "relayout launch");
  return GLM53_OK;
}

int glm53_bank_create(const glm53_bank* desc, void* stream, glm53_bank** out) {
  CHECK_ARG(desc != nullptr && out != nullptr, "null pointer argument");
  *out = nullptr;
  CHECK_ARG(desc->gate_up_weight && desc->gate_up_scale_inv && desc->down_weight && desc->down_scale_inv,
            "null bank tensor");
  CHECK_ARG(desc->experts > 0 && desc->hidden > 0 && desc->intermediate > 0, "invalid bank dimensions");
  CHECK_ARG(aligned(desc->gate_up_weight, 16) && aligned(desc->down_weight, 16),
            "bank weights must be 16-byte aligned");
  int rc = check_bank(desc, desc->hidden, desc->intermediate, desc->experts);
  if (rc) return rc;
  int32_t* flag = nullptr;
  HIP_TRY(hipMalloc(&flag, sizeof(int32_t)), "bank code flag hipMalloc");
  const int64_t gu = desc->experts * 2 * desc->intermediate * desc->hidden;
  const int64_t dn = desc->experts * desc->hidden * desc->intermediate;
  hipError_t e = launch_scan_480(desc->gate_up_weight, gu, flag, true, S(stream));
  if (e == hipSuccess) e = launch_scan_480(desc->down_weight, dn, flag, false, S(stream));
  if (e != hipSuccess) {
    (void)hipFree(flag);
    return hip_fail(e, "bank code scan");
  }
  auto* b = new BankHandle{};
  b->pub = *desc;
  b->pub.code_flags = flag;
  b->owned[0] = flag;
  *out = &b->pub;
  return GLM53_OK;
}

int glm53_bank_import(const glm53_bank* desc, int32_t row_group_log2, void* stream, glm53_bank** out) {
  CHECK_ARG(desc != nullptr && out != nullptr, "null pointer argument");
  *out = nullptr;
  CHECK_ARG(desc->gate_up_weight && desc->gate_up_scale_inv && desc->down_weight && desc->down_scale_inv,
            "null bank tensor");
  CHECK_ARG(desc->experts > 0 && desc->hidden > 0 && desc->intermediate > 0, "invalid bank dimensions");
  const int64_t E = desc->experts, H = desc->hidden, I = desc->intermediate;
  int rc = check_bank(desc, H, I, E);
  if (rc) return rc;
  glm53_bank want = *desc;
  want.row_group_log2 = row_group_log2;
  if ((rc = check_bank(&want, H, I, E))) return rc;
  if ((rc = check_layout_args(E, 2 * I, H, desc->row_group_log2, row_group_log2))) return rc;
  if ((rc = check_layout_args(E, H, I, desc->row_group_log2, row_group_log2))) return rc;
  CHECK_ARG(aligned(desc->gate_up_weight, 16) && aligned(desc->down_weight, 16),
            "bank weights must be 16-byte aligned");
  const size_t gu = static_cast<size_t>(E * 2 * I * H), dn = static_cast<size_t>(E * H * I);
  const size_t gus = sizeof(float) * static_cast<size_t>(E * 2 * cdiv(I, 128) * cdiv(H, 128));
  const size_t dns = sizeof(float) * static_cast<size_t>(E * cdiv(H, 128) * cdiv(I, 128));
  hipStream_t st = S(stream);
  auto* b = new BankHandle{};
  auto cleanup = [&](int code) {
    for (void* q : b->owned)
      if (q) (void)hipFree(q);
    delete b;
    return code;
  };
  const size_t sizes[5] = {sizeof(int32_t), gu, gus, dn, dns};
  for (int i = 0; i < 5; ++i) {
    hipError_t e = hipMalloc(&b->owned[i], sizes[i]);
    if (e != hipSuccess) return cleanup(hip_fail(e, "bank import hipMalloc"));
  }
  uint8_t* gw = static_cast<uint8_t*>(b->owned[1]);
  uint8_t* dw = static_cast<uint8_t*>(b->owned[3]);
  RelayoutArgs r1{desc->gate_up_weight, gw, 2 * I, H, E, 2 * I * H, desc->row_group_log2, row_group_log2};
  RelayoutArgs r2{desc->down_weight, dw, H, I, E, H * I, desc->row_group_log2, row_group_log2};
  hipError_t e = launch_relayout(r1, st);
  if (e == hipSuccess) e = launch_relayout(r2, st);
  if (e == hipSuccess) e = hipMemcpyAsync(b->owned[2], desc->gate_up_scale_inv, gus, hipMemcpyDeviceToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(b->owned[4], desc->down_scale_inv, dns, hipMemcpyDeviceToDevice, st);
  int32_t* flag = static_cast<int32_t*>(b->owned[0]);
  if (e == hipSuccess) e = launch_scan_480(gw, static_cast<int64_t>(gu), flag, true, st);
  if (e == hipSuccess) e = launch_scan_480(dw, static_cast<int64_t>(dn), flag, false, st);
  // the caller's buffers may be released once this returns
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return cleanup(hip_fail(e, "bank import"));
  b->pub = want;
  b->pub.gate_up_weight = gw;
  b->pub.gate_up_scale_inv = static_cast<const float*>(b->owned[2]);
  b->pub.down_weight = dw;
  b->pub.down_scale_inv = static_cast<const float*>(b->owned[4]);
  b->pub.code_flags = flag;
  *out = &b->pub;
  return GLM53_OK;
}

void glm53_bank_destroy(glm53_bank* bank) {
  if (bank == nullptr) return;
  auto* b = reinterpret_cast<BankHandle*>(bank);
  for (void* q : b->owned)
    if (q) (void)hipFree(q);
  delete b;
}

int glm53_fp8_linear(const void* x, int64_t M, int64_t K, const uint8_t* weight, int64_t N, const float* scale_inv,
                     const int32_t* code_flags, void* y, void* workspace, size_t workspace_bytes, void* stream) {
  CHECK_ARG(M >= 0 && K > 0 && N > 0, "invalid shape M=%lld K=%lld N=%lld", (long long)M, (long long)K, (long long)N);
  if (M == 0) return GLM53_OK;
  CHECK_ARG(x && weight && scale_inv && y, "null pointer argument");
  hipStream_t st = S(stream);
  if (M == 1 && fast_width_supported(K) && aligned(x, 16) && aligned(weight, 16)) {
    GemvArgs a{};
    a.x = static_cast<const uint16_t*>(x);
    a.weight = weight;
    a.scale = scale_inv;
    a.N = N;
    a.K = K;
    a.rows_per_wave = 4;
    a.y = static_cast<uint16_t*>(y);
    a.flags = code_flags;
    HIP_TRY(launch_gemv(a, st), "gemv launch");
    return GLM53_OK;
  }
  if (M == 1 && split_width_supported(K) && aligned(x, 16) && aligned(weight, 16)) {
    GemvArgs a{};
    a.x = static_cast<const uint16_t*>(x);
    a.weight = weight;
    a.scale = scale_inv;
    a.N = N;
    a.K = K;
    a.rows_per_wave = 4;  // rows per workgroup of K / 4096 wavefronts
    a.y = static_cast<uint16_t*>(y);
    a.flags = code_flags;
    HIP_TRY(launch_gemv_split(a, st), "split gemv launch");
    return GLM53_OK;
  }
  const size_t need = glm53_fp8_linear_workspace_bytes(M, N, K);
  if (need > 0 && aligned(weight, 16) && workspace != nullptr && workspace_bytes >= need) {
    SplitBuf b = carve_split(workspace, M, K);
    const int32_t* flag = code_flags;
    if (flag == nullptr) {
      int32_t* f = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + split_bytes(M, K));
      HIP_TRY(launch_scan_480(weight, N * K, f, true, st), "scan launch");
      flag = f;
    }
    HIP_TRY(split(x, M, K, b, st), "split launch");
    GroupedGemmArgs g{};
    g.fixup = flag;
    g.a_hi = b.hi;
    g.a_lo = b.lo;
    g.a_scale = b.scale;
    g.K = K;
    g.routes = M;
    g.experts = 1;
    g.weight = weight;
    g.scale = scale_inv;
    g.s_cols = K / 128;
    g.N = N;
    g.out = static_cast<uint16_t*>(y);
    g.out_row_stride = N;
    HIP_TRY(launch_grouped_gemm(g, GEMM_PLAIN, cdiv(M, kGemmTileRows), st), "grouped gemm launch");
    return GLM53_OK;
  }
  GenericLinearArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_row_stride = K;
  a.weight = weight;
  a.scale = scale_inv;
  a.s_cols = cdiv(K, 128);
  a.M = M;
  a.G = 1;
  a.N = N;
  a.K = K;
  a.rows_per_wave = 4;
  a.tile_rows = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kGenericRows, 16384 / K)));
  a.y = static_cast<uint16_t*>(y);
  a.y_row_stride = N;
  CHECK_ARG(K <= 16384, "generic path supports K <= 16384");
  HIP_TRY(launch_linear_generic(a, st), "generic linear launch");
  return GLM53_OK;
}

// ------------------------------------------------------------ router ------

size_t glm53_router_workspace_bytes(int64_t tokens, int64_t hidden, int64_t experts) {
  if (tokens <= 1) return round_up(sizeof(float) * experts);
  return round_up(router_space_bytes(tokens, experts)) + round_up(sizeof(float) * tokens * experts);
}

int glm53_router_topk(const glm53_router* router, const void* x, int64_t tokens, int32_t* ids, float* scores,
                      void* workspace, size_t workspace_bytes, void* stream) {
  CHECK_ARG(router && router->weight && router->bias, "router is null");
  CHECK_ARG(router->experts > 0 && router->experts <= kMaxRouterExperts, "router experts must be in [1, %d]",
            kMaxRouterExperts);
  CHECK_ARG(router->top_k > 0 && router->top_k <= kMaxTopK && router->top_k <= router->experts,
            "top_k must be in [1, %d]", kMaxTopK);
  if (int rc = check_groups(router)) return rc;
  CHECK_ARG(tokens >= 0, "tokens < 0");
  if (tokens == 0) return GLM53_OK;
  CHECK_ARG(x && ids && scores, "null pointer argument");
  CHECK_ARG(workspace_bytes >= glm53_router_workspace_bytes(tokens, router->hidden, router->experts) && workspace,
            "router workspace too small");
  hipStream_t st = S(stream);
  if (tokens == 1) {
    float* logits = static_cast<float*>(workspace);
    RouterArgs a{};
    a.x = static_cast<const uint16_t*>(x);
    a.weight = router->weight;
    a.experts = router->experts;
    a.hidden = router->hidden;
    a.logits_out = logits;
    HIP_TRY(launch_router(a, st), "router launch");
    return topk(logits, router, 1, ids, scores, st);
  }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* space = reinterpret_cast<float*>(ws);
  float* logits = reinterpret_cast<float*>(ws + round_up(router_space_bytes(tokens, router->experts)));
  return route_tokens(router, x, tokens, space, logits, ids, scores, st);
}

// ------------------------------------------------------------ decode ------

namespace {

// What one three-launch decode step reads and writes besides its inputs and
// outputs: the plan's arena, or the library's static scratch for callers
// that cannot allocate (glm53_decode_moe_static).
struct StepContext {
  int64_t H, I, Is, E, k;
  float limit;
  uint16_t* hidden;                  // [(k + 1) * max(I, Is)] SwiGLU rows: routed slots, then shared
  unsigned long long* route_words;   // [E] launch-1 router words
  uint32_t* router_count;            // launch-1 arrival counter (reset by the last arriver)
  int32_t* ids;                      // [k]
  float* scores;                     // [k]
  int* err;                          // bit 0: an expert id was out of range
  uint16_t* shared_out;              // [H] T(shared down)
  int* step_slots;                   // cached CUs x resident workgroups of the gate/up launch (0: unknown)
};

}  // namespace

struct glm53_decode_plan {
  int64_t H, I, Is, E, k;
  float limit;
  // fixed scratch (one arena, allocated at creation)
  uint16_t* hidden = nullptr;  // [(k + 1) * max(I, Is)]
  float* sig = nullptr;        // [E] router logits
  unsigned long long* route_words = nullptr;  // [E] three-launch step's router words
  uint32_t* router_count = nullptr;           // arrival counter of the step's router launch
  int32_t* ids = nullptr;      // [k]
  float* scores = nullptr;     // [k]
  int* err = nullptr;
  // any-shape composition scratch
  uint16_t* gate = nullptr;    // [k, I]
  uint16_t* up = nullptr;      // [k, I]
  uint16_t* down = nullptr;    // [k, H]
  uint16_t* routed = nullptr;  // [H]
  uint16_t* shared_gate = nullptr;  // [Is]
  uint16_t* shared_up = nullptr;
  uint16_t* shared_out = nullptr;   // [H]
  uint16_t* moe_out = nullptr;      // [H] before a residual add
  void* arena = nullptr;
  size_t arena_bytes = 0;
  int gate_up_rows_per_wave = 8;   // launch shape (glm53_decode_plan_tune), swept on MI355X
  int down_rows_per_wg = 16;
  int step_slots = 0;              // CUs x resident workgroups of the routed gate/up launch
  // bound weights (glm53_decode_plan_bind)
  bool bound = false;
  glm53_bank bank{};
  glm53_shared_expert shared{};
  bool has_shared = false;
  glm53_router router{};
  bool has_router = false;
  // read-only counters (glm53_decode_plan_counters)
  uint64_t executions = 0;
  uint64_t static_validations = 0;
  uint64_t dynamic_validations = 0;
  uint64_t host_syncs = 0;

  StepContext step() {
    return {H, I, Is, E, k, limit, hidden, route_words, router_count, ids, scores, err, shared_out, &step_slots};
  }
};

int glm53_decode_plan_create(int64_t hidden, int64_t intermediate, int64_t shared_intermediate, int64_t experts,
                             int64_t top_k, float swiglu_limit, glm53_decode_plan** out) {
  CHECK_ARG(out != nullptr, "out is null");
  *out = nullptr;
  CHECK_ARG(hidden > 0 && intermediate > 0 && shared_intermediate >= 0, "invalid dimensions");
  CHECK_ARG(experts > 0 && experts <= kMaxExperts, "experts must be in [1, %d]", kMaxExperts);
  CHECK_ARG(top_k > 0 && top_k <= kMaxTopK && top_k <= experts, "top_k must be in [1, %d]", kMaxTopK);
  auto* p = new glm53_decode_plan();
  p->H = hidden;
  p->I = intermediate;
  p->Is = shared_intermediate;
  p->E = experts;
  p->k = top_k;
  p->limit = swiglu_limit;
  const int64_t Imax = std::max(intermediate, shared_intermediate);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += round_up(bytes);
    return o;
  };
  size_t o_hidden = take(2 * (top_k + 1) * Imax);
  size_t o_sig = take(4 * experts), o_words = take(8 * experts), o_ids = take(4 * top_k);
  size_t o_scores = take(4 * top_k), o_err = take(4);
  size_t o_gate = take(2 * top_k * intermediate), o_up = take(2 * top_k * intermediate);
  size_t o_down = take(2 * top_k * hidden), o_routed = take(2 * hidden);
  size_t o_sg = take(2 * std::max<int64_t>(shared_intermediate, 1)), o_su = take(2 * std::max<int64_t>(shared_intermediate, 1));
  size_t o_so = take(2 * hidden), o_mo = take(2 * hidden), o_rc = take(4);
  p->arena_bytes = off;
  hipError_t e = hipMalloc(&p->arena, off);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(e, "decode plan hipMalloc");
  }
  e = hipMemset(p->arena, 0, off);
  if (e != hipSuccess) {
    (void)hipFree(p->arena);
    delete p;
    return hip_fail(e, "decode plan hipMemset");
  }
  uint8_t* b = static_cast<uint8_t*>(p->arena);
  p->hidden = reinterpret_cast<uint16_t*>(b + o_hidden);
  p->sig = reinterpret_cast<float*>(b + o_sig);
  p->route_words = reinterpret_cast<unsigned long long*>(b + o_words);
  p->ids = reinterpret_cast<int32_t*>(b + o_ids);
  p->scores = reinterpret_cast<float*>(b + o_scores);
  p->err = reinterpret_cast<int*>(b + o_err);
  p->gate = reinterpret_cast<uint16_t*>(b + o_gate);
  p->up = reinterpret_cast<uint16_t*>(b + o_up);
  p->down = reinterpret_cast<uint16_t*>(b + o_down);
  p->routed = reinterpret_cast<uint16_t*>(b + o_routed);
  p->shared_gate = reinterpret_cast<uint16_t*>(b + o_sg);
  p->shared_up = reinterpret_cast<uint16_t*>(b + o_su);
  p->shared_out = reinterpret_cast<uint16_t*>(b + o_so);
  p->moe_out = reinterpret_cast<uint16_t*>(b + o_mo);
  p->router_count = reinterpret_cast<uint32_t*>(b + o_rc);
  *out = p;
  return GLM53_OK;
}

void glm53_decode_plan_destroy(glm53_decode_plan* plan) {
  if (plan == nullptr) return;
  if (plan->arena) (void)hipFree(plan->arena);
  delete plan;
}

namespace {


int check_decode_inputs(glm53_decode_plan* p, const glm53_bank* bank, const glm53_shared_expert* shared) {
  CHECK_ARG(p != nullptr, "plan is null");
  int rc = check_bank(bank, p->H, p->I, p->E);
  if (rc) return rc;
  if (shared != nullptr) {
    CHECK_ARG(p->Is > 0, "plan was created without a shared expert");
    if ((rc = check_linear(shared->gate, p->Is, p->H, "shared gate"))) return rc;
    if ((rc = check_linear(shared->up, p->Is, p->H, "shared up"))) return rc;
    if ((rc = check_linear(shared->down, p->H, p->Is, "shared down"))) return rc;
  }
  return GLM53_OK;
}

bool decode_fast_ok(int64_t H, int64_t I, int64_t Is, const glm53_bank* bank, const glm53_shared_expert* shared,
                    const void* x) {
  if (!fast_width_supported(H) || !fast_width_supported(I)) return false;
  if (H / 128 * 128 != H) return false;
  if (shared != nullptr && Is != I) return false;
  if (!aligned(x, 16) || !aligned(bank->gate_up_weight, 16) || !aligned(bank->down_weight, 16)) return false;
  if (shared != nullptr && (!aligned(shared->gate.weight, 16) || !aligned(shared->up.weight, 16) ||
                            !aligned(shared->down.weight, 16)))
    return false;
  return true;
}

int generic_linear(const void* x, int64_t x_group_stride, int64_t M, int64_t G, const uint8_t* w,
                   int64_t w_expert_stride, int64_t w_row_offset, const float* s, int64_t s_expert_stride,
                   int64_t s_row_offset, int64_t s_cols, const int32_t* ids, int64_t experts, int64_t N, int64_t K,
                   uint16_t* y, int64_t y_group_stride, int* err, hipStream_t st, int wg = 0) {
  CHECK_ARG(K <= 16384, "generic path supports K <= 16384");
  GenericLinearArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_row_stride = K;
  a.x_group_stride = x_group_stride;
  a.weight = w;
  a.w_expert_stride = w_expert_stride;
  a.w_row_offset = w_row_offset;
  a.w_group_log2 = wg;
  a.scale = s;
  a.s_expert_stride = s_expert_stride;
  a.s_row_offset = s_row_offset;
  a.s_cols = s_cols;
  a.expert_ids = ids;
  a.experts = experts;
  a.M = M;
  a.G = G;
  a.N = N;
  a.K = K;
  a.rows_per_wave = 4;
  a.tile_rows = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kGenericRows, 16384 / K)));
  a.y = y;
  a.y_row_stride = N;
  a.y_group_stride = y_group_stride;
  a.error_flag = err;
  HIP_TRY(launch_linear_generic(a, st), "generic linear launch");
  return GLM53_OK;
}

// stages: bit 1 = routed + shared gate/up/SwiGLU, bit 2 = down + reduction
// (+ shared, + residual).  The any-shape composition runs only whole.
// With topk_router the selection runs from the plan's router logits (fused
// into the gate/up launch on the fast path) and ids / scores are the plan's.
int run_decode(glm53_decode_plan* p, const glm53_bank* bank, const glm53_shared_expert* shared, const void* x,
               const int32_t* ids, const float* scores, const glm53_router* topk_router, const void* residual,
               void* out, int stages, hipStream_t st) {
  const int64_t H = p->H, I = p->I, Is = p->Is, k = p->k;
  if (topk_router != nullptr) {
    ids = p->ids;
    scores = p->scores;
  }
  if (decode_fast_ok(p->H, p->I, p->Is, bank, shared, x)) {
    GateUpArgs g{};
    g.x = static_cast<const uint16_t*>(x);
    g.expert_ids = ids;
    if (topk_router != nullptr) {
      g.router_logits = p->sig;
      g.router_bias = topk_router->bias;
      g.routed_scaling_factor = topk_router->routed_scaling_factor;
      g.norm_topk_prob = topk_router->norm_topk_prob;
      g.n_group = router_groups(topk_router);
      g.topk_group = router_topk_groups(topk_router);
      g.ids_out = p->ids;
      g.scores_out = p->scores;
    }
    g.top_k = static_cast<int>(k);
    g.experts = p->E;
    g.gate_up_weight = bank->gate_up_weight;
    g.gate_up_scale = bank->gate_up_scale_inv;
    g.bank_group_log2 = bank->row_group_log2;
    if (shared != nullptr) {
      g.shared_gate_weight = shared->gate.weight;
      g.shared_gate_scale = shared->gate.scale_inv;
      g.shared_up_weight = shared->up.weight;
      g.shared_up_scale = shared->up.scale_inv;
    }
    g.hidden = H;
    g.intermediate = I;
    g.shared_intermediate = shared != nullptr ? Is : 0;
    g.limit = p->limit;
    g.rows_per_wave = p->gate_up_rows_per_wave;
    g.wgs_per_slot = cdiv(I, 4 * g.rows_per_wave);
    g.hidden_out = p->hidden;
    g.error_flag = p->err;
    g.routed_flags = bank->code_flags;
    if (shared != nullptr) {
      g.shared_flags = shared->gate.code_flags;
      g.shared_flags2 = shared->up.code_flags;
    }
    if (stages & GLM53_STAGE_GATE_UP) HIP_TRY(launch_gate_up(g, st), "gate/up launch");
    DownArgs d{};
    d.hidden_in = p->hidden;
    d.expert_ids = ids;
    d.scores = scores;
    d.top_k = static_cast<int>(k);
    d.experts = p->E;
    d.down_weight = bank->down_weight;
    d.down_scale = bank->down_scale_inv;
    d.bank_group_log2 = bank->row_group_log2;
    if (shared != nullptr) {
      d.shared_down_weight = shared->down.weight;
      d.shared_down_scale = shared->down.scale_inv;
    }
    d.hidden = H;
    d.intermediate = I;
    d.rows_per_wg = p->down_rows_per_wg;
    d.residual = static_cast<const uint16_t*>(residual);
    d.routed_flags = bank->code_flags;
    if (shared != nullptr) d.shared_flags = shared->down.code_flags;
    d.out = static_cast<uint16_t*>(out);
    d.error_flag = p->err;
    if (stages & GLM53_STAGE_DOWN) HIP_TRY(launch_down(d, st), "down launch");
    return GLM53_OK;
  }
  CHECK_ARG((stages & (GLM53_STAGE_GATE_UP | GLM53_STAGE_DOWN)) == (GLM53_STAGE_GATE_UP | GLM53_STAGE_DOWN),
            "partial stages need the fused fast path (aligned pointers, supported widths)");
  if (topk_router != nullptr) {
    int rc0 = topk(p->sig, topk_router, 1, p->ids, p->scores, st);
    if (rc0) return rc0;
  }
  uint16_t* final_out = static_cast<uint16_t*>(out);
  if (residual != nullptr) out = p->moe_out;
  // Any-shape composition of the reference's separate stages
  // (packed.py:473-655): gate, up, SwiGLU, down, weighted reduction, shared.
  const int64_t SR = cdiv(I, 128), SC = cdiv(H, 128), SH = cdiv(H, 128), SI = cdiv(I, 128);
  int rc;
  const int bg = bank->row_group_log2;
  if ((rc = generic_linear(x, 0, 1, k, bank->gate_up_weight, 2 * I * H, 0, bank->gate_up_scale_inv, 2 * SR * SC, 0,
                           SC, ids, p->E, I, H, p->gate, I, p->err, st, bg)))
    return rc;
  if ((rc = generic_linear(x, 0, 1, k, bank->gate_up_weight, 2 * I * H, I, bank->gate_up_scale_inv, 2 * SR * SC, SR,
                           SC, ids, p->E, I, H, p->up, I, p->err, st, bg)))
    return rc;
  SwigluArgs sw{};
  sw.gate = p->gate;
  sw.up = p->up;
  sw.gate_row_stride = I;
  sw.up_row_stride = I;
  sw.rows = k;
  sw.cols = I;
  sw.limit = p->limit;
  sw.out = p->hidden;
  sw.out_row_stride = I;
  HIP_TRY(launch_swiglu(sw, st), "swiglu launch");
  if ((rc = generic_linear(p->hidden, I, 1, k, bank->down_weight, H * I, 0, bank->down_scale_inv, SH * SI, 0, SI, ids,
                           p->E, H, I, p->down, H, p->err, st, bg)))
    return rc;
  WeightedReductionArgs wr{};
  wr.down = p->down;
  wr.scores = scores;
  wr.top_k = static_cast<int>(k);
  wr.H = H;
  if (shared == nullptr) {
    wr.out = static_cast<uint16_t*>(out);
    HIP_TRY(launch_weighted_reduction(wr, st), "reduction launch");
    if (residual != nullptr)
      HIP_TRY(launch_add_bf16(static_cast<const uint16_t*>(residual), p->moe_out, final_out, H, st), "add launch");
    return GLM53_OK;
  }
  wr.out = p->routed;
  HIP_TRY(launch_weighted_reduction(wr, st), "reduction launch");
  const int64_t SIs = cdiv(Is, 128);
  if ((rc = generic_linear(x, 0, 1, 1, shared->gate.weight, 0, 0, shared->gate.scale_inv, 0, 0, SC, nullptr, 1, Is, H,
                           p->shared_gate, 0, p->err, st)))
    return rc;
  if ((rc = generic_linear(x, 0, 1, 1, shared->up.weight, 0, 0, shared->up.scale_inv, 0, 0, SC, nullptr, 1, Is, H,
                           p->shared_up, 0, p->err, st)))
    return rc;
  uint16_t* shared_hidden = p->hidden + k * std::max(I, Is);
  sw.gate = p->shared_gate;
  sw.up = p->shared_up;
  sw.gate_row_stride = Is;
  sw.up_row_stride = Is;
  sw.rows = 1;
  sw.cols = Is;
  sw.out = shared_hidden;
  sw.out_row_stride = Is;
  HIP_TRY(launch_swiglu(sw, st), "swiglu launch");
  if ((rc = generic_linear(shared_hidden, 0, 1, 1, shared->down.weight, 0, 0, shared->down.scale_inv, 0, 0, SIs,
                           nullptr, 1, H, Is, p->shared_out, 0, p->err, st)))
    return rc;
  HIP_TRY(launch_add_bf16(p->routed, p->shared_out, static_cast<uint16_t*>(out), H, st), "add launch");
  if (residual != nullptr)
    HIP_TRY(launch_add_bf16(static_cast<const uint16_t*>(residual), p->moe_out, final_out, H, st), "add launch");
  return GLM53_OK;
}

// The three-launch step (step.hip) when the shape is instantiated; returns
// -1 (nothing launched) otherwise.  router != NULL: launch 1 computes the
// logits and the selection into the context's ids / scores; else the
// routed launches read `ids` / `scores`, or the context's when those are
// NULL (the selection of an earlier router stage).
int run_step(const StepContext& c, const glm53_bank* bank, const glm53_shared_expert* shared,
             const glm53_router* router, const void* x, const int32_t* ids, const float* scores,
             const void* residual, void* out, int stages, int gate_up_rows_per_wave, hipStream_t st) {
  (void)gate_up_rows_per_wave;
  if (!decode_fast_ok(c.H, c.I, c.Is, bank, shared, x) || !step_shape_supported(c.H, c.I)) return -1;
  if (router != nullptr && (router->experts > 320 || !aligned(router->weight, 16))) return -1;
  if (!aligned(out, 4)) return -1;
  if (*c.step_slots == 0) {
    int dev = 0, cus = 0;
    HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
    const int occ = step_gate_up_occupancy(c.H, c.I);
    if (occ <= 0 || cus <= 0) return -1;
    *c.step_slots = cus * occ;
  }
  StepArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.residual = static_cast<const uint16_t*>(residual);
  a.out = static_cast<uint16_t*>(out);
  a.hidden = c.H;
  a.intermediate = c.I;
  a.experts = c.E;
  a.top_k = static_cast<int>(c.k);
  a.limit = c.limit;
  if (router != nullptr) {
    a.router_weight = router->weight;
    a.router_bias = router->bias;
    a.routed_scaling_factor = router->routed_scaling_factor;
    a.norm_topk_prob = router->norm_topk_prob;
    a.n_group = router_groups(router);
    a.topk_group = router_topk_groups(router);
    a.ids = c.ids;
    a.scores = c.scores;
    a.router_wgs = static_cast<int>(cdiv(c.E, 4));
  } else {
    a.ids = ids != nullptr ? const_cast<int32_t*>(ids) : c.ids;
    a.scores = scores != nullptr ? const_cast<float*>(scores) : c.scores;
  }
  a.route_words = c.route_words;
  a.router_count = c.router_count;
  a.gate_up_weight = bank->gate_up_weight;
  a.gate_up_scale = bank->gate_up_scale_inv;
  a.down_weight = bank->down_weight;
  a.down_scale = bank->down_scale_inv;
  a.bank_group_log2 = bank->row_group_log2;
  a.routed_flags = bank->code_flags;
  if (shared != nullptr) {
    a.shared_gate_weight = shared->gate.weight;
    a.shared_gate_scale = shared->gate.scale_inv;
    a.shared_up_weight = shared->up.weight;
    a.shared_up_scale = shared->up.scale_inv;
    a.shared_down_weight = shared->down.weight;
    a.shared_down_scale = shared->down.scale_inv;
    a.shared_gate_flags = shared->gate.code_flags;
    a.shared_up_flags = shared->up.code_flags;
    a.shared_down_flags = shared->down.code_flags;
  }
  a.hidden_act = c.hidden;
  a.shared_out = c.shared_out;
  a.error_flag = c.err;
  a.shared_rows_per_wave = 2;
  a.shared_delay = kStepSharedDelay;
  const int sd_wgs = shared != nullptr ? static_cast<int>(cdiv(c.H, 64)) : 0;
  a.routed_wgs = std::max(64, *c.step_slots - sd_wgs);
  HIP_TRY(launch_step(a, stages, st), "decode step launch");
  return GLM53_OK;
}

int run_router_decode(glm53_decode_plan* p, const glm53_router* r, const void* x, hipStream_t st) {
  RouterArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.weight = r->weight;
  a.experts = r->experts;
  a.hidden = r->hidden;
  a.logits_out = p->sig;  // the plan's [E] FP32 logits
  HIP_TRY(launch_router(a, st), "router launch");
  return GLM53_OK;
}

// Routed + shared decode with caller-chosen (ids, scores): the step kernels
// when the shape has them, else the any-shape composition.
int decode_routed_impl(glm53_decode_plan* p, const glm53_bank* bank, const glm53_shared_expert* shared,
                       const void* x, const int32_t* ids, const float* scores, void* out, hipStream_t st) {
  int rc = run_step(p->step(), bank, shared, nullptr, x, ids, scores, nullptr, out, GLM53_STAGE_ALL,
                    p->gate_up_rows_per_wave, st);
  if (rc < 0) rc = run_decode(p, bank, shared, x, ids, scores, nullptr, nullptr, out, GLM53_STAGE_ALL, st);
  if (rc == GLM53_OK) ++p->executions;
  return rc;
}

// Router + routed + shared decode; ids / scores land in the plan.
int decode_full_impl(glm53_decode_plan* p, const glm53_bank* bank, const glm53_shared_expert* shared,
                     const glm53_router* router, const void* x, void* out, hipStream_t st) {
  int rc = run_step(p->step(), bank, shared, router, x, nullptr, nullptr, nullptr, out, GLM53_STAGE_ALL,
                    p->gate_up_rows_per_wave, st);
  if (rc < 0) {
    if ((rc = run_router_decode(p, router, x, st))) return rc;
    rc = run_decode(p, bank, shared, x, p->ids, p->scores, router, nullptr, out, GLM53_STAGE_ALL, st);
  }
  if (rc == GLM53_OK) ++p->executions;
  return rc;
}

}  // namespace

int glm53_decode_moe_routed(glm53_decode_plan* plan, const glm53_bank* bank, const glm53_shared_expert* shared,
                            const void* x, const int32_t* expert_ids, const float* scores, void* out, void* stream) {
  int rc = check_decode_inputs(plan, bank, shared);
  if (rc) return rc;
  ++plan->static_validations;
  CHECK_ARG(x && expert_ids && scores && out, "null pointer argument");
  ++plan->dynamic_validations;
  return decode_routed_impl(plan, bank, shared, x, expert_ids, scores, out, S(stream));
}

int glm53_decode_moe(glm53_decode_plan* plan, const glm53_bank* bank, const glm53_shared_expert* shared,
                     const glm53_router* router, const void* x, void* out, int32_t* ids_out, float* scores_out,
                     void* stream) {
  int rc = check_decode_inputs(plan, bank, shared);
  if (rc) return rc;
  if ((rc = check_router(router, plan->H, plan->E, plan->k))) return rc;
  ++plan->static_validations;
  CHECK_ARG(x && out, "null pointer argument");
  ++plan->dynamic_validations;
  hipStream_t st = S(stream);
  if ((rc = decode_full_impl(plan, bank, shared, router, x, out, st))) return rc;
  if (ids_out) HIP_TRY(hipMemcpyAsync(ids_out, plan->ids, 4 * plan->k, hipMemcpyDeviceToDevice, st), "copy ids");
  if (scores_out)
    HIP_TRY(hipMemcpyAsync(scores_out, plan->scores, 4 * plan->k, hipMemcpyDeviceToDevice, st), "copy scores");
  return GLM53_OK;
}

int glm53_decode_plan_bind(glm53_decode_plan* plan, const glm53_bank* bank, const glm53_shared_expert* shared,
                           const glm53_router* router) {
  CHECK_ARG(plan != nullptr, "plan is null");
  if (plan->bound) return fail(GLM53_BAD_STATE, "decode plan weights are already bound");
  int rc = check_decode_inputs(plan, bank, shared);
  if (rc) return rc;
  if (router != nullptr && (rc = check_router(router, plan->H, plan->E, plan->k))) return rc;
  ++plan->static_validations;
  plan->bank = *bank;
  plan->has_shared = shared != nullptr;
  if (shared) plan->shared = *shared;
  plan->has_router = router != nullptr;
  if (router) plan->router = *router;
  plan->bound = true;
  return GLM53_OK;
}

int glm53_decode_moe_bound(glm53_decode_plan* plan, const void* x, void* out, void* stream) {
  CHECK_ARG(plan != nullptr, "plan is null");
  if (!plan->bound) return fail(GLM53_BAD_STATE, "decode plan has no bound weights");
  if (!plan->has_router) return fail(GLM53_BAD_STATE, "decode plan was bound without a router");
  CHECK_ARG(x && out, "null pointer argument");
  ++plan->dynamic_validations;
  return decode_full_impl(plan, &plan->bank, plan->has_shared ? &plan->shared : nullptr, &plan->router, x, out,
                          S(stream));
}

int glm53_decode_moe_bound_routed(glm53_decode_plan* plan, const void* x, const int32_t* expert_ids,
                                  const float* scores, void* out, void* stream) {
  CHECK_ARG(plan != nullptr, "plan is null");
  if (!plan->bound) return fail(GLM53_BAD_STATE, "decode plan has no bound weights");
  CHECK_ARG(x && expert_ids && scores && out, "null pointer argument");
  ++plan->dynamic_validations;
  return decode_routed_impl(plan, &plan->bank, plan->has_shared ? &plan->shared : nullptr, x, expert_ids, scores,
                            out, S(stream));
}

int glm53_decode_moe_ex(glm53_decode_plan* plan, const glm53_bank* bank, const glm53_shared_expert* shared,
                        const glm53_router* router, const void* x, const void* residual, void* out, int32_t stages,
                        void* stream) {
  int rc = check_decode_inputs(plan, bank, shared);
  if (rc) return rc;
  CHECK_ARG(x && out, "null pointer argument");
  CHECK_ARG(stages > 0 && (stages & ~GLM53_STAGE_ALL) == 0, "invalid stage mask %d", stages);
  if (stages & GLM53_STAGE_ROUTER) {
    if ((rc = check_router(router, plan->H, plan->E, plan->k))) return rc;
  }
  ++plan->static_validations;
  ++plan->dynamic_validations;
  hipStream_t st = S(stream);
  // Without the router stage the routed launches read the selection the
  // plan holds (written by an earlier call's router stage).
  const glm53_router* stage_router = (stages & GLM53_STAGE_ROUTER) ? router : nullptr;
  rc = run_step(plan->step(), bank, shared, stage_router, x, nullptr, nullptr, residual, out, stages,
                plan->gate_up_rows_per_wave, st);
  if (rc < 0) {
    CHECK_ARG(stages == GLM53_STAGE_ALL && router != nullptr,
              "partial stage masks need the fused step shapes (aligned pointers, instantiated widths)");
    if ((rc = check_router(router, plan->H, plan->E, plan->k))) return rc;
    if ((rc = run_router_decode(plan, router, x, st))) return rc;
    rc = run_decode(plan, bank, shared, x, plan->ids, plan->scores, router, residual, out, GLM53_STAGE_ALL, st);
  }
  if (rc == GLM53_OK) ++plan->executions;
  return rc;
}

int glm53_decode_plan_tune(glm53_decode_plan* plan, int32_t gate_up_rows_per_wave, int32_t down_rows_per_wg) {
  CHECK_ARG(plan != nullptr, "plan is null");
  CHECK_ARG(gate_up_rows_per_wave >= 1 && gate_up_rows_per_wave <= 64, "gate_up_rows_per_wave must be in [1, 64]");
  CHECK_ARG(down_rows_per_wg >= 1 && down_rows_per_wg <= kMaxDownRowsPerWg, "down_rows_per_wg must be in [1, %d]",
            kMaxDownRowsPerWg);
  plan->gate_up_rows_per_wave = gate_up_rows_per_wave;
  plan->down_rows_per_wg = down_rows_per_wg;
  return GLM53_OK;
}

int glm53_decode_plan_scratch(glm53_decode_plan* plan, int32_t which, void** ptr, size_t* bytes) {
  CHECK_ARG(plan && ptr && bytes, "null pointer argument");
  switch (which) {
    case 0:
      *ptr = plan->hidden;
      *bytes = 2 * (plan->k + 1) * std::max(plan->I, plan->Is);
      return GLM53_OK;
    case 1:
      *ptr = plan->ids;
      *bytes = 4 * plan->k;
      return GLM53_OK;
    case 2:
      *ptr = plan->scores;
      *bytes = 4 * plan->k;
      return GLM53_OK;
    case 3:
      *ptr = plan->route_words;
      *bytes = 8 * plan->E;
      return GLM53_OK;
    case 4:
      *ptr = plan->arena;
      *bytes = plan->arena_bytes;
      return GLM53_OK;
    case 5:
      *ptr = plan->shared_out;
      *bytes = 2 * plan->H;
      return GLM53_OK;
    default:
      return fail(GLM53_INVALID_ARGUMENT, "unknown scratch id %d", which);
  }
}

int glm53_decode_plan_error_flag(glm53_decode_plan* plan, int32_t* host_value) {
  CHECK_ARG(plan && host_value, "null pointer argument");
  HIP_TRY(hipMemcpy(host_value, plan->err, sizeof(int32_t), hipMemcpyDeviceToHost), "read error flag");
  HIP_TRY(hipMemset(plan->err, 0, sizeof(int32_t)), "clear error flag");
  ++plan->host_syncs;
  return GLM53_OK;
}

int glm53_decode_plan_counters(const glm53_decode_plan* plan, glm53_plan_counters* out) {
  CHECK_ARG(plan && out, "null pointer argument");
  *out = glm53_plan_counters{};
  out->execution_count = plan->executions;
  out->dynamic_allocation_count = 0;
  out->host_synchronization_count = plan->host_syncs;
  out->static_input_validation_count = plan->static_validations;
  out->dynamic_input_validation_count = plan->dynamic_validations;
  out->scratch_bytes = plan->arena_bytes;
  out->weights_bound = plan->bound ? 1 : 0;
  out->router_bound = plan->has_router ? 1 : 0;
  return GLM53_OK;
}

int glm53_decode_plan_identities(const glm53_decode_plan* plan, int32_t which, uint64_t* out, int32_t capacity,
                                 int32_t* count) {
  CHECK_ARG(plan && count && (capacity == 0 || out), "null pointer argument");
  uint64_t ids[16];
  int n = 0;
  auto put = [&](const void* q) { ids[n++] = reinterpret_cast<uint64_t>(q); };
  if (which == 0) {
    for (const void* q : {static_cast<const void*>(plan->hidden), static_cast<const void*>(plan->sig),
                          static_cast<const void*>(plan->route_words), static_cast<const void*>(plan->ids),
                          static_cast<const void*>(plan->scores), static_cast<const void*>(plan->err),
                          static_cast<const void*>(plan->shared_out), static_cast<const void*>(plan->router_count)})
      put(q);
  } else if (which == 1) {
    if (!plan->bound) return fail(GLM53_BAD_STATE, "decode plan has no bound weights");
    put(plan->bank.gate_up_weight);
    put(plan->bank.gate_up_scale_inv);
    put(plan->bank.down_weight);
    put(plan->bank.down_scale_inv);
    if (plan->has_shared) {
      for (const glm53_linear* l : {&plan->shared.gate, &plan->shared.up, &plan->shared.down}) {
        put(l->weight);
        put(l->scale_inv);
      }
    }
    if (plan->has_router) {
      put(plan->router.weight);
      put(plan->router.bias);
    }
  } else {
    return fail(GLM53_INVALID_ARGUMENT, "unknown identity set %d", which);
  }
  *count = n;
  for (int i = 0; i < n && i < capacity; ++i) out[i] = ids[i];
  return GLM53_OK;
}


// ------------------------------------------------- routed diagnostic ------

struct glm53_routed_diagnostic {
  int64_t H, I, E, k;
  float limit;
  void* arena = nullptr;
  size_t arena_bytes = 0;
  uint16_t* stage[5] = {};  // gate, up, sigmoid, silu, hidden: bf16 [k, I] each
  int* err = nullptr;
  uint64_t executions = 0;
};

int glm53_routed_diagnostic_create(int64_t hidden, int64_t intermediate, int64_t experts, int64_t top_k,
                                   float swiglu_limit, glm53_routed_diagnostic** out) {
  CHECK_ARG(out != nullptr, "out is null");
  *out = nullptr;
  CHECK_ARG(hidden > 0 && hidden <= 16384 && intermediate > 0 && intermediate <= 16384,
            "invalid dimensions (the diagnostic runs the any-shape GEMV: widths up to 16384)");
  CHECK_ARG(experts > 0 && experts <= kMaxExperts && top_k > 0 && top_k <= kMaxTopK && top_k <= experts,
            "invalid expert count or top_k");
  auto* d = new glm53_routed_diagnostic();
  d->H = hidden;
  d->I = intermediate;
  d->E = experts;
  d->k = top_k;
  d->limit = swiglu_limit;
  const size_t plane = round_up(2 * static_cast<size_t>(top_k * intermediate));
  d->arena_bytes = 5 * plane + 256;
  hipError_t e = hipMalloc(&d->arena, d->arena_bytes);
  if (e == hipSuccess) e = hipMemset(d->arena, 0, d->arena_bytes);
  if (e != hipSuccess) {
    if (d->arena) (void)hipFree(d->arena);
    delete d;
    return hip_fail(e, "routed diagnostic allocation");
  }
  uint8_t* b = static_cast<uint8_t*>(d->arena);
  for (int i = 0; i < 5; ++i) d->stage[i] = reinterpret_cast<uint16_t*>(b + i * plane);
  d->err = reinterpret_cast<int*>(b + 5 * plane);
  *out = d;
  return GLM53_OK;
}

void glm53_routed_diagnostic_destroy(glm53_routed_diagnostic* diag) {
  if (diag == nullptr) return;
  if (diag->arena) (void)hipFree(diag->arena);
  delete diag;
}

int glm53_routed_diagnostic_execute(glm53_routed_diagnostic* d, const void* x, const int32_t* expert_ids,
                                    const uint8_t* gate_up_weight, const float* gate_up_scale_inv,
                                    int32_t row_group_log2, void* stream) {
  CHECK_ARG(d != nullptr, "diagnostic is null");
  CHECK_ARG(x && expert_ids && gate_up_weight && gate_up_scale_inv, "null pointer argument");
  const int64_t H = d->H, I = d->I, k = d->k;
  CHECK_ARG(row_group_log2 >= 0 && row_group_log2 <= GLM53_MAX_ROW_GROUP_LOG2 &&
                (row_group_log2 == 0 || (H % 128 == 0 && I % 128 == 0)),
            "invalid row_group_log2 %d for H=%lld, I=%lld", (int)row_group_log2, (long long)H, (long long)I);
  hipStream_t st = S(stream);
  const int64_t SR = cdiv(I, 128), SC = cdiv(H, 128);
  int rc;
  if ((rc = generic_linear(x, 0, 1, k, gate_up_weight, 2 * I * H, 0, gate_up_scale_inv, 2 * SR * SC, 0, SC,
                           expert_ids, d->E, I, H, d->stage[0], I, d->err, st, row_group_log2)))
    return rc;
  if ((rc = generic_linear(x, 0, 1, k, gate_up_weight, 2 * I * H, I, gate_up_scale_inv, 2 * SR * SC, SR, SC,
                           expert_ids, d->E, I, H, d->stage[1], I, d->err, st, row_group_log2)))
    return rc;
  SwigluArgs a{};
  a.gate = d->stage[0];
  a.up = d->stage[1];
  a.gate_row_stride = I;
  a.up_row_stride = I;
  a.rows = k;
  a.cols = I;
  a.limit = d->limit;
  a.out = d->stage[4];
  a.out_row_stride = I;
  HIP_TRY(launch_swiglu_stages(a, d->stage[2], d->stage[3], st), "swiglu stages launch");
  ++d->executions;
  return GLM53_OK;
}

int glm53_routed_diagnostic_stage(glm53_routed_diagnostic* d, int32_t which, void** ptr, size_t* bytes) {
  CHECK_ARG(d && ptr && bytes, "null pointer argument");
  CHECK_ARG(which >= 0 && which < 5, "unknown stage %d", which);
  *ptr = d->stage[which];
  *bytes = 2 * static_cast<size_t>(d->k * d->I);
  return GLM53_OK;
}

int glm53_routed_diagnostic_counters(const glm53_routed_diagnostic* d, uint64_t* execution_count,
                                     uint64_t* scratch_bytes) {
  CHECK_ARG(d && execution_count && scratch_bytes, "null pointer argument");
  *execution_count = d->executions;
  *scratch_bytes = d->arena_bytes;
  return GLM53_OK;
}

// ---------------------------------------------------- prefill pieces ------

size_t glm53_route_plan_workspace_bytes(int64_t routes, int64_t experts) {
  const int64_t blocks = std::max<int64_t>(cdiv(routes, 256), 1);
  return round_up(sizeof(unsigned) * blocks * experts) + round_up(sizeof(unsigned) * blocks);
}

namespace {

int route_plan_impl(const int32_t* expert_ids, const float* scores, int64_t routes, int64_t top_k, int64_t experts,
                    int64_t tile_rows, int32_t* sorted_route, int32_t* inverse, int32_t* sorted_expert,
                    int32_t* sorted_token, float* sorted_score, uint32_t* route_offsets, uint32_t* tile_offsets,
                    int32_t* tile_expert, int32_t* tile_start, int32_t* tile_len, int64_t capacity, uint32_t* status,
                    void* workspace, hipStream_t st) {
  RoutePlanArgs a{};
  a.expert_ids = expert_ids;
  a.scores = scores;
  a.routes = routes;
  a.top_k = static_cast<int>(top_k);
  a.experts = static_cast<int>(experts);
  a.tile_rows = static_cast<int>(tile_rows);
  a.blocks = cdiv(routes, 256);
  a.capacity = capacity;
  a.block_counts = static_cast<unsigned*>(workspace);
  a.block_invalid = reinterpret_cast<unsigned*>(static_cast<uint8_t*>(workspace) +
                                                round_up(sizeof(unsigned) * std::max<int64_t>(a.blocks, 1) * experts));
  a.sorted_route = sorted_route;
  a.inverse = inverse;
  a.sorted_expert = sorted_expert;
  a.sorted_token = sorted_token;
  a.sorted_score = sorted_score;
  a.route_offsets = route_offsets;
  a.tile_offsets = tile_offsets;
  a.tile_expert = tile_expert;
  a.tile_start = tile_start;
  a.tile_len = tile_len;
  a.status = status;
  HIP_TRY(launch_route_plan(a, st), "route plan launch");
  return GLM53_OK;
}

}  // namespace

int glm53_route_plan(const int32_t* expert_ids, const float* scores, int64_t routes, int64_t top_k, int64_t experts,
                     int64_t tile_rows, int32_t* sorted_route, int32_t* inverse, int32_t* sorted_expert,
                     int32_t* sorted_token, float* sorted_score, uint32_t* route_offsets, uint32_t* tile_offsets,
                     int32_t* tile_expert, int32_t* tile_start, int32_t* tile_len, int64_t capacity, uint32_t* status,
                     void* workspace, size_t workspace_bytes, void* stream) {
  CHECK_ARG(routes >= 0 && top_k > 0 && experts > 0 && experts <= kPlanMaxExperts && tile_rows > 0,
            "invalid route plan dimensions");
  CHECK_ARG(routes < (int64_t(1) << 31), "too many routes");
  CHECK_ARG(capacity >= cdiv(routes, tile_rows) + experts, "descriptor capacity %lld < ceil(routes/tile)+experts",
            (long long)capacity);
  CHECK_ARG(workspace && workspace_bytes >= glm53_route_plan_workspace_bytes(routes, experts),
            "route plan workspace too small");
  CHECK_ARG(sorted_route && inverse && sorted_expert && sorted_token && route_offsets && tile_offsets && tile_expert &&
                tile_start && tile_len && status && (routes == 0 || expert_ids),
            "null pointer argument");
  CHECK_ARG(scores == nullptr || sorted_score != nullptr, "sorted_score is null");
  return route_plan_impl(expert_ids, scores, routes, top_k, experts, tile_rows, sorted_route, inverse, sorted_expert,
                         sorted_token, sorted_score, route_offsets, tile_offsets, tile_expert, tile_start, tile_len,
                         capacity, status, workspace, S(stream));
}

int glm53_split_activations(const void* x, int64_t rows, int64_t cols, int64_t x_row_stride, uint8_t* hi, uint8_t* lo,
                            float* scale, void* stream) {
  CHECK_ARG(rows >= 0 && cols > 0 && cols % 128 == 0 && x_row_stride >= cols,
            "split needs cols a positive multiple of 128 and x_row_stride >= cols; got cols=%lld, stride=%lld",
            (long long)cols, (long long)x_row_stride);
  if (rows == 0) return GLM53_OK;
  CHECK_ARG(x && hi && lo && scale, "null pointer argument");
  CHECK_ARG(aligned(x, 2) && aligned(hi, 8) && aligned(lo, 8) && aligned(scale, 4),
            "x must be 2-byte, hi and lo 8-byte, scale 4-byte aligned");
  SplitArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_row_stride = x_row_stride;
  a.rows = rows;
  a.cols = cols;
  a.hi = hi;
  a.lo = lo;
  a.scale = scale;
  HIP_TRY(launch_split_activations(a, S(stream)), "split launch");
  return GLM53_OK;
}

size_t glm53_grouped_linear_workspace_bytes(int64_t act_rows, int64_t K) {
  if (K % 128 != 0) return 0;
  return split_bytes(act_rows, K) + 256;
}

int glm53_grouped_linear(const void* x, int64_t act_rows, const int32_t* row_index, int64_t routes, int64_t K,
                         const int32_t* tile_expert, const int32_t* tile_start, const int32_t* tile_len,
                         int64_t descriptors, const uint8_t* weight, const float* scale_inv,
                         const int32_t* code_flags, int64_t experts, int64_t N, void* y, void* workspace,
                         size_t workspace_bytes, void* stream) {
  CHECK_ARG(K > 0 && K % 128 == 0 && N > 0 && N % 16 == 0,
            "grouped path requires block-aligned projection dimensions; got out=%lld, in=%lld", (long long)N,
            (long long)K);
  CHECK_ARG(routes >= 0 && act_rows >= 0 && descriptors >= 0 && experts > 0, "invalid dimensions");
  if (routes == 0) return GLM53_OK;
  CHECK_ARG(x && weight && scale_inv && y && tile_expert && tile_start && tile_len, "null pointer argument");
  CHECK_ARG(aligned(weight, 16), "weight must be 16-byte aligned");
  CHECK_ARG(workspace && workspace_bytes >= glm53_grouped_linear_workspace_bytes(act_rows, K),
            "grouped linear workspace too small");
  hipStream_t st = S(stream);
  SplitBuf b = carve_split(workspace, act_rows, K);
  if (code_flags == nullptr) {
    int32_t* flag = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + split_bytes(act_rows, K));
    HIP_TRY(launch_scan_480(weight, experts * N * K, flag, true, st), "scan launch");
    code_flags = flag;
  }
  HIP_TRY(split(x, act_rows, K, b, st), "split launch");
  GroupedGemmArgs g{};
  g.fixup = code_flags;
  g.a_hi = b.hi;
  g.a_lo = b.lo;
  g.a_scale = b.scale;
  g.a_row_index = row_index;
  g.K = K;
  g.routes = routes;
  g.tile_expert = tile_expert;
  g.tile_start = tile_start;
  g.tile_len = tile_len;
  g.experts = experts;
  g.weight = weight;
  g.w_expert_stride = N * K;
  g.scale = scale_inv;
  g.s_expert_stride = cdiv(N, 128) * (K / 128);
  g.s_cols = K / 128;
  g.N = N;
  g.out = static_cast<uint16_t*>(y);
  g.out_row_stride = N;
  HIP_TRY(launch_grouped_gemm(g, GEMM_PLAIN, descriptors, st), "grouped gemm launch");
  return GLM53_OK;
}

int glm53_activate_gate_up(const void* gate_up, int64_t rows, int64_t intermediate, float limit, void* out,
                           void* stream) {
  CHECK_ARG(rows >= 0 && intermediate > 0, "invalid dimensions");
  if (rows == 0) return GLM53_OK;
  CHECK_ARG(gate_up && out, "null pointer argument");
  SwigluArgs a{};
  a.gate = static_cast<const uint16_t*>(gate_up);
  a.up = static_cast<const uint16_t*>(gate_up) + intermediate;
  a.gate_row_stride = 2 * intermediate;
  a.up_row_stride = 2 * intermediate;
  a.rows = rows;
  a.cols = intermediate;
  a.limit = limit;
  a.out = static_cast<uint16_t*>(out);
  a.out_row_stride = intermediate;
  HIP_TRY(launch_swiglu(a, S(stream)), "swiglu launch");
  return GLM53_OK;
}

int glm53_restore_and_reduce(const void* sorted_out, const float* sorted_score, const int32_t* inverse, int64_t tokens,
                             int64_t top_k, int64_t H, const void* shared, void* out, void* stream) {
  CHECK_ARG(tokens >= 0 && top_k > 0 && top_k <= kMaxReduceTopK && H > 0, "invalid dimensions");
  if (tokens == 0) return GLM53_OK;
  CHECK_ARG(sorted_out && sorted_score && inverse && out, "null pointer argument");
  ReduceArgs a{};
  a.route_out = static_cast<const uint16_t*>(sorted_out);
  a.inverse = inverse;
  a.sorted_score = sorted_score;
  a.shared = static_cast<const uint16_t*>(shared);
  a.tokens = tokens;
  a.H = H;
  a.top_k = static_cast<int>(top_k);
  a.out = static_cast<uint16_t*>(out);
  HIP_TRY(launch_reduce(a, false, S(stream)), "reduce launch");
  return GLM53_OK;
}

int glm53_direct_order_reduce(const void* sorted_out, const int32_t* inverse, const int32_t* expert_ids,
                              const float* scores, int64_t tokens, int64_t top_k, int64_t H, const void* shared,
                              void* out, void* stream) {
  CHECK_ARG(tokens >= 0 && top_k > 0 && top_k <= kMaxReduceTopK && H > 0, "invalid dimensions");
  if (tokens == 0) return GLM53_OK;
  CHECK_ARG(sorted_out && inverse && expert_ids && scores && out, "null pointer argument");
  ReduceArgs a{};
  a.route_out = static_cast<const uint16_t*>(sorted_out);
  a.inverse = inverse;
  a.route_score = scores;
  a.expert_ids = expert_ids;
  a.shared = static_cast<const uint16_t*>(shared);
  a.tokens = tokens;
  a.H = H;
  a.top_k = static_cast<int>(top_k);
  a.out = static_cast<uint16_t*>(out);
  HIP_TRY(launch_reduce(a, true, S(stream)), "reduce launch");
  return GLM53_OK;
}

// ------------------------------------------------------- prefill plan ------

struct glm53_prefill_plan {
  int64_t H, I, Is, E, k, max_tokens;
  float limit;
  int64_t capacity_max;
  void* arena = nullptr;
  // router
  float* router_partial = nullptr;  // [kMaxRouterSplits, T, E] router partial sums
  float* logits = nullptr;
  int32_t* ids = nullptr;
  float* scores = nullptr;
  // activations
  SplitBuf xq{};
  SplitBuf hq{};
  SplitBuf sq{};
  // route plan
  void* plan_ws = nullptr;
  int32_t *sorted_route = nullptr, *inverse = nullptr, *sorted_expert = nullptr, *sorted_token = nullptr;
  float* sorted_score = nullptr;
  uint32_t *route_offsets = nullptr, *tile_offsets = nullptr, *status = nullptr;
  int32_t *tile_expert = nullptr, *tile_start = nullptr, *tile_len = nullptr;
  // intermediates
  uint16_t* h = nullptr;         // [R, I]
  uint16_t* down = nullptr;      // [R, H]
  uint16_t* hs = nullptr;        // [T, Is]
  uint16_t* shared_out = nullptr;  // [T, H]
  int32_t* flags = nullptr;        // [4] code flags scanned when the caller has none: bank gate/up, bank
                                   // down, shared gate + up, shared down
  int64_t last_tokens = 0;
  size_t arena_bytes = 0;
  // read-only counters (glm53_prefill_plan_counters)
  uint64_t executions = 0;
  uint64_t static_validations = 0;
  uint64_t dynamic_validations = 0;
  uint64_t host_syncs = 0;
};

int glm53_prefill_plan_create(int64_t hidden, int64_t intermediate, int64_t shared_intermediate, int64_t experts,
                              int64_t top_k, int64_t max_tokens, float swiglu_limit, glm53_prefill_plan** out) {
  CHECK_ARG(out != nullptr, "out is null");
  *out = nullptr;
  CHECK_ARG(hidden > 0 && hidden % 128 == 0 && intermediate > 0 && intermediate % 128 == 0,
            "grouped path requires block-aligned projection dimensions; got hidden=%lld, intermediate=%lld",
            (long long)hidden, (long long)intermediate);
  CHECK_ARG(shared_intermediate >= 0 && shared_intermediate % 128 == 0, "shared intermediate must be a multiple of 128");
  CHECK_ARG(experts > 0 && experts <= kPlanMaxExperts, "experts must be in [1, %d]", kPlanMaxExperts);
  CHECK_ARG(top_k > 0 && top_k <= kMaxTopK && top_k <= experts, "top_k must be in [1, %d]", kMaxTopK);
  CHECK_ARG(max_tokens > 0 && max_tokens * top_k < (int64_t(1) << 31), "invalid max_tokens");
  auto* p = new glm53_prefill_plan();
  p->H = hidden;
  p->I = intermediate;
  p->Is = shared_intermediate;
  p->E = experts;
  p->k = top_k;
  p->max_tokens = max_tokens;
  p->limit = swiglu_limit;
  const int64_t T = max_tokens, R = T * top_k;
  // the separate shared hidden rows (hs) and their split (sq) serve only a
  // shared expert of another width than the routed one: one of the routed
  // width runs merged into the routed buffers (below)
  const bool separate_shared = shared_intermediate > 0 && shared_intermediate != intermediate;
  const int64_t Ism = separate_shared ? shared_intermediate : 0;
  p->capacity_max = cdiv(R, kGemmMinTileRows) + experts;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += round_up(bytes);
    return o;
  };
  size_t o_xf = take(router_space_bytes(T, experts)), o_logits = take(4 * T * experts), o_ids = take(4 * R),
         o_scores = take(4 * R);
  // a shared expert of the routed width keeps its hidden rows right after
  // the routed ones (h and hq), so that one split launch covers both
  const int64_t RH = shared_intermediate == intermediate ? R + T : R;
  size_t o_xq = take(split_bytes(T, hidden)), o_hq = take(split_bytes(RH, intermediate));
  size_t o_sq = take(separate_shared ? split_bytes(T, Ism) : 0);
  size_t o_pws = take(glm53_route_plan_workspace_bytes(R, experts));
  size_t o_sr = take(4 * R), o_inv = take(4 * R), o_se = take(4 * R), o_st = take(4 * R), o_ss = take(4 * R);
  size_t o_ro = take(4 * (experts + 1)), o_to = take(4 * (experts + 1)), o_status = take(8);
  // the descriptor arrays back to back: int32 [3, capacity_max]
  const size_t o_te = take(4 * 3 * p->capacity_max), o_ts = o_te + 4 * p->capacity_max,
               o_tl = o_ts + 4 * p->capacity_max;
  size_t o_h = take(2 * RH * intermediate), o_down = take(2 * R * hidden), o_hs = take(2 * T * Ism);
  size_t o_so = take(2 * T * hidden), o_flags = take(32);
  p->arena_bytes = off;
  hipError_t e = hipMalloc(&p->arena, off);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(e, "prefill plan hipMalloc");
  }
  e = hipMemset(p->arena, 0, off);
  if (e != hipSuccess) {
    (void)hipFree(p->arena);
    delete p;
    return hip_fail(e, "prefill plan hipMemset");
  }
  uint8_t* b = static_cast<uint8_t*>(p->arena);
  p->router_partial = reinterpret_cast<float*>(b + o_xf);
  p->logits = reinterpret_cast<float*>(b + o_logits);
  p->ids = reinterpret_cast<int32_t*>(b + o_ids);
  p->scores = reinterpret_cast<float*>(b + o_scores);
  p->xq = carve_split(b + o_xq, T, hidden);
  p->hq = carve_split(b + o_hq, RH, intermediate);
  p->sq = separate_shared ? carve_split(b + o_sq, T, Ism) : SplitBuf{nullptr, nullptr, nullptr};
  p->plan_ws = b + o_pws;
  p->sorted_route = reinterpret_cast<int32_t*>(b + o_sr);
  p->inverse = reinterpret_cast<int32_t*>(b + o_inv);
  p->sorted_expert = reinterpret_cast<int32_t*>(b + o_se);
  p->sorted_token = reinterpret_cast<int32_t*>(b + o_st);
  p->sorted_score = reinterpret_cast<float*>(b + o_ss);
  p->route_offsets = reinterpret_cast<uint32_t*>(b + o_ro);
  p->tile_offsets = reinterpret_cast<uint32_t*>(b + o_to);
  p->status = reinterpret_cast<uint32_t*>(b + o_status);
  p->tile_expert = reinterpret_cast<int32_t*>(b + o_te);
  p->tile_start = reinterpret_cast<int32_t*>(b + o_ts);
  p->tile_len = reinterpret_cast<int32_t*>(b + o_tl);
  p->h = reinterpret_cast<uint16_t*>(b + o_h);
  p->down = reinterpret_cast<uint16_t*>(b + o_down);
  p->hs = separate_shared ? reinterpret_cast<uint16_t*>(b + o_hs) : nullptr;
  p->shared_out = reinterpret_cast<uint16_t*>(b + o_so);
  p->flags = reinterpret_cast<int32_t*>(b + o_flags);
  *out = p;
  return GLM53_OK;
}

void glm53_prefill_plan_destroy(glm53_prefill_plan* plan) {
  if (plan == nullptr) return;
  if (plan->arena) (void)hipFree(plan->arena);
  delete plan;
}

// The prefill body; out = the BF16 MoE output, or (hc_out set) the
// hyper-connection streams built from it in the reduction's epilogue.
static int prefill_run(glm53_prefill_plan* p, const glm53_bank* bank, const glm53_shared_expert* shared,
                       const glm53_router* router, const void* x, int64_t tokens, const int32_t* expert_ids,
                       const float* scores, int32_t reduction, void* out, const void* hc_residual, const float* hc_post,
                       const float* hc_comb, void* hc_out, void* stream) {
  CHECK_ARG(p != nullptr, "plan is null");
  CHECK_ARG(tokens >= 0 && tokens <= p->max_tokens, "tokens %lld outside [0, %lld]", (long long)tokens,
            (long long)p->max_tokens);
  CHECK_ARG(reduction == GLM53_REDUCE_GROUPED || reduction == GLM53_REDUCE_DIRECT, "unknown reduction %d", reduction);
  int rc = check_bank(bank, p->H, p->I, p->E);
  if (rc) return rc;
  if (shared != nullptr) {
    CHECK_ARG(p->Is > 0, "plan was created without a shared expert");
    if ((rc = check_linear(shared->gate, p->Is, p->H, "shared gate"))) return rc;
    if ((rc = check_linear(shared->up, p->Is, p->H, "shared up"))) return rc;
    if ((rc = check_linear(shared->down, p->H, p->Is, "shared down"))) return rc;
    CHECK_ARG(aligned(shared->gate.weight, 16) && aligned(shared->up.weight, 16) && aligned(shared->down.weight, 16),
              "shared weights must be 16-byte aligned");
  }
  CHECK_ARG(aligned(bank->gate_up_weight, 16) && aligned(bank->down_weight, 16), "bank weights must be 16-byte aligned");
  if (expert_ids == nullptr) {
    if ((rc = check_router(router, p->H, p->E, p->k))) return rc;
  } else {
    CHECK_ARG(scores != nullptr, "scores are required with expert_ids");
  }
  ++p->static_validations;
  p->last_tokens = tokens;
  if (tokens == 0) return GLM53_OK;
  CHECK_ARG(x && (out || hc_out), "null pointer argument");
  ++p->dynamic_validations;
  hipStream_t st = S(stream);
  const int64_t T = tokens, k = p->k, R = T * k, H = p->H, I = p->I, Is = p->Is, E = p->E;
  const int64_t SC = H / 128, SR = I / 128, SI = I / 128;
  const int32_t* ids = expert_ids;
  const float* sc = scores;
  if (ids == nullptr) {
    if ((rc = route_tokens(router, x, T, p->router_partial, p->logits, p->ids, p->scores, st))) return rc;
    ids = p->ids;
    sc = p->scores;
  } else {
    HIP_TRY(hipMemcpyAsync(p->ids, expert_ids, 4 * R, hipMemcpyDeviceToDevice, st), "copy ids");
    HIP_TRY(hipMemcpyAsync(p->scores, scores, 4 * R, hipMemcpyDeviceToDevice, st), "copy scores");
  }
  // 0. 0x7F/0xFF code flags of every weight the MFMA reads (scan when absent)
  const int32_t* bank_flag = bank->code_flags;
  if (bank_flag == nullptr) {
    HIP_TRY(launch_scan_480(bank->gate_up_weight, E * 2 * I * H, p->flags, true, st), "scan bank");
    HIP_TRY(launch_scan_480(bank->down_weight, E * H * I, p->flags + 1, true, st), "scan bank");
    bank_flag = p->flags;
  }
  // shared gate and up share one MFMA call; the GEMM ORs their two flags
  const int32_t* shared_gate_flag = nullptr;
  const int32_t* shared_up_flag = nullptr;
  const int32_t* shared_down_flag = nullptr;
  if (shared != nullptr) {
    if (shared->gate.code_flags != nullptr && shared->up.code_flags != nullptr) {
      shared_gate_flag = shared->gate.code_flags;
      shared_up_flag = shared->up.code_flags;
    } else {
      HIP_TRY(launch_scan_480(shared->gate.weight, Is * H, p->flags + 2, true, st), "scan shared gate");
      HIP_TRY(launch_scan_480(shared->up.weight, Is * H, p->flags + 2, false, st), "scan shared up");
      shared_gate_flag = p->flags + 2;
    }
    shared_down_flag = shared->down.code_flags;
    if (shared_down_flag == nullptr) {
      HIP_TRY(launch_scan_480(shared->down.weight, H * Is, p->flags + 3, true, st), "scan shared down");
      shared_down_flag = p->flags + 3;
    }
  }
  // 1. activations -> exact hi/lo E4M3 split
  HIP_TRY(split(x, T, H, p->xq, st), "split x");
  // 2. expert-sorted route plan: 128-route descriptors (the wide GEMM shape)
  // when experts average at least 48 routes, 64-route ones from 32 (fewer
  // re-reads of each weight tile), 32-route ones (a deeper load ring per
  // workgroup) below
  const int64_t act_rows = R > T ? R : T;
  const bool wide_fits = wide_offsets_fit(I, H, act_rows) && wide_offsets_fit(H, I, act_rows);
  const int tile = R >= 48 * E && wide_fits ? kGemmWideRows : R >= 32 * E ? kGemmTileRows : kGemmMinTileRows;
  const int64_t cap = cdiv(R, tile) + E;
  if ((rc = route_plan_impl(ids, sc, R, k, E, tile, p->sorted_route, p->inverse, p->sorted_expert,
                            p->sorted_token, p->sorted_score, p->route_offsets, p->tile_offsets, p->tile_expert,
                            p->tile_start, p->tile_len, cap, p->status, p->plan_ws, st)))
    return rc;
  // 3. grouped gate/up + SwiGLU (token rows gathered through sorted_token);
  // with a shared expert of the routed width, its dense gate/up (all T
  // tokens, identity rows) runs in the same launch as extra descriptors, so
  // its few items fill in beside the routed ones instead of running alone
  const bool merge_shared = shared != nullptr && Is == I;
  // merged: the shared hidden rows are rows R .. R + T - 1 of h and of its split
  uint16_t* const hs = merge_shared ? p->h + R * I : p->hs;
  const SplitBuf sq = merge_shared ? SplitBuf{p->hq.hi + R * I, p->hq.lo + R * I, p->hq.scale + R * SI} : p->sq;
  GroupedGemmArgs g{};
  g.a_hi = p->xq.hi;
  g.a_lo = p->xq.lo;
  g.a_scale = p->xq.scale;
  g.a_row_index = p->sorted_token;
  g.K = H;
  g.routes = R;
  g.tile_expert = p->tile_expert;
  g.tile_start = p->tile_start;
  g.tile_len = p->tile_len;
  g.tile_rows = tile;
  g.used_descriptors = p->status + 1;
  g.experts = E;
  g.weight = bank->gate_up_weight;
  g.weight_up = bank->gate_up_weight + I * H;  // row I: a whole number of row groups
  g.w_expert_stride = 2 * I * H;
  g.w_group_log2 = bank->row_group_log2;
  g.scale = bank->gate_up_scale_inv;
  g.scale_up = bank->gate_up_scale_inv + SR * SC;
  g.s_expert_stride = 2 * SR * SC;
  g.s_cols = SC;
  g.N = I;
  g.limit = p->limit;
  g.out = p->h;
  g.out_row_stride = I;
  g.fixup = bank_flag;
  if (merge_shared) {
    g.x_descriptors = cdiv(T, tile);
    g.x_routes = T;
    g.x_a_hi = p->xq.hi;
    g.x_a_lo = p->xq.lo;
    g.x_a_scale = p->xq.scale;
    g.x_weight = shared->gate.weight;
    g.x_weight_up = shared->up.weight;
    g.x_scale = shared->gate.scale_inv;
    g.x_scale_up = shared->up.scale_inv;
    g.x_out = hs;
    g.x_out_row_stride = Is;
    g.x_fixup = shared_gate_flag;
    g.x_fixup_up = shared_up_flag;
  }
  HIP_TRY(launch_grouped_gemm(g, GEMM_SWIGLU, cap, st), "grouped gate/up launch");
  // 4. hidden -> split, 5. grouped down (+ the shared down when merged)
  HIP_TRY(split(p->h, merge_shared ? R + T : R, I, p->hq, st), "split hidden");
  const int32_t* down_flag = bank->code_flags != nullptr ? bank->code_flags : p->flags + 1;
  GroupedGemmArgs d{};
  d.a_hi = p->hq.hi;
  d.a_lo = p->hq.lo;
  d.a_scale = p->hq.scale;
  d.K = I;
  d.routes = R;
  d.tile_expert = p->tile_expert;
  d.tile_start = p->tile_start;
  d.tile_len = p->tile_len;
  d.tile_rows = tile;
  d.used_descriptors = p->status + 1;
  d.experts = E;
  d.weight = bank->down_weight;
  d.w_expert_stride = H * I;
  d.w_group_log2 = bank->row_group_log2;
  d.scale = bank->down_scale_inv;
  d.s_expert_stride = (H / 128) * SI;
  d.s_cols = SI;
  d.N = H;
  d.out = p->down;
  d.out_row_stride = H;
  d.fixup = down_flag;
  if (merge_shared) {
    d.x_descriptors = cdiv(T, tile);
    d.x_routes = T;
    d.x_a_hi = sq.hi;
    d.x_a_lo = sq.lo;
    d.x_a_scale = sq.scale;
    d.x_weight = shared->down.weight;
    d.x_scale = shared->down.scale_inv;
    d.x_out = p->shared_out;
    d.x_out_row_stride = H;
    d.x_fixup = shared_down_flag;
  }
  HIP_TRY(launch_grouped_gemm(d, GEMM_PLAIN, cap, st), "grouped down launch");
  // 6. a shared expert of another width as its own dense M = T GEMM pair
  const uint16_t* shared_add = merge_shared ? p->shared_out : nullptr;
  if (shared != nullptr && !merge_shared) {
    GroupedGemmArgs sg{};
    sg.a_hi = p->xq.hi;
    sg.a_lo = p->xq.lo;
    sg.a_scale = p->xq.scale;
    sg.K = H;
    sg.routes = T;
    sg.experts = 1;
    sg.weight = shared->gate.weight;
    sg.weight_up = shared->up.weight;
    sg.scale = shared->gate.scale_inv;
    sg.scale_up = shared->up.scale_inv;
    sg.s_cols = SC;
    sg.N = Is;
    sg.limit = p->limit;
    sg.out = p->hs;
    sg.out_row_stride = Is;
    sg.fixup = shared_gate_flag;
    sg.fixup_up = shared_up_flag;
    const int stile = T >= 16 * kGemmTileRows ? kGemmTileRows : kGemmMinTileRows;
    sg.tile_rows = stile;
    HIP_TRY(launch_grouped_gemm(sg, GEMM_SWIGLU, cdiv(T, stile), st), "shared gate/up launch");
    HIP_TRY(split(p->hs, T, Is, p->sq, st), "split shared hidden");
    GroupedGemmArgs sd{};
    sd.a_hi = p->sq.hi;
    sd.a_lo = p->sq.lo;
    sd.a_scale = p->sq.scale;
    sd.K = Is;
    sd.routes = T;
    sd.experts = 1;
    sd.weight = shared->down.weight;
    sd.scale = shared->down.scale_inv;
    sd.s_cols = Is / 128;
    sd.N = H;
    sd.out = p->shared_out;
    sd.out_row_stride = H;
    sd.fixup = shared_down_flag;
    sd.tile_rows = stile;
    HIP_TRY(launch_grouped_gemm(sd, GEMM_PLAIN, cdiv(T, stile), st), "shared down launch");
    shared_add = p->shared_out;
  }
  // 7. combine
  ReduceArgs r{};
  r.route_out = p->down;
  r.inverse = p->inverse;
  r.sorted_score = p->sorted_score;
  r.route_score = p->scores;
  r.expert_ids = p->ids;
  r.shared = shared_add;
  r.tokens = T;
  r.H = H;
  r.top_k = static_cast<int>(k);
  r.out = static_cast<uint16_t*>(out);
  r.hc_residual = static_cast<const uint16_t*>(hc_residual);
  r.hc_post = hc_post;
  r.hc_comb = hc_comb;
  r.hc_out = static_cast<uint16_t*>(hc_out);
  HIP_TRY(launch_reduce(r, reduction == GLM53_REDUCE_DIRECT, st), "reduce launch");
  ++p->executions;
  return GLM53_OK;
}

int glm53_prefill_moe(glm53_prefill_plan* p, const glm53_bank* bank, const glm53_shared_expert* shared,
                      const glm53_router* router, const void* x, int64_t tokens, const int32_t* expert_ids,
                      const float* scores, int32_t reduction, void* out, void* stream) {
  CHECK_ARG(tokens == 0 || out != nullptr, "null pointer argument");
  return prefill_run(p, bank, shared, router, x, tokens, expert_ids, scores, reduction, out, nullptr, nullptr, nullptr,
                     nullptr, stream);
}

int glm53_prefill_moe_hc(glm53_prefill_plan* p, const glm53_bank* bank, const glm53_shared_expert* shared,
                         const glm53_router* router, const void* x, int64_t tokens, const int32_t* expert_ids,
                         const float* scores, int32_t reduction, const void* residual, const float* post,
                         const float* comb, void* out_hc, void* stream) {
  CHECK_ARG(tokens == 0 || (residual && post && comb && out_hc), "null pointer argument");
  return prefill_run(p, bank, shared, router, x, tokens, expert_ids, scores, reduction, nullptr, residual, post, comb,
                     out_hc, stream);
}

int glm53_prefill_plan_status(glm53_prefill_plan* plan, uint32_t* invalid_routes) {
  CHECK_ARG(plan && invalid_routes, "null pointer argument");
  if (plan->last_tokens == 0) {
    *invalid_routes = 0;
    return GLM53_OK;
  }
  HIP_TRY(hipMemcpy(invalid_routes, plan->status, sizeof(uint32_t), hipMemcpyDeviceToHost), "read status");
  ++plan->host_syncs;
  return GLM53_OK;
}

int glm53_prefill_plan_counters(const glm53_prefill_plan* plan, glm53_plan_counters* out) {
  CHECK_ARG(plan && out, "null pointer argument");
  *out = glm53_plan_counters{};
  out->execution_count = plan->executions;
  out->dynamic_allocation_count = 0;
  out->host_synchronization_count = plan->host_syncs;
  out->static_input_validation_count = plan->static_validations;
  out->dynamic_input_validation_count = plan->dynamic_validations;
  out->scratch_bytes = plan->arena_bytes;
  return GLM53_OK;
}

int glm53_prefill_plan_identities(const glm53_prefill_plan* plan, uint64_t* out, int32_t capacity, int32_t* count) {
  CHECK_ARG(plan && count && (capacity == 0 || out), "null pointer argument");
  const void* bufs[] = {plan->router_partial, plan->logits, plan->ids, plan->scores, plan->xq.hi,
                        plan->hq.hi, plan->sq.hi, plan->plan_ws, plan->sorted_route, plan->inverse,
                        plan->tile_expert, plan->h, plan->down, plan->hs, plan->shared_out, plan->flags};
  const int n = static_cast<int>(sizeof(bufs) / sizeof(bufs[0]));
  *count = n;
  for (int i = 0; i < n && i < capacity; ++i) out[i] = reinterpret_cast<uint64_t>(bufs[i]);
  return GLM53_OK;
}

int glm53_prefill_plan_scratch(glm53_prefill_plan* plan, int32_t which, void** ptr, size_t* bytes) {
  CHECK_ARG(plan && ptr && bytes, "null pointer argument");
  const int64_t R = plan->last_tokens * plan->k;
  switch (which) {
    case 0:
      *ptr = plan->ids;
      *bytes = 4 * R;
      return GLM53_OK;
    case 1:
      *ptr = plan->scores;
      *bytes = 4 * R;
      return GLM53_OK;
    case 2:
      *ptr = plan->sorted_route;
      *bytes = 4 * R;
      return GLM53_OK;
    case 3:
      *ptr = plan->tile_expert;
      *bytes = 4 * 3 * plan->capacity_max;
      return GLM53_OK;
    default:
      return fail(GLM53_INVALID_ARGUMENT, "unknown scratch id %d", which);
  }
}

int glm53_sigmoid_bf16(const void* gate, int64_t n, void* out, void* stream) {
  CHECK_ARG(n >= 0 && (n == 0 || (gate && out)), "invalid arguments");
  HIP_TRY(launch_sigmoid_bf16(static_cast<const uint16_t*>(gate), static_cast<uint16_t*>(out), n, S(stream)),
          "sigmoid launch");
  return GLM53_OK;
}

// --------------------------------------------------------- synthetic ------

int glm53_synth_fp8(uint8_t* codes, float* scale_inv, int64_t rows, int64_t cols, uint64_t seed, float std,
                    void* stream) {
  return glm53_synth_fp8_batched(codes, scale_inv, rows, cols, 1, 0, 0, seed, std, 0, stream);
}

int glm53_synth_fp8_batched(uint8_t* codes, float* scale_inv, int64_t rows, int64_t cols, int64_t batch,
                            int64_t codes_stride, int64_t scale_stride, uint64_t seed, float std,
                            int32_t row_group_log2, void* stream) {
  CHECK_ARG(rows >= 0 && cols >= 0 && batch >= 0 && batch < 65536, "invalid dimensions");
  CHECK_ARG(row_group_log2 >= 0 && row_group_log2 <= GLM53_MAX_ROW_GROUP_LOG2, "invalid row_group_log2");
  CHECK_ARG(row_group_log2 == 0 || (cols % 128 == 0 && rows % (int64_t{1} << row_group_log2) == 0),
            "a row-group layout needs cols % 128 == 0 and whole row groups");
  if (rows == 0 || cols == 0 || batch == 0) return GLM53_OK;
  CHECK_ARG(codes && scale_inv, "null pointer argument");
  SynthFp8Args a{codes, scale_inv, rows, cols, seed, std, batch, codes_stride, scale_stride, row_group_log2};
  HIP_TRY(launch_synth_fp8(a, S(stream)), "synth launch");
  return GLM53_OK;
}

int glm53_probe_read(const void* buf, int64_t bytes, uint32_t* sink, int32_t blocks, void* stream) {
  CHECK_ARG(buf && sink && bytes >= 0 && blocks > 0 && blocks <= (1 << 20), "invalid arguments");
  CHECK_ARG(aligned(buf, 16), "buffer must be 16-byte aligned");
  HIP_TRY(launch_probe_read(static_cast<const uint8_t*>(buf), bytes, sink, blocks, S(stream)), "probe launch");
  return GLM53_OK;
}

int glm53_synth_step_input(void* out, int64_t n, uint64_t seed, float std, uint32_t* counter, void* stream) {
  CHECK_ARG(n >= 0 && out && counter, "invalid arguments");
  HIP_TRY(launch_synth_step_input(static_cast<uint16_t*>(out), n, seed, std, counter, S(stream)), "synth launch");
  return GLM53_OK;
}

int glm53_synth_f32(float* out, int64_t n, uint64_t seed, float std, float lo, float hi, int32_t uniform, void* stream) {
  CHECK_ARG(n >= 0 && (n == 0 || out), "invalid arguments");
  HIP_TRY(launch_synth_f32(out, n, seed, std, lo, hi, uniform, S(stream)), "synth launch");
  return GLM53_OK;
}

int glm53_synth_bf16(void* out, int64_t n, uint64_t seed, float std, void* stream) {
  CHECK_ARG(n >= 0 && (n == 0 || out), "invalid arguments");
  HIP_TRY(launch_synth_bf16(static_cast<uint16_t*>(out), n, seed, std, S(stream)), "synth launch");
  return GLM53_OK;
}

}  // extern "C"
// ------------------------------------------------- allocation-free decode --
//
// glm53_decode_moe_static is glm53_decode_moe_ex (whole stage mask) without a
// plan, for callers that cannot allocate.  Its scratch is one file-scope
// device array; each GPU holds its own copy at its own address, which host
// code takes from hipGetSymbolAddress once per device -- the array's name in
// host code is only a stand-in, never a device address.

static __device__ __align__(256) uint8_t scratch[GLM53_DECODE_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kStaticMaxDevices = 64;
std::mutex g_static_mutex;
uint8_t* g_static_base[kStaticMaxDevices] = {};  // device address of `scratch` per GPU, set up once

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = 0u;
}

// Byte offsets inside the static scratch (each region 256-byte aligned).
struct StaticLayout {
  size_t count, err, ids, scores, words, shared_out, hidden, end;
};
StaticLayout static_layout(int64_t H, int64_t I, int64_t E, int64_t k) {
  StaticLayout l{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += round_up(bytes);
    return o;
  };
  l.count = take(4);  // launch-1 arrival counter: zero between calls (the last arriver resets it)
  l.err = take(4);
  l.ids = take(4 * k);
  l.scores = take(4 * k);
  l.words = take(8 * E);
  l.shared_out = take(2 * H);
  l.hidden = take(2 * (k + 1) * I);
  l.end = off;
  return l;
}

// The copy of the scratch on the GPU of `st`, which must be the current
// device (hipGetSymbolAddress resolves the current device's copy, and the
// kernels run on the stream's).  The first call on a GPU looks the address
// up and clears the whole array with a fill kernel on `st`, then waits for
// that kernel, so calls on any stream of that GPU start from the cleared
// array (that first call cannot be under graph capture, where waiting is not
// allowed).
int static_scratch_base(hipStream_t st, uint8_t** out) {
  int dev = 0, stream_dev = 0;
  HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  HIP_TRY(hipStreamGetDevice(st, &stream_dev), "hipStreamGetDevice");
  CHECK_ARG(stream_dev == dev, "the stream belongs to device %d but device %d is current; make the stream's device "
            "current before calling glm53_decode_moe_static", stream_dev, dev);
  CHECK_ARG(dev >= 0 && dev < kStaticMaxDevices, "device %d is beyond the static scratch table (%d devices)", dev,
            kStaticMaxDevices);
  std::lock_guard<std::mutex> lock(g_static_mutex);
  if (g_static_base[dev] == nullptr) {
    void* ptr = nullptr;
    HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, st, static_cast<uint32_t*>(ptr),
                       static_cast<int64_t>(GLM53_DECODE_STATIC_SCRATCH_BYTES / 4));
    HIP_TRY(hipGetLastError(), "static scratch clear launch");
    HIP_TRY(hipStreamSynchronize(st), "static scratch clear (first call on this GPU; not under graph capture)");
    g_static_base[dev] = static_cast<uint8_t*>(ptr);
  }
  *out = g_static_base[dev];
  return GLM53_OK;
}

}  // namespace

extern "C" int glm53_decode_moe_static(int64_t hidden, int64_t intermediate, int64_t experts, int64_t top_k,
                                       float swiglu_limit, const glm53_bank* bank, const glm53_shared_expert* shared,
                                       const glm53_router* router, const void* x, const void* residual, void* out,
                                       void* stream) {
  const int64_t H = hidden, I = intermediate, E = experts, k = top_k;
  CHECK_ARG(H > 0 && I > 0 && E > 0 && k > 0 && k <= kMaxTopK && k <= E, "invalid dimensions");
  CHECK_ARG(step_shape_supported(H, I),
            "glm53_decode_moe_static runs the fused step shapes only; (hidden %lld, intermediate %lld) is not one",
            (long long)H, (long long)I);
  CHECK_ARG(E <= 320, "glm53_decode_moe_static supports at most 320 experts (got %lld)", (long long)E);
  const StaticLayout lay = static_layout(H, I, E, k);
  CHECK_ARG(lay.end <= GLM53_DECODE_STATIC_SCRATCH_BYTES,
            "this shape needs %zu bytes of static scratch, more than its maximum of %d", lay.end,
            GLM53_DECODE_STATIC_SCRATCH_BYTES);
  int rc = check_bank(bank, H, I, E);
  if (rc) return rc;
  if (shared != nullptr) {
    if ((rc = check_linear(shared->gate, I, H, "shared gate"))) return rc;
    if ((rc = check_linear(shared->up, I, H, "shared up"))) return rc;
    if ((rc = check_linear(shared->down, H, I, "shared down"))) return rc;
  }
  if ((rc = check_router(router, H, E, k))) return rc;
  CHECK_ARG(x && out, "null pointer argument");
  CHECK_ARG(decode_fast_ok(H, I, I, bank, shared, x) && aligned(router->weight, 16) && aligned(out, 4),
            "glm53_decode_moe_static needs 16-byte aligned x and weights and a 4-byte aligned out");
  hipStream_t st = S(stream);
  uint8_t* base = nullptr;
  if ((rc = static_scratch_base(st, &base))) return rc;
  int slots = 0;  // launch width: depends on the shape, so found per call (a host-side query)
  const StepContext c{H, I, I, E, k, swiglu_limit,
                      reinterpret_cast<uint16_t*>(base + lay.hidden),
                      reinterpret_cast<unsigned long long*>(base + lay.words),
                      reinterpret_cast<uint32_t*>(base + lay.count),
                      reinterpret_cast<int32_t*>(base + lay.ids),
                      reinterpret_cast<float*>(base + lay.scores),
                      reinterpret_cast<int*>(base + lay.err),
                      reinterpret_cast<uint16_t*>(base + lay.shared_out),
                      &slots};
  rc = run_step(c, bank, shared, router, x, nullptr, nullptr, residual, out, GLM53_STAGE_ALL, 8, st);
  if (rc < 0) return fail(GLM53_INVALID_ARGUMENT, "glm53_decode_moe_static: inputs outside the fused step kernels");
  return rc;
}
