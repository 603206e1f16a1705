// C ABI of libicpp_hip.so: instance table, argument validation and launchers.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "icpp_registry.hpp"

static_assert((int)ICPP_CONV_EPI_BN == (int)icpp::CEPI_BN && (int)ICPP_CONV_EPI_RESIDUAL == (int)icpp::CEPI_RESIDUAL &&
                  (int)ICPP_CONV_EPI_VAR_CLAMP == (int)icpp::CEPI_VAR_CLAMP,
              "conv epilogue flags: header and kernels agree");

namespace icpp {

namespace {
std::vector<Instance>& table(int family) {
  static std::vector<Instance> t[ICPP_NUM_FAMILIES];
  return t[family];
}
bool& sorted_flag() {
  static bool s = false;
  return s;
}
thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// Instances register from static initializers in unspecified order; present
// them sorted by name so indices are stable across builds of the same list.
void ensure_sorted() {
  if (sorted_flag()) return;
  for (int f = 0; f < ICPP_NUM_FAMILIES; ++f) {
    std::stable_sort(table(f).begin(), table(f).end(), [](const Instance& a, const Instance& b) {
      return strcmp(a.tile.name, b.tile.name) < 0;
    });
  }
  sorted_flag() = true;
}

const Instance* lookup(int family, int inst) {
  ensure_sorted();
  if (family < 0 || family >= ICPP_NUM_FAMILIES) return nullptr;
  if (inst < 0 || inst >= (int)table(family).size()) return nullptr;
  return &table(family)[inst];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
int esz_of(int dt) { return dt == DT_FP8 ? 1 : 2; }
int ceil_div(int a, int b) { return (a + b - 1) / b; }

int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ICPP_OK;
}

// Workspace of the co-resident LayerNorm: per-(row, tile column) (mean, M2) pairs, a
// 16-byte block whose first int flags a wait that ran out, then the [tiles_m][2]
// arrival / departure counters.
struct LnCrLayout { size_t err_off, ctr_off, bytes; };
LnCrLayout ln_cr_layout(const icpp_tile_t& t, int M, int N) {
  LnCrLayout l;
  const size_t stats = (size_t)M * ceil_div(N, t.block_n) * 2 * sizeof(float);
  l.err_off = (stats + 15) / 16 * 16;
  l.ctr_off = l.err_off + 16;
  l.bytes = l.ctr_off + (size_t)ceil_div(M, t.block_m) * 2 * sizeof(int);
  return l;
}

// Workgroups of an instance's co-resident LayerNorm kernel the current device holds at
// once: CUs x workgroups per CU (the occupancy query, capped by the LDS a CU has).
// (The CU count and the occupancy are queried once per device and instance.)
int ln_cr_capacity(const Instance* in, int* cus_out = nullptr) {
  static std::mutex mu;
  static std::map<std::pair<int, const Instance*>, std::pair<int, int>> cache;  // -> (cus, per CU)
  int dev = 0;
  if (cus_out) *cus_out = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::pair<int, int> v;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({dev, in});
    if (it != cache.end()) {
      v = it->second;
    } else {
      int cus = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
      int per_cu = in->resident_ln_cr ? in->resident_ln_cr() : 0;
      per_cu = std::min(per_cu, (160 * 1024) / std::max(1, in->tile.lds_bytes));
      v = {std::max(0, cus), std::max(0, per_cu)};
      cache[{dev, in}] = v;
    }
  }
  if (cus_out) *cus_out = v.first;
  return v.first * v.second;
}

hipError_t launch_splitk_reduce(int dt, const float* ws, void* C, const void* bias, int M, int N, int ldc,
                                int splits, float alpha, int act, hipStream_t s, ConvEpiArgs ce = ConvEpiArgs{}) {
  const size_t groups = (size_t)M * (N / 4);
  // small outputs (skinny-M decode rows) spread over one-wave workgroups, so that more
  // CUs issue the partial loads: a CU's request rate, not HBM, bounds a grid this small
  const int threads = groups < (size_t)256 * 512 ? 64 : 256;
  const int blocks = (int)std::min<size_t>((groups + threads - 1) / threads, 4096);
  if (dt == DT_F16)
    hipLaunchKernelGGL(splitk_reduce_kernel<DT_F16>, dim3(blocks), dim3(threads), 0, s, ws, C, bias, M, N, ldc, splits, alpha, act, ce);
  else if (dt == DT_BF16)
    hipLaunchKernelGGL(splitk_reduce_kernel<DT_BF16>, dim3(blocks), dim3(threads), 0, s, ws, C, bias, M, N, ldc, splits, alpha, act, ce);
  else
    hipLaunchKernelGGL(splitk_reduce_kernel<DT_FP8>, dim3(blocks), dim3(threads), 0, s, ws, C, bias, M, N, ldc, splits, alpha, act, ce);
  return hipGetLastError();
}

// Split the nkt K tiles of a problem over at most `split_k` slices of
// ceil(nkt / split_k) tiles each (the last one may be shorter, none is empty).
// Returns the number of slices; *k_split receives the K elements per slice.
int plan_splits(int nkt, int block_k, int split_k, int* k_split) {
  const int per = ceil_div(nkt, split_k);
  *k_split = per * block_k;
  return ceil_div(nkt, per);
}

FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const uint32_t p = 31 + l;
  return FastDiv{(uint32_t)((1ull << p) / d + 1), p};
}

KArgs base_args() {
  KArgs a;
  memset(&a, 0, sizeof(a));
  a.alpha = 1.f;
  a.eps = 1e-5f;
  return a;
}

// Validate an icpp_gemm-style call and fill the kernel arguments (split-K planned,
// no workspace attached).  `what` names the entry point in error messages.
int gemm_prepare(const char* what, int inst, const void* A, const void* B, const void* bias, void* C, int M, int N,
                 int K, int lda, int ldb, int ldc, int act, float scale_a, float scale_b, int split_k,
                 const Instance** out_in, KArgs* out) {
  const Instance* in = lookup(ICPP_FAMILY_GEMM, inst);
  if (!in) return fail(ICPP_E_INSTANCE, "%s: no GEMM instance %d", what, inst);
  const icpp_tile_t& t = in->tile;
  if (!A || !B || !C) return fail(ICPP_E_ARG, "%s: null tensor", what);
  if (M <= 0 || N <= 0 || K <= 0) return fail(ICPP_E_SHAPE, "%s: empty shape M=%d N=%d K=%d", what, M, N, K);
  if (act < ICPP_ACT_NONE || act > ICPP_ACT_GELU_ERF) return fail(ICPP_E_ARG, "%s: bad act %d", what, act);
  if (split_k < 1) return fail(ICPP_E_ARG, "%s: split_k=%d", what, split_k);
  const int e = esz_of(t.dtype);
  const int vec = 16 / e;
  if (N % 8 || lda % vec || ldb % vec || ldc % 8 || lda < K || ldb < N || ldc < N)
    return fail(ICPP_E_SHAPE, "%s: need N%%8==0, lda,ldb multiples of %d, ldc%%8==0 (N=%d lda=%d ldb=%d ldc=%d)",
                what, vec, N, lda, ldb, ldc);
  if (K % t.block_k || split_k > K / t.block_k)
    return fail(ICPP_E_SHAPE, "%s: K=%d must be a multiple of block_k=%d with at least split_k=%d K tiles", what, K,
                t.block_k, split_k);
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || (bias && !aligned16(bias)))
    return fail(ICPP_E_ARG, "%s: pointers must be 16-byte aligned", what);
  if ((uint64_t)t.block_m * lda * e > 0x7FFFFFFFull || (uint64_t)K * ldb * e > 0xFFFFFFF0ull ||
      (uint64_t)t.block_m * ldc * 2 > 0x7FFFFFFFull)
    return fail(ICPP_E_SHAPE, "%s: operand exceeds the buffer range (block rows of A / C < 2 GiB, B < 4 GiB)", what);
  KArgs a = base_args();
  a.A = A; a.B = B; a.bias = bias; a.C = C;
  a.M = M; a.N = N; a.K = K; a.lda = lda; a.ldb = ldb; a.ldc = ldc;
  a.act = act; a.alpha = scale_a * scale_b;
  a.splits = plan_splits(K / t.block_k, t.block_k, split_k, &a.k_split);
  a.tiles_m = ceil_div(M, t.block_m);
  a.tiles_n = ceil_div(N, t.block_n);
  *out_in = in;
  *out = a;
  return ICPP_OK;
}

}  // namespace

int register_instance(const Instance& inst) {
  if (inst.tile.family < 0 || inst.tile.family >= ICPP_NUM_FAMILIES) return -1;
  table(inst.tile.family).push_back(inst);
  sorted_flag() = false;
  return (int)table(inst.tile.family).size();
}

// The row-op translation unit (icpp_rowops.hip) reports through the same buffer.
int set_last_error(int code, const char* msg) { return fail(code, "%s", msg); }
int layernorm_rows_f16(const void* X, const void* R, const float* block_mean, int bm_cols, int bm_width, const void* W,
                       const void* B, void* Y, int M, int N, float eps, hipStream_t s);  // icpp_rowops.hip

}  // namespace icpp

using namespace icpp;

extern "C" {

int icpp_abi_version(void) { return ICPP_ABI_VERSION; }

const char* icpp_last_error(void) { return g_err.c_str(); }

int icpp_num_instances(int family) {
  ensure_sorted();
  if (family < 0 || family >= ICPP_NUM_FAMILIES) return fail(ICPP_E_INSTANCE, "bad family %d", family);
  return (int)table(family).size();
}

int icpp_instance_info(int family, int idx, icpp_tile_t* out) {
  const Instance* in = lookup(family, idx);
  if (!in) return fail(ICPP_E_INSTANCE, "no instance %d in family %d", idx, family);
  if (!out) return fail(ICPP_E_ARG, "null output");
  *out = in->tile;
  return ICPP_OK;
}

size_t icpp_workspace_bytes(int family, int inst, int M, int N, int K, int split_k) {
  (void)K;
  const Instance* in = lookup(family, inst);
  if (!in || M <= 0 || N <= 0) return 0;
  if (family == ICPP_FAMILY_GEMM_LN_STATS) {
    const size_t stat_cols = (size_t)ceil_div(N, in->wave_tile_n);
    return (size_t)M * stat_cols * 2 * sizeof(float);
  }
  if ((family == ICPP_FAMILY_GEMM || family == ICPP_FAMILY_CONV2D) && split_k > 1)
    return (size_t)split_k * M * N * sizeof(float);
  return 0;
}

int icpp_gemm(int inst, const void* A, const void* B, const void* bias, void* C,
              int M, int N, int K, int lda, int ldb, int ldc, int act,
              float scale_a, float scale_b, int split_k,
              void* workspace, size_t ws_bytes, void* stream) {
  const Instance* in = nullptr;
  KArgs a;
  if (int rc = gemm_prepare("icpp_gemm", inst, A, B, bias, C, M, N, K, lda, ldb, ldc, act, scale_a, scale_b, split_k,
                            &in, &a))
    return rc;
  const icpp_tile_t& t = in->tile;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(a.tiles_m * a.tiles_n * a.splits);  // one workgroup per (tile, K split) item
  if (a.splits > 1) {
    const size_t need = (size_t)split_k * M * N * sizeof(float);
    if (!workspace || ws_bytes < need || !aligned16(workspace))
      return fail(ICPP_E_WORKSPACE, "icpp_gemm: split_k=%d needs %zu workspace bytes (got %zu)", split_k, need, ws_bytes);
    if (ldc != N) return fail(ICPP_E_SHAPE, "icpp_gemm: split-K output needs ldc == N");
    a.partial = 1;
    a.ws = (float*)workspace;
    int rc = check_launch(in->launch(a, grid, s), t.name);
    if (rc) return rc;
    return check_launch(launch_splitk_reduce(t.dtype, a.ws, C, bias, M, N, ldc, a.splits, a.alpha, act, s), "splitk_reduce");
  }
  return check_launch(in->launch(a, grid, s), t.name);
}

size_t icpp_gemm_bias_layernorm_workspace_bytes(int family, int inst, int M, int N, int K) {
  (void)K;
  if (M <= 0 || N <= 0) return 0;
  if (family == ICPP_FAMILY_GEMM) {
    const Instance* in = lookup(ICPP_FAMILY_GEMM, inst);
    if (!in) return 0;
    return (size_t)M * ceil_div(N, in->wave_tile_n) * sizeof(float);
  }
  if (family == ICPP_FAMILY_GEMM_LN_STATS) return icpp_workspace_bytes(family, inst, M, N, K, 1);
  if (family == ICPP_LN_CORESIDENT) {
    const Instance* in = lookup(ICPP_FAMILY_GEMM, inst);
    if (!in || !in->launch_ln_cr) return 0;
    const LnCrLayout l = ln_cr_layout(in->tile, M, N);
    return l.bytes;
  }
  return 0;
}

int icpp_gemm_bias_layernorm(int family, int inst, const void* A, const void* B, const void* bias,
                             const void* gamma, const void* beta, void* Y,
                             int M, int N, int K, float eps,
                             void* workspace, size_t ws_bytes, void* stream) {
  return icpp_gemm_bias_residual_layernorm(family, inst, A, B, bias, nullptr, gamma, beta, Y, M, N, K, eps,
                                           workspace, ws_bytes, stream);
}

int icpp_gemm_bias_residual_layernorm(int family, int inst, const void* A, const void* B, const void* bias,
                                      const void* residual, const void* gamma, const void* beta, void* Y,
                                      int M, int N, int K, float eps,
                                      void* workspace, size_t ws_bytes, void* stream) {
  if (family == ICPP_LN_CORESIDENT) {
    // One launch per chunk of row blocks that the device keeps resident at once; the
    // tiles of a row block exchange their (mean, M2) and normalise from registers.
    if (!gamma || !beta) return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: null tensor");
    const Instance* gi = lookup(ICPP_FAMILY_GEMM, inst);
    if (!gi) return fail(ICPP_E_INSTANCE, "icpp_gemm_bias_layernorm: no GEMM instance %d", inst);
    if (gi->tile.dtype != DT_F16 || !gi->launch_ln_cr)
      return fail(ICPP_E_INSTANCE, "icpp_gemm_bias_layernorm: GEMM instance %s has no co-resident LayerNorm kernel",
                  gi->tile.name);
    if (!(eps > 0.f)) return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: eps must be > 0");
    if ((residual && !aligned16(residual)) || !aligned16(gamma) || !aligned16(beta))
      return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: pointers must be 16-byte aligned");
    KArgs a;
    if (int rc = gemm_prepare("icpp_gemm_bias_layernorm", inst, A, B, bias, Y, M, N, K, K, N, N, ICPP_ACT_NONE, 1.f,
                              1.f, 1, &gi, &a))
      return rc;
    const icpp_tile_t& t = gi->tile;
    {
      // a row block's [block_m][tiles_n] (mean, M2) pairs go to two stage arrays, an even
      // number of rows in the first (the kernel's split), the rest in the second
      const size_t per = (size_t)gi->ln_cr_stage_bytes / ((size_t)a.tiles_n * 2 * sizeof(float));
      if ((size_t)t.block_m > (per & ~(size_t)1) + per)
        return fail(ICPP_E_SHAPE, "icpp_gemm_bias_layernorm: N=%d is too wide for %s: a row block's statistics exceed two LDS stages",
                    N, t.name);
    }
    int cus = 0;
    const int cap = ln_cr_capacity(gi, &cus);
    if (cap < a.tiles_n)
      return fail(ICPP_E_SHAPE, "icpp_gemm_bias_layernorm: %s: the %d tiles of a row block cannot be resident at once (%d)",
                  t.name, a.tiles_n, cap);
    const LnCrLayout l = ln_cr_layout(t, M, N);
    if (!workspace || ws_bytes < l.bytes || !aligned16(workspace))
      return fail(ICPP_E_WORKSPACE, "icpp_gemm_bias_layernorm: needs %zu workspace bytes (got %zu)", l.bytes, ws_bytes);
    a.gamma = gamma; a.beta = beta; a.eps = eps; a.residual = residual;
    char* w = (char*)workspace;
    int* ctr = (int*)(w + l.ctr_off);
    a.ln_err = (int*)(w + l.err_off);
    const int max_rows = cap / a.tiles_n;
    hipStream_t s = (hipStream_t)stream;
    if (a.tiles_m > max_rows && cus % 8 == 0) {
      // More row blocks than the device holds at once: one launch in rounds of R row
      // blocks, when the round splits into 8 equal per-XCD blocks of (R / xa) x
      // (tiles_n / xb) tiles that fit each XCD's share of the CUs (the fewest A + B
      // panels per XCD, and among those the most row splits: a row block then spans
      // the fewest XCDs and waits on fewer of them); otherwise even chunks, one launch
      // each.  (Every XCD has the
      // same share of the CUs only when their count divides by 8.)
      int best_a = 0, best_cost = 1 << 30;
      const int per_xcd = cap / 8;
      for (int xa = 1; xa <= 8; xa *= 2) {
        const int xb = 8 / xa;
        if (max_rows % xa || a.tiles_n % xb) continue;
        if ((max_rows / xa) * (a.tiles_n / xb) > per_xcd) continue;
        const int cost = max_rows / xa + a.tiles_n / xb;
        if (cost <= best_cost) best_cost = cost, best_a = xa;
      }
      if (best_a) {
        KArgs b = a;
        b.cr_rows = max_rows;
        b.cr_xa = best_a;
        b.cr_xb = 8 / best_a;
        b.ws = (float*)w;
        b.ln_ctr = ctr;
        const int rounds = ceil_div(a.tiles_m, max_rows);
        return check_launch(gi->launch_ln_cr(b, dim3(rounds * max_rows * a.tiles_n), s), t.name);
      }
    }
    // even chunks of at most cap / tiles_n row blocks
    const int chunks = ceil_div(a.tiles_m, max_rows);
    const int chunk_tm = ceil_div(a.tiles_m, chunks);
    for (int tm0 = 0; tm0 < a.tiles_m; tm0 += chunk_tm) {
      const int r0 = tm0 * t.block_m;
      KArgs b = a;
      b.A = (const char*)A + (size_t)r0 * K * 2;
      b.C = (char*)Y + (size_t)r0 * N * 2;
      if (residual) b.residual = (const char*)residual + (size_t)r0 * N * 2;
      b.M = std::min(M - r0, chunk_tm * t.block_m);
      b.tiles_m = ceil_div(b.M, t.block_m);
      b.ws = (float*)w + (size_t)r0 * a.tiles_n * 2;
      b.ln_ctr = ctr + 2 * tm0;
      if (int rc = check_launch(gi->launch_ln_cr(b, dim3(b.tiles_m * b.tiles_n), s), t.name)) return rc;
    }
    return ICPP_OK;
  }
  if (family == ICPP_FAMILY_GEMM) {
    // GEMM-then-LayerNorm: a plain f16 GEMM + bias into Y (staged epilogue, any GEMM tile), then
    // the row LayerNorm kernel in place (adding the residual); the same HBM traffic as two-pass
    if (!gamma || !beta) return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: null tensor");
    const Instance* gi = lookup(ICPP_FAMILY_GEMM, inst);
    if (!gi) return fail(ICPP_E_INSTANCE, "icpp_gemm_bias_layernorm: no GEMM instance %d", inst);
    if (gi->tile.dtype != DT_F16) return fail(ICPP_E_INSTANCE, "icpp_gemm_bias_layernorm: GEMM instance %d is not f16", inst);
    if (!(eps > 0.f)) return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: eps must be > 0");
    if ((residual && !aligned16(residual)) || !aligned16(gamma) || !aligned16(beta))
      return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: pointers must be 16-byte aligned");
    if (residual && M > 0 && N > 0) {
      // the GEMM writes Y before the LayerNorm reads the residual: they must not share memory
      const char* r0 = (const char*)residual;
      const char* y0 = (const char*)Y;
      const size_t bytes = (size_t)M * N * 2;
      if (r0 < y0 + bytes && y0 < r0 + bytes)
        return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: the GEMM family needs a residual that does not overlap Y");
    }
    // The GEMM stores Y centred on per-(row, wave column block) means and writes the
    // means (fp32) into the workspace; the row LayerNorm adds them back.
    KArgs a;
    if (int rc = gemm_prepare("icpp_gemm_bias_layernorm", inst, A, B, bias, Y, M, N, K, K, N, N, ICPP_ACT_NONE, 1.f,
                              1.f, 1, &gi, &a))
      return rc;
    a.stat_cols = ceil_div(N, gi->wave_tile_n);
    const size_t need = (size_t)M * a.stat_cols * sizeof(float);
    if (!workspace || ws_bytes < need || !aligned16(workspace))
      return fail(ICPP_E_WORKSPACE, "icpp_gemm_bias_layernorm: needs %zu workspace bytes (got %zu)", need, ws_bytes);
    a.ws = (float*)workspace;
    hipStream_t s = (hipStream_t)stream;
    int rc = check_launch(gi->launch(a, dim3(a.tiles_m * a.tiles_n), s), gi->tile.name);
    if (rc) return rc;
    return layernorm_rows_f16(Y, residual, a.ws, a.stat_cols, gi->wave_tile_n, gamma, beta, Y, M, N, eps, s);
  }
  if (family != ICPP_FAMILY_GEMM_LN_ROW && family != ICPP_FAMILY_GEMM_LN_STATS)
    return fail(ICPP_E_INSTANCE, "icpp_gemm_bias_layernorm: family %d is not a LayerNorm family", family);
  const Instance* in = lookup(family, inst);
  if (!in) return fail(ICPP_E_INSTANCE, "icpp_gemm_bias_layernorm: no instance %d in family %d", inst, family);
  const icpp_tile_t& t = in->tile;
  if (!A || !B || !Y || !gamma || !beta) return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: null tensor");
  if (M <= 0 || N <= 0 || K <= 0) return fail(ICPP_E_SHAPE, "icpp_gemm_bias_layernorm: empty shape");
  if (N % 8 || K % 8) return fail(ICPP_E_SHAPE, "icpp_gemm_bias_layernorm: need N%%8==0 and K%%8==0");
  if (K % t.block_k) return fail(ICPP_E_SHAPE, "icpp_gemm_bias_layernorm: K=%d not a multiple of block_k=%d", K, t.block_k);
  if (!aligned16(A) || !aligned16(B) || !aligned16(Y) || !aligned16(gamma) || !aligned16(beta) || (bias && !aligned16(bias)) ||
      (residual && !aligned16(residual)))
    return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: pointers must be 16-byte aligned");
  if (!(eps > 0.f)) return fail(ICPP_E_ARG, "icpp_gemm_bias_layernorm: eps must be > 0");
  KArgs a = base_args();
  a.A = A; a.B = B; a.bias = bias; a.C = Y; a.gamma = gamma; a.beta = beta; a.residual = residual;
  a.M = M; a.N = N; a.K = K; a.lda = K; a.ldb = N; a.ldc = N; a.eps = eps;
  a.k_split = K;
  a.splits = 1;
  a.tiles_m = ceil_div(M, t.block_m);
  a.tiles_n = ceil_div(N, t.block_n);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(a.tiles_m * a.tiles_n);
  if (family == ICPP_FAMILY_GEMM_LN_ROW) {
    if (a.tiles_n != 1) return fail(ICPP_E_SHAPE, "row LayerNorm instance %s needs N <= block_n (N=%d)", t.name, N);
    return check_launch(in->launch(a, grid, s), t.name);
  }
  a.stat_cols = ceil_div(N, in->wave_tile_n);
  const size_t need = (size_t)M * a.stat_cols * 2 * sizeof(float);
  if (!workspace || ws_bytes < need || !aligned16(workspace))
    return fail(ICPP_E_WORKSPACE, "icpp_gemm_bias_layernorm: needs %zu workspace bytes (got %zu)", need, ws_bytes);
  a.ws = (float*)workspace;
  int rc = check_launch(in->launch(a, grid, s), t.name);
  if (rc) return rc;
  hipLaunchKernelGGL(ln_finalize_kernel<DT_F16>, dim3(ceil_div(M, 4)), dim3(256), 0, s, Y, (const float*)a.ws, gamma, beta,
                     M, N, N, a.stat_cols, in->wave_tile_n, eps);
  return check_launch(hipGetLastError(), "ln_finalize");
}

int icpp_conv2d_nhwc(int inst, const void* X, const void* Wt, void* Y,
                     int N, int H, int W, int C, int F, int KH, int KW,
                     int stride, int pad, int dilation, int split_k,
                     void* workspace, size_t ws_bytes, void* stream) {
  return icpp_conv2d_nhwc_fused(inst, X, Wt, Y, nullptr, nullptr, nullptr, nullptr, nullptr, 0.f, 0, ICPP_ACT_NONE,
                                N, H, W, C, F, KH, KW, stride, pad, dilation, split_k, workspace, ws_bytes, stream);
}

int icpp_conv2d_nhwc_fused(int inst, const void* X, const void* Wt, void* Y, const void* residual,
                           const void* gamma, const void* beta, const void* mean, const void* var,
                           float eps, int epi_flags, int act,
                           int N, int H, int W, int C, int F, int KH, int KW,
                           int stride, int pad, int dilation, int split_k,
                           void* workspace, size_t ws_bytes, void* stream) {
  const Instance* in = lookup(ICPP_FAMILY_CONV2D, inst);
  if (!in) return fail(ICPP_E_INSTANCE, "icpp_conv2d_nhwc: no conv instance %d", inst);
  const icpp_tile_t& t = in->tile;
  if (!X || !Wt || !Y) return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: null tensor");
  if (epi_flags & ~(ICPP_CONV_EPI_BN | ICPP_CONV_EPI_RESIDUAL | ICPP_CONV_EPI_VAR_CLAMP))
    return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: unknown epilogue flags 0x%x", epi_flags);
  if (act != ICPP_ACT_NONE && act != ICPP_ACT_RELU)
    return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: act must be NONE or RELU (got %d)", act);
  const bool bn = (epi_flags & ICPP_CONV_EPI_BN) != 0;
  if (bn && (!gamma || !beta || !mean || !var))
    return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: BN needs gamma, beta, mean and var");
  if ((epi_flags & ICPP_CONV_EPI_VAR_CLAMP) && !bn) return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: VAR_CLAMP without BN");
  if ((epi_flags & ICPP_CONV_EPI_RESIDUAL) && !residual) return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: RESIDUAL needs a residual");
  if (bn && !(eps >= 0.f)) return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: eps must be >= 0");
  if ((bn && (!aligned16(gamma) || !aligned16(beta) || !aligned16(mean) || !aligned16(var))) ||
      ((epi_flags & ICPP_CONV_EPI_RESIDUAL) && !aligned16(residual)))
    return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: epilogue pointers must be 16-byte aligned");
  if (N <= 0 || H <= 0 || W <= 0 || C <= 0 || F <= 0 || KH <= 0 || KW <= 0 || stride <= 0 || pad < 0 || dilation <= 0)
    return fail(ICPP_E_SHAPE, "icpp_conv2d_nhwc: bad geometry");
  if (split_k < 1) return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: split_k=%d", split_k);
  const int OH = (H + 2 * pad - dilation * (KH - 1) - 1) / stride + 1;
  const int OW = (W + 2 * pad - dilation * (KW - 1) - 1) / stride + 1;
  if (OH <= 0 || OW <= 0) return fail(ICPP_E_SHAPE, "icpp_conv2d_nhwc: empty output");
  if (C % 8 || F % 8) return fail(ICPP_E_SHAPE, "icpp_conv2d_nhwc: need C%%8==0 and F%%8==0 (C=%d F=%d)", C, F);
  const long long Mg = (long long)N * OH * OW;
  const long long Kg = (long long)KH * KW * C;
  // rows of the last M tile (up to tiles_m * block_m - 1) index the gather: they stay below 2^31
  if (Mg > 0x7FFFFFFFll - t.block_m || Kg % t.block_k || split_k > Kg / t.block_k)
    return fail(ICPP_E_SHAPE, "icpp_conv2d_nhwc: K=%lld must be a multiple of block_k=%d with at least split_k=%d K tiles",
                Kg, t.block_k, split_k);
  const unsigned long long xbytes = (unsigned long long)N * H * W * C * 2;
  // padding taps load from offset xbytes (past the range): keep it and the output block rows below 2 GiB
  if (xbytes > 0x7FFFFFF0ull || (uint64_t)t.block_m * F * 2 > 0x7FFFFFFFull)
    return fail(ICPP_E_SHAPE, "icpp_conv2d_nhwc: input or output exceeds the 2 GiB buffer range");
  if (!aligned16(X) || !aligned16(Wt) || !aligned16(Y)) return fail(ICPP_E_ARG, "icpp_conv2d_nhwc: pointers must be 16-byte aligned");
  KArgs a = base_args();
  a.A = X; a.B = Wt; a.C = Y;
  a.M = (int)Mg; a.N = F; a.K = (int)Kg; a.lda = 0; a.ldb = F; a.ldc = F;
  a.splits = plan_splits((int)(Kg / t.block_k), t.block_k, split_k, &a.k_split);
  a.tiles_m = ceil_div(a.M, t.block_m);
  a.tiles_n = ceil_div(F, t.block_n);
  a.cH = H; a.cW = W; a.cC = C; a.cKH = KH; a.cKW = KW; a.cS = stride; a.cP = pad; a.cD = dilation; a.cOH = OH;
  a.cOW = OW;
  a.dv_ohw = make_fastdiv((uint32_t)(OH * OW));
  a.dv_ow = make_fastdiv((uint32_t)OW);
  a.dv_w = make_fastdiv((uint32_t)W);
  a.dv_wp = make_fastdiv((uint32_t)(W + 2));
  a.dv_h = make_fastdiv((uint32_t)H);
  a.tap_rows = 0;
  for (int kh = 0; kh < KH && kh * KW < 32; ++kh) a.tap_rows |= 1u << (kh * KW);
  a.a_bytes_total = (uint32_t)xbytes;
  a.act = act;
  a.ce.flags = epi_flags;
  a.ce.eps = eps;
  a.ce.gamma = gamma; a.ce.beta = beta; a.ce.mean = mean; a.ce.var = var;
  a.ce.residual = residual;
  hipStream_t s = (hipStream_t)stream;
  // A loader: the input halo (3x3, stride 1, pad 1, one K tile per tap, no split and the
  // tile's halo -- its output rows spanned plus a one-row border, W pixels each, and
  // one zero pixel, 128 B per pixel -- within the instance's halo capacity); else the
  // per-tile-tap gather when every K tile lies inside one tap; else the per-chunk gather
  const long long halo_rows = (t.block_m - 1) / W + 2 + 2;  // rows a tile can span, plus the border
  const bool halo = in->launch_halo && KH == 3 && KW == 3 && stride == 1 && dilation == 1 && pad == 1 &&
                    C == t.block_k && a.splits == 1 && (halo_rows * W + 1) * 128 <= in->halo_bytes;
  const LaunchFn launch = halo ? in->launch_halo
                               : (C % t.block_k == 0 && KH * KW <= 32) ? in->launch : in->launch_gather;
  const dim3 grid(a.tiles_m * a.tiles_n * a.splits);  // one workgroup per (tile, K split) item
  if (a.splits > 1) {
    const size_t need = (size_t)split_k * a.M * F * sizeof(float);
    if (!workspace || ws_bytes < need || !aligned16(workspace))
      return fail(ICPP_E_WORKSPACE, "icpp_conv2d_nhwc: split_k=%d needs %zu workspace bytes (got %zu)", split_k, need, ws_bytes);
    a.partial = 1;
    a.ws = (float*)workspace;
    int rc = check_launch(launch(a, grid, s), t.name);
    if (rc) return rc;
    return check_launch(launch_splitk_reduce(DT_F16, a.ws, Y, nullptr, a.M, F, F, a.splits, 1.f, act, s, a.ce),
                        "splitk_reduce");
  }
  return check_launch(launch(a, grid, s), t.name);
}

}  // extern "C"
