// The audio encoder's self-attention block (include/ffai_encoder.h): hipBLASLt GEMMs for the
// projections, with their outputs laid out so that the fused attention reads them by stride,
// replacing EncoderAttention::forward (crates/ffai-mercury/src/asr/text_decoder.rs:1059-1139).
//
// A call runs its windows in passes of at most kMaxRows rows (one 1500-frame window for
// whisper, several shorter ones), each pass through the same workspace, as the reference loops
// over batch items (text_decoder.rs:1069-1076). Below, B is the windows of one pass.
//
// Workspace (compute dtype T = bf16 or f16; B batch, S seq, N n_state, H heads, hd = N / H):
//   attention workspace, first and at least the split counters' size: the counters must stay at
//                          the same place, untouched by anything else, for calls of any shape
//                          through one workspace (zeroed once, left zero by every call)
//   q      (B, S, N)     = x Wq^T + bq       read by the kernel as (B, H, S, hd), strides (S N, hd, N, 1)
//   v      (B, S, N)     = x Wv^T + bv       likewise
//   kt     (N, B S)      = Wk_scaled x^T over every window at once: element (b, h, j, s) at
//                          (h hd + j) B S + b S + s, read by the kernel as K^T with strides
//                          (S, hd B S, B S, 1) -- one plain GEMM, no batched GEMM
//   merged (B, S, N)     attention output, the kernel writing the merged layout directly
//   hipBLASLt scratch
// With packed weights (wqkv, bqkv) the first three regions hold instead
//   qkv    (B, S, 3N)    = x Wqkv^T + bqkv in one GEMM: q, k and v of one frame side by side,
//                          read by the kernel with strides (S 3N, hd, 3N, 1) and K as rows
// All GEMMs are column-major in hipBLASLt's terms: a row-major (rows, cols) matrix is a
// column-major (cols, rows) one, so Y = X W^T (row-major, X (M, K), W (N, K)) is computed as
// Y^T = W X^T with A = W (op T), B = X (op N), and the bias runs along Y^T's rows (features).

#include "../../include/ffai_encoder.h"

#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "attn_kernels.h"

namespace {

using ffai::api_check_device;
using ffai::api_clear_error;
using ffai::api_fail;

constexpr size_t kGemmScratch = size_t(32) << 20;  // hipBLASLt workspace ceiling
// Rows (windows x seq) per pass: one 30 s window, the reference's own granularity (it loops over
// windows, text_decoder.rs:1069-1076). A call of more windows runs several passes; a single pass
// of more rows is refused (it has not been validated on the GPU).
constexpr int64_t kMaxRows = 1500;
constexpr int kMaxDevices = 64;

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

std::mutex g_mu;
hipblasLtHandle_t g_handle[kMaxDevices] = {};

// Heuristic choice per GEMM (dtype, ops, m, n, k, leading dimensions, bias, workspace): the first
// one hipBLASLt offers for the workspace ceiling. Handles are per device; algorithms are data.
using GemmKey = std::tuple<int, int, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                           int, int>;
std::map<GemmKey, hipblasLtMatmulAlgo_t> g_algo;

int lt_check(hipblasStatus_t st, const char* what) {
  if (st == HIPBLAS_STATUS_SUCCESS) return FFAI_OK;
  return api_fail(FFAI_ERR_HIP, (std::string("hipBLASLt ") + what + " failed (status " +
                                 std::to_string((int)st) + ")").c_str());
}

int handle_for_current(hipblasLtHandle_t* h) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return api_fail(FFAI_ERR_HIP, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return api_fail(FFAI_ERR_DEVICE, "device index out of range");
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_handle[dev]) {
    const int rc = lt_check(hipblasLtCreate(&g_handle[dev]), "create");
    if (rc != FFAI_OK) return rc;
  }
  *h = g_handle[dev];
  return FFAI_OK;
}

struct Gemm {
  hipblasOperation_t ta, tb;
  int64_t m, n, k;               // D is m x n (column-major), op(A) m x k, op(B) k x n
  const void* a; int64_t lda;
  const void* b; int64_t ldb;
  void* d; int64_t ldd;
  const void* bias;              // length m, or null
};

// RAII holders for the descriptors of one call
struct Descs {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  ~Descs() {
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (ld) hipblasLtMatrixLayoutDestroy(ld);
    if (lb) hipblasLtMatrixLayoutDestroy(lb);
    if (la) hipblasLtMatrixLayoutDestroy(la);
    if (op) hipblasLtMatmulDescDestroy(op);
  }
};

int layout(hipblasLtMatrixLayout_t* l, hipDataType dt, int64_t rows, int64_t cols, int64_t ld) {
  return lt_check(hipblasLtMatrixLayoutCreate(l, dt, rows, cols, ld), "layout");
}

int run_gemm(hipblasLtHandle_t h, const Gemm& g, hipDataType dt, void* scratch, size_t scratch_bytes,
             hipStream_t st) {
  Descs ds;
  int rc = lt_check(hipblasLtMatmulDescCreate(&ds.op, HIPBLAS_COMPUTE_32F, HIP_R_32F), "matmul desc");
  if (rc != FFAI_OK) return rc;
  rc = lt_check(hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_TRANSA, &g.ta, sizeof(g.ta)), "transA");
  if (rc != FFAI_OK) return rc;
  rc = lt_check(hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_TRANSB, &g.tb, sizeof(g.tb)), "transB");
  if (rc != FFAI_OK) return rc;
  if (g.bias) {
    const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bdt = (int32_t)dt;
    rc = lt_check(hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)), "epilogue");
    if (rc != FFAI_OK) return rc;
    rc = lt_check(hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &g.bias, sizeof(g.bias)), "bias");
    if (rc != FFAI_OK) return rc;
    rc = lt_check(hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bdt, sizeof(bdt)), "bias type");
    if (rc != FFAI_OK) return rc;
  }
  const bool at = g.ta == HIPBLAS_OP_T, bt = g.tb == HIPBLAS_OP_T;
  if ((rc = layout(&ds.la, dt, at ? g.k : g.m, at ? g.m : g.k, g.lda)) != FFAI_OK) return rc;
  if ((rc = layout(&ds.lb, dt, bt ? g.n : g.k, bt ? g.k : g.n, g.ldb)) != FFAI_OK) return rc;
  if ((rc = layout(&ds.ld, dt, g.m, g.n, g.ldd)) != FFAI_OK) return rc;

  const GemmKey key{(int)dt, (int)g.ta, (int)g.tb, g.m, g.n, g.k, g.lda, g.ldb, g.ldd,
                    g.bias != nullptr, (int)(scratch_bytes >> 20)};
  hipblasLtMatmulAlgo_t algo;
  bool have = false;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_algo.find(key);
    if (it != g_algo.end()) { algo = it->second; have = true; }
  }
  if (!have) {
    rc = lt_check(hipblasLtMatmulPreferenceCreate(&ds.pref), "preference");
    if (rc != FFAI_OK) return rc;
    const uint64_t ws = scratch_bytes;
    rc = lt_check(hipblasLtMatmulPreferenceSetAttribute(ds.pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)), "workspace pref");
    if (rc != FFAI_OK) return rc;
    hipblasLtMatmulHeuristicResult_t res[1];
    int n = 0;
    rc = lt_check(hipblasLtMatmulAlgoGetHeuristic(h, ds.op, ds.la, ds.lb, ds.ld, ds.ld, ds.pref, 1, res, &n), "heuristic");
    if (rc != FFAI_OK) return rc;
    if (n < 1) return api_fail(FFAI_ERR_HIP, "hipBLASLt offers no algorithm for an encoder GEMM");
    algo = res[0].algo;
    std::lock_guard<std::mutex> lk(g_mu);
    g_algo.emplace(key, algo);
  }
  const float alpha = 1.f, beta = 0.f;
  return lt_check(hipblasLtMatmul(h, ds.op, &alpha, g.a, ds.la, g.b, ds.lb, &beta, g.d, ds.ld, g.d, ds.ld,
                                  &algo, scratch, scratch_bytes, st), "matmul");
}

struct Sizes {
  size_t q, kt, v, merged, attn, gemm, total;
};

int check(const ffai_encoder_attn_desc* d) {
  if (!d) return api_fail(FFAI_ERR_INVALID, "null descriptor");
  if (d->dtype != FFAI_BF16 && d->dtype != FFAI_F16)
    return api_fail(FFAI_ERR_INVALID, "dtype must be FFAI_BF16 or FFAI_F16");
  if (d->batch < 1 || d->seq < 1 || d->n_state < 1 || d->n_head < 1)
    return api_fail(FFAI_ERR_INVALID, "sizes must be positive");
  if (d->n_state % d->n_head) return api_fail(FFAI_ERR_INVALID, "n_state must be a multiple of n_head");
  const int hd = d->n_state / d->n_head;
  if (hd != 64 && hd != 128) return api_fail(FFAI_ERR_INVALID, "head_dim must be 64 or 128");
  if (d->seq > kMaxRows) return api_fail(FFAI_ERR_INVALID, "seq above 1500 frames per window is not enabled");
  return FFAI_OK;
}

// The windows of one pass: as many as fit kMaxRows rows (at least one; check() bounds seq).
int windows_per_pass(const ffai_encoder_attn_desc* d) {
  return (int)std::max<int64_t>(1, std::min<int64_t>(d->batch, kMaxRows / d->seq));
}

// The descriptor of a pass of `windows` windows.
ffai_encoder_attn_desc pass_desc(const ffai_encoder_attn_desc* d, int windows) {
  ffai_encoder_attn_desc p = *d;
  p.batch = windows;
  return p;
}

// `packed`: q, k and v side by side in one (B, S, 3N) buffer, K read as rows.
void attn_desc(const ffai_encoder_attn_desc* d, bool packed, ffai_attn_desc* a) {
  const int hd = d->n_state / d->n_head;
  const int64_t S = d->seq, N = d->n_state;
  ffai_attn_desc_init(a, d->dtype, d->dtype, d->dtype, d->batch, d->n_head, d->n_head, d->seq,
                      d->seq, hd, packed ? FFAI_K_ROWS : FFAI_K_TRANSPOSED);
  a->scale = 1.0f;  // head_dim^-0.5 is folded into wk_scaled
  const int64_t os[4] = {S * N, hd, N, 1};          // the merged output (and unpacked q, v): (B, S, N)
  const int64_t ps[4] = {S * 3 * N, hd, 3 * N, 1};  // packed q, k, v: (B, S, 3N)
  const int64_t BS = (int64_t)d->batch * S;
  const int64_t ks[4] = {S, (int64_t)hd * BS, BS, 1};   // kt: (N, B S) seen as (B, H, hd, S)
  std::memcpy(a->q_strides, packed ? ps : os, sizeof(os));
  std::memcpy(a->v_strides, packed ? ps : os, sizeof(os));
  std::memcpy(a->k_strides, packed ? ps : ks, sizeof(os));
  std::memcpy(a->o_strides, os, sizeof(os));
}

int sizes_of(const ffai_encoder_attn_desc* d, Sizes* z) {
  const size_t el = 2, act = (size_t)d->batch * d->seq * d->n_state * el;
  z->q = z->kt = z->v = z->merged = align256(act);
  size_t aw = 0;
  for (const bool packed : {false, true}) {
    ffai_attn_desc a;
    attn_desc(d, packed, &a);
    size_t b = 0;
    const int rc = ffai_attn_workspace_bytes(&a, &b);
    if (rc != FFAI_OK) return rc;
    aw = std::max(aw, b);
  }
  z->attn = align256(std::max(aw, ffai::kCounterBytes));
  z->gemm = kGemmScratch;
  z->total = z->q + z->kt + z->v + z->merged + z->attn + z->gemm;
  return FFAI_OK;
}

// The layout every pass of a call runs in: the first (fullest) pass's activation regions, which
// no shorter pass exceeds, and an attention region as large as the largest need of any pass. A
// shorter last pass can need more attention workspace than a full one: its grid is smaller, so
// the planner splits its keys into more pieces (whisper-large-v3 width, 6 windows of 300 frames:
// the 5-window pass needs no partials, the 1-window remainder ~6 MB).
int call_sizes(const ffai_encoder_attn_desc* d, Sizes* z) {
  const int wpp = windows_per_pass(d);
  const ffai_encoder_attn_desc first = pass_desc(d, wpp);
  int rc = sizes_of(&first, z);
  if (rc != FFAI_OK) return rc;
  if (const int rem = d->batch % wpp) {
    const ffai_encoder_attn_desc last = pass_desc(d, rem);
    Sizes zl;
    if ((rc = sizes_of(&last, &zl)) != FFAI_OK) return rc;
    z->total += std::max(z->attn, zl.attn) - z->attn;
    z->attn = std::max(z->attn, zl.attn);
  }
  return FFAI_OK;
}

}  // namespace

extern "C" {

int ffai_encoder_attn_workspace_bytes(const ffai_encoder_attn_desc* d, size_t* bytes) {
  api_clear_error();
  if (!bytes) return api_fail(FFAI_ERR_INVALID, "null bytes pointer");
  int rc = check(d);
  if (rc != FFAI_OK) return rc;
  Sizes z;
  rc = call_sizes(d, &z);
  if (rc != FFAI_OK) return rc;
  *bytes = z.total;
  return FFAI_OK;
}

}  // extern "C"

namespace {

// One pass: the windows of `d` (at most kMaxRows rows) through the workspace laid out by `z`.
int run_pass(const ffai_encoder_attn_desc* d, const void* x, const ffai_encoder_attn_weights* w,
             bool packed, void* out, void* workspace, const Sizes& z, hipblasLtHandle_t h,
             void* stream) {
  if ((int64_t)d->batch * d->seq > kMaxRows)
    return api_fail(FFAI_ERR_INVALID, "one pass holds at most 1500 rows");
  int rc = FFAI_OK;
  char* ws = static_cast<char*>(workspace);
  void* attn_ws = ws;
  void* q = ws + z.attn;
  void* kt = ws + z.attn + z.q;
  void* v = ws + z.attn + z.q + z.kt;
  void* merged = ws + z.attn + z.q + z.kt + z.v;
  void* scratch = ws + z.attn + z.q + z.kt + z.v + z.merged;
  const hipDataType dt = d->dtype == FFAI_BF16 ? HIP_R_16BF : HIP_R_16F;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t BS = (int64_t)d->batch * d->seq, N = d->n_state;

  // q, v: (B S, N) = x W^T + b  ->  D^T (N x BS) = W (op T) * x^T
  Gemm g{};
  g.ta = HIPBLAS_OP_T; g.tb = HIPBLAS_OP_N;
  g.m = N; g.n = BS; g.k = N;
  g.lda = N; g.ldb = N; g.ldd = N;
  g.b = x;
  ffai_attn_desc a;
  attn_desc(d, packed, &a);
  if (packed) {
    // qkv: (B S, 3N) = x Wqkv^T + bqkv  ->  D^T (3N x BS) = Wqkv (op T) * x^T; the regions of
    // q, kt and v are contiguous and hold it
    Gemm gp = g;
    gp.m = 3 * N; gp.ldd = 3 * N;
    gp.a = w->wqkv; gp.d = q; gp.bias = w->bqkv;
    if ((rc = run_gemm(h, gp, dt, scratch, z.gemm, st)) != FFAI_OK) return rc;
    const size_t es = 2;
    const char* qkv = static_cast<const char*>(q);
    if ((rc = ffai_attn_fwd(&a, qkv, qkv + N * es, qkv + 2 * N * es, merged, attn_ws, z.attn,
                            stream)) != FFAI_OK)
      return rc;
    g.b = merged; g.a = w->wo; g.d = out; g.bias = w->bo;
    return run_gemm(h, g, dt, scratch, z.gemm, st);
  }
  g.a = w->wq; g.d = q; g.bias = w->bq;
  if ((rc = run_gemm(h, g, dt, scratch, z.gemm, st)) != FFAI_OK) return rc;
  g.a = w->wv; g.d = v; g.bias = w->bv;
  if ((rc = run_gemm(h, g, dt, scratch, z.gemm, st)) != FFAI_OK) return rc;
  // kt: (N, B S) = Wk_s x^T  ->  column-major (B S x N) = x (op T, stored N x B S) * Wk_s^T
  // (stored N x N, op N)
  Gemm gk{};
  gk.ta = HIPBLAS_OP_T; gk.tb = HIPBLAS_OP_N;
  gk.m = BS; gk.n = N; gk.k = N;
  gk.a = x; gk.lda = N;
  gk.b = w->wk_scaled; gk.ldb = N;
  gk.d = kt; gk.ldd = BS;
  gk.bias = nullptr;
  if ((rc = run_gemm(h, gk, dt, scratch, z.gemm, st)) != FFAI_OK) return rc;
  // attention: reads q, kt, v by stride and writes the merged (B, S, N) layout
  if ((rc = ffai_attn_fwd(&a, q, kt, v, merged, attn_ws, z.attn, stream)) != FFAI_OK) return rc;
  // out: (B S, N) = merged Wo^T + bo
  g.b = merged; g.a = w->wo; g.d = out; g.bias = w->bo;
  return run_gemm(h, g, dt, scratch, z.gemm, st);
}

}  // namespace

extern "C" {

int ffai_encoder_attn_fwd(const ffai_encoder_attn_desc* d, const void* x,
                          const ffai_encoder_attn_weights* w, void* out, void* workspace,
                          size_t workspace_bytes, void* stream) {
  api_clear_error();
  int rc = check(d);
  if (rc != FFAI_OK) return rc;
  if (!x || !out || !w || !w->wo || !w->bo) return api_fail(FFAI_ERR_INVALID, "null pointer");
  const bool packed = w->wqkv && w->bqkv;
  if (!packed && (!w->wq || !w->bq || !w->wk_scaled || !w->wv || !w->bv))
    return api_fail(FFAI_ERR_INVALID, "null pointer (give wq, bq, wk_scaled, wv, bv or wqkv, bqkv)");
  const int wpp = windows_per_pass(d);
  Sizes z;
  if ((rc = call_sizes(d, &z)) != FFAI_OK) return rc;
  if (!workspace || workspace_bytes < z.total)
    return api_fail(FFAI_ERR_WORKSPACE, "workspace smaller than ffai_encoder_attn_workspace_bytes");
  if ((uintptr_t)workspace % 256) return api_fail(FFAI_ERR_INVALID, "workspace must be 256-byte aligned");
  if ((rc = api_check_device()) != FFAI_OK) return rc;
  hipblasLtHandle_t h;
  if ((rc = handle_for_current(&h)) != FFAI_OK) return rc;
  // passes in window order, stream-ordered through the one workspace (the reference's loop over
  // batch items); every pass uses the call's layout z, whose attention region holds the largest
  // need of any pass, so no pass is refused after an earlier one has written part of `out`
  const size_t window_bytes = (size_t)d->seq * d->n_state * 2;
  for (int b0 = 0; b0 < d->batch; b0 += wpp) {
    const ffai_encoder_attn_desc p = pass_desc(d, std::min(wpp, d->batch - b0));
    rc = run_pass(&p, static_cast<const char*>(x) + b0 * window_bytes, w, packed,
                  static_cast<char*>(out) + b0 * window_bytes, workspace, z, h, stream);
    if (rc != FFAI_OK) return rc;
  }
  return FFAI_OK;
}

}  // extern "C"
