// C ABI entry points (include/swvr.h): argument checks, error reporting,
// launch timing, and dispatch to the forward / backward launchers.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <cstddef>
#include <mutex>
#include <vector>

#include "../../include/swvr.h"
#include "launch.hpp"

namespace swvr {

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(SWVR_EHIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// ---- launch timing: event pairs per kernel kind, recorded on the launch stream
struct TimedLaunch {
  int kind;
  hipEvent_t start, stop;
};
std::mutex g_tmu;
bool g_timing = false;
std::vector<TimedLaunch> g_launches;
std::vector<hipEvent_t> g_pool;
// Start events of launches whose end is not yet recorded, keyed by (stream, kind):
// launches of one kind on different streams (or threads) pair their own events.
struct PendingLaunch {
  hipStream_t stream;
  int kind;
  hipEvent_t start;
};
std::vector<PendingLaunch> g_pending;

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

const char* kKindNames[kNumKinds] = {"fwd_tile_kernel",   "fwd_combine_kernel", "bwd_pack_kernel",
                                     "bwd_scores_kernel", "bwd_gemm_kernel",    "bwd_reduce_kernel",
                                     "fill_zero_kernel",  "operand_packing",    "bwd_expand_kernel",
                                     "mse_loss",          "quantize_e4m3",      "readout_f64",
                                     "probe_mfma"};

bool is_dtype(int d) { return d == SWVR_BF16 || d == SWVR_F16 || d == SWVR_F32; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h, int64_t ldh, const void* W,
                 int64_t ldw, const void* E, int64_t lde) {
  if (!is_dtype(dtype)) return fail(SWVR_EDTYPE, "unsupported operand dtype tag %d", dtype);
  if (N < 0 || K < 0 || V < 0 || D < 0) return fail(SWVR_EINVAL, "negative size N=%lld K=%lld V=%lld D=%lld",
                                                    (long long)N, (long long)K, (long long)V, (long long)D);
  if (N > INT32_MAX || K > INT32_MAX || V > INT32_MAX || D > INT32_MAX)
    return fail(SWVR_EINVAL, "sizes must fit in 32 bits");
  if (D > swvr_max_d(dtype))
    return fail(SWVR_EDTYPE, "D=%lld exceeds the maximum %lld for this dtype", (long long)D,
                (long long)swvr_max_d(dtype));
  if (K % 8 != 0) return fail(SWVR_EINVAL, "K=%lld must be a multiple of 8 (pad h and W)", (long long)K);
  // tile-relative byte offsets of the kernels are 32-bit: 128 rows x K fp32 stay below 2^31
  if (K > (int64_t)1 << 21) return fail(SWVR_EINVAL, "K=%lld exceeds the maximum %lld", (long long)K, 1LL << 21);
  if (ldh < K || ldh % 8 != 0) return fail(SWVR_EINVAL, "ldh=%lld must be >= K and a multiple of 8", (long long)ldh);
  if (ldw < K || ldw % 8 != 0) return fail(SWVR_EINVAL, "ldw=%lld must be >= K and a multiple of 8", (long long)ldw);
  if (lde < D) return fail(SWVR_EINVAL, "lde=%lld must be >= D", (long long)lde);
  if (N > 0 && K > 0 && (!h || !aligned16(h))) return fail(SWVR_EINVAL, "h must be a non-null 16-byte aligned pointer");
  if (V > 0 && K > 0 && (!W || !aligned16(W))) return fail(SWVR_EINVAL, "W must be a non-null 16-byte aligned pointer");
  if (V > 0 && D > 0 && !E) return fail(SWVR_EINVAL, "E must be non-null");
  return SWVR_OK;
}

}  // namespace

void timing_begin(int kind, hipStream_t stream) {
  if (!g_timing) return;
  std::lock_guard<std::mutex> lk(g_tmu);
  hipEvent_t e = take_event();
  if (e && hipEventRecord(e, stream) == hipSuccess) g_pending.push_back({stream, kind, e});
}

void timing_end(int kind, hipStream_t stream) {
  if (!g_timing) return;
  std::lock_guard<std::mutex> lk(g_tmu);
  // the latest unmatched start of this kind on this stream
  for (size_t i = g_pending.size(); i-- > 0;) {
    if (g_pending[i].stream != stream || g_pending[i].kind != kind) continue;
    const hipEvent_t s = g_pending[i].start;
    g_pending.erase(g_pending.begin() + (std::ptrdiff_t)i);
    hipEvent_t e = take_event();
    if (e && hipEventRecord(e, stream) == hipSuccess)
      g_launches.push_back({kind, s, e});
    else
      g_pool.push_back(s);
    return;
  }
}

namespace {

// Storage dtype of h or W: the compute dtype, or fp32 under a 2-byte compute dtype.
int check_storage(int dtype, int h_dtype, int w_dtype) {
  const bool two = dtype == SWVR_BF16 || dtype == SWVR_F16;
  if (!(h_dtype == dtype || (two && h_dtype == SWVR_F32)))
    return fail(SWVR_EDTYPE, "h dtype tag %d with compute dtype %d", h_dtype, dtype);
  if (!(w_dtype == dtype || (two && w_dtype == SWVR_F32)))
    return fail(SWVR_EDTYPE, "W dtype tag %d with compute dtype %d", w_dtype, dtype);
  return SWVR_OK;
}

int fwd_common(int dtype, int h_dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h,
               int64_t ldh, const void* W, int64_t ldw, const void* E, int64_t lde, const float* bias,
               float logit_scale, float* O, float* lse, float* m_out, float* l_out, void* workspace,
               size_t workspace_bytes, void* stream, bool active = false, const float* weight = nullptr) {
  g_err[0] = 0;
  int rc = check_common(dtype, N, K, V, D, h, ldh, W, ldw, E, lde);
  if (rc != SWVR_OK) return rc;
  if ((rc = check_storage(dtype, h_dtype, w_dtype)) != SWVR_OK) return rc;
  if (N > 0 && ((D > 0 && !O) || (m_out ? !l_out : !lse)))
    return fail(SWVR_EINVAL, m_out ? "m, l and acc must be non-null" : "O and lse must be non-null");
  FwdPlan plan;
  if (!fwd_plan(dtype, N, K, V, D, &plan, active))
    return fail(SWVR_EDTYPE, "no forward kernel for dtype %d, D=%lld", dtype, (long long)D);
  if (N == 0) return SWVR_OK;
  if (!workspace || workspace_bytes < plan.ws_bytes)
    return fail(SWVR_EWORKSPACE, "forward workspace of %zu bytes needed, %zu given", plan.ws_bytes, workspace_bytes);
  FwdParams p{};
  p.h = h;
  p.ldh = ldh;
  p.W = W;
  p.ldw = ldw;
  p.E = E;
  p.lde = lde;
  p.bias = bias;
  p.scale = logit_scale;
  p.N = (int)N;
  p.K = (int)K;
  p.V = (int)V;
  p.D = (int)D;
  p.h_f32 = h_dtype != dtype;
  p.w_f32 = w_dtype != dtype;
  hipError_t e = active ? fwd_launch_active(dtype, plan, p, weight, static_cast<char*>(workspace), O, lse,
                                            static_cast<hipStream_t>(stream))
                        : fwd_launch(dtype, plan, p, static_cast<char*>(workspace), O, lse, m_out, l_out,
                                     static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "forward launch");
  return SWVR_OK;
}

int bwd_common(int dtype, int h_dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h,
                   int64_t ldh, const void* W, int64_t ldw, const void* E, int64_t lde, const float* bias,
                   float logit_scale, const float* O, const float* lse, const float* gO, const float* glse,
                   int64_t chunk, void* gh, int gh_dtype, void* gW, int gW_dtype, void* gE, int gE_dtype, float* gb,
                   void* workspace, size_t workspace_bytes, void* stream, const void* hq = nullptr,
                   int64_t K8 = 0, int64_t ldhq = 0, const float* h_scale = nullptr, const void* Wq = nullptr,
                   int64_t ldwq = 0, const float* w_scale = nullptr) {
  g_err[0] = 0;
  int rc = check_common(dtype, N, K, V, D, h, ldh, W, ldw, E, lde);
  if (rc != SWVR_OK) return rc;
  if ((rc = check_storage(dtype, h_dtype, w_dtype)) != SWVR_OK) return rc;
  if (chunk <= 0) return fail(SWVR_EINVAL, "chunk must be positive, got %lld", (long long)chunk);
  if (gh && !is_dtype(gh_dtype)) return fail(SWVR_EDTYPE, "unsupported gh dtype tag %d", gh_dtype);
  if (gW && !is_dtype(gW_dtype)) return fail(SWVR_EDTYPE, "unsupported gW dtype tag %d", gW_dtype);
  if (gE && !is_dtype(gE_dtype)) return fail(SWVR_EDTYPE, "unsupported gE dtype tag %d", gE_dtype);
  if (gb && !bias) return fail(SWVR_EINVAL, "gb requested without a bias");
  if (N > 0 && (!lse || !glse || (D > 0 && (!O || !gO)))) return fail(SWVR_EINVAL, "O, lse, gO and glse must be non-null");
  BwdPlan plan;
  if (!bwd_plan(dtype, N, K, V, D, chunk, gh != nullptr, &plan, w_dtype != dtype, hq ? K8 : 0))
    return fail(SWVR_EDTYPE, "no backward kernel for dtype %d, D=%lld", dtype, (long long)D);
  if (N > 0 && (!workspace || workspace_bytes < plan.ws_bytes))
    return fail(SWVR_EWORKSPACE, "backward workspace of %zu bytes needed, %zu given", plan.ws_bytes, workspace_bytes);
  BwdParams p{};
  p.h = h;
  p.ldh = ldh;
  p.W = W;
  p.ldw = ldw;
  p.E = E;
  p.lde = lde;
  p.bias = bias;
  p.scale = logit_scale;
  p.N = (int)N;
  p.K = (int)K;
  p.V = (int)V;
  p.D = (int)D;
  p.O = O;
  p.lse = lse;
  p.gO = gO;
  p.glse = glse;
  p.gh = gh;
  p.gh_dtype = gh_dtype;
  p.gW = gW;
  p.gW_dtype = gW_dtype;
  p.gE = gE;
  p.gE_dtype = gE_dtype;
  p.gb = gb;
  p.ws = static_cast<char*>(workspace);
  p.h_f32 = h_dtype != dtype;
  p.w_f32 = w_dtype != dtype;
  p.hq = hq;
  p.ldhq = ldhq;
  p.Wq = Wq;
  p.ldwq = ldwq;
  p.h_scale = h_scale;
  p.w_scale = w_scale;
  p.K8 = (int)K8;
  hipError_t e = bwd_launch(dtype, plan, p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "backward launch");
  return SWVR_OK;
}

}  // namespace

}  // namespace swvr

using namespace swvr;

extern "C" {

int swvr_abi_version(void) { return SWVR_ABI_VERSION; }

const char* swvr_last_error(void) { return g_err; }

int64_t swvr_max_d(int dtype) {
  if (dtype == SWVR_F32 || dtype == SWVR_BF16 || dtype == SWVR_F16) return SWVR_MAX_D;
  return 0;
}

size_t swvr_fwd_workspace_size(int dtype, int64_t N, int64_t K, int64_t V, int64_t D) {
  FwdPlan plan;
  if (N < 0 || V < 0 || D < 0 || !fwd_plan(dtype, N, K, V, D, &plan)) return 0;
  return plan.ws_bytes;
}

int swvr_fwd(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h, int64_t ldh, const void* W,
             int64_t ldw, const void* E, int64_t lde, const float* bias, float logit_scale, float* O, float* lse,
             void* workspace, size_t workspace_bytes, void* stream) {
  return fwd_common(dtype, dtype, dtype, N, K, V, D, h, ldh, W, ldw, E, lde, bias, logit_scale, O, lse, nullptr,
                    nullptr, workspace, workspace_bytes, stream);
}

int swvr_fwd_mixed(int dtype, int h_dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h,
                   int64_t ldh, const void* W, int64_t ldw, const void* E, int64_t lde, const float* bias,
                   float logit_scale, float* O, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return fwd_common(dtype, h_dtype, w_dtype, N, K, V, D, h, ldh, W, ldw, E, lde, bias, logit_scale, O, lse, nullptr,
                    nullptr, workspace, workspace_bytes, stream);
}

size_t swvr_fwd_active_workspace_size(int dtype, int64_t N, int64_t K, int64_t V, int64_t D) {
  FwdPlan plan;
  if (N < 0 || V < 0 || D < 0 || !fwd_plan(dtype, N, K, V, D, &plan, true)) return 0;
  return plan.ws_bytes;
}

int swvr_fwd_active(int dtype, int h_dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h,
                    int64_t ldh, const void* W, int64_t ldw, const void* E, int64_t lde, const float* bias,
                    float logit_scale, const float* weight, float* O, float* lse, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (N > 0 && !weight) {
    g_err[0] = 0;
    return fail(SWVR_EINVAL, "weight must be non-null");
  }
  return fwd_common(dtype, h_dtype, w_dtype, N, K, V, D, h, ldh, W, ldw, E, lde, bias, logit_scale, O, lse, nullptr,
                    nullptr, workspace, workspace_bytes, stream, true, weight);
}

int swvr_fwd_partial(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h, int64_t ldh,
                     const void* W, int64_t ldw, const void* E, int64_t lde, const float* bias, float logit_scale,
                     float* m, float* l, float* acc, void* workspace, size_t workspace_bytes, void* stream) {
  if (!m && N > 0) {
    g_err[0] = 0;
    return fail(SWVR_EINVAL, "m, l and acc must be non-null");
  }
  return fwd_common(dtype, dtype, dtype, N, K, V, D, h, ldh, W, ldw, E, lde, bias, logit_scale, acc, nullptr, m, l,
                    workspace, workspace_bytes, stream);
}

int swvr_combine(int64_t S, int64_t N, int64_t D, const float* m, const float* l, const float* acc, float* O,
                 float* lse, void* stream) {
  g_err[0] = 0;
  if (S < 1 || N < 0 || D < 0) return fail(SWVR_EINVAL, "bad sizes S=%lld N=%lld D=%lld", (long long)S, (long long)N,
                                           (long long)D);
  if (S > INT32_MAX || N > INT32_MAX || D > INT32_MAX) return fail(SWVR_EINVAL, "sizes must fit in 32 bits");
  if (N == 0) return SWVR_OK;
  if (!m || !l || !lse || (D > 0 && (!acc || !O))) return fail(SWVR_EINVAL, "m, l, acc, O and lse must be non-null");
  hipError_t e = shard_combine((int)S, (int)N, (int)D, m, l, acc, O, lse, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "combine launch");
  return SWVR_OK;
}

size_t swvr_bwd_workspace_size_mixed(int dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D,
                                     int64_t chunk, int need_gh) {
  BwdPlan plan;
  if (N < 0 || V < 0 || D < 0 || chunk <= 0 ||
      !bwd_plan(dtype, N, K, V, D, chunk, need_gh != 0, &plan, w_dtype != dtype))
    return 0;
  return plan.ws_bytes;
}

size_t swvr_bwd_workspace_size(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, int64_t chunk, int need_gh) {
  return swvr_bwd_workspace_size_mixed(dtype, dtype, N, K, V, D, chunk, need_gh);
}

int swvr_bwd_tiling(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, int64_t chunk, int64_t* out, int n_out) {
  g_err[0] = 0;
  if (!out || n_out < 0) return fail(SWVR_EINVAL, "out must be non-null");
  BwdPlan plan;
  if (N < 0 || K < 0 || V < 0 || D < 0 || chunk <= 0)
    return fail(SWVR_EINVAL, "bad sizes N=%lld K=%lld V=%lld D=%lld chunk=%lld", (long long)N, (long long)K,
                (long long)V, (long long)D, (long long)chunk);
  if (!bwd_plan(dtype, N, K, V, D, chunk, true, &plan))
    return fail(SWVR_EDTYPE, "no backward kernel for dtype %d, D=%lld", dtype, (long long)D);
  const int64_t v[7] = {plan.BM, plan.BV, plan.G, plan.C, plan.n_chunks, plan.DP, plan.kind};
  const int n = n_out < 7 ? n_out : 7;
  for (int i = 0; i < n; ++i) out[i] = v[i];
  return 7;
}

int swvr_bwd_mixed(int dtype, int h_dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h,
                   int64_t ldh, const void* W, int64_t ldw, const void* E, int64_t lde, const float* bias,
                   float logit_scale, const float* O, const float* lse, const float* gO, const float* glse,
                   int64_t chunk, void* gh, int gh_dtype, void* gW, int gW_dtype, void* gE, int gE_dtype, float* gb,
                   void* workspace, size_t workspace_bytes, void* stream) {
  return bwd_common(dtype, h_dtype, w_dtype, N, K, V, D, h, ldh, W, ldw, E, lde, bias, logit_scale, O, lse, gO, glse,
                    chunk, gh, gh_dtype, gW, gW_dtype, gE, gE_dtype, gb, workspace, workspace_bytes, stream);
}

size_t swvr_bwd_fp8_workspace_size(int64_t N, int64_t K, int64_t K8, int64_t V, int64_t D, int64_t chunk,
                                   int need_gh) {
  BwdPlan plan;
  if (N < 0 || V < 0 || D < 0 || chunk <= 0 || K8 <= 0 ||
      !bwd_plan(SWVR_BF16, N, K, V, D, chunk, need_gh != 0, &plan, false, K8))
    return 0;
  return plan.ws_bytes;
}

int swvr_bwd_fp8(int64_t N, int64_t K, int64_t V, int64_t D, const void* h, int64_t ldh, const void* W, int64_t ldw,
                 const void* E, int64_t lde, const float* bias, float logit_scale, const void* hq, int64_t K8,
                 int64_t ldhq, const float* h_scale, const void* Wq, int64_t ldwq, const float* w_scale,
                 const float* O, const float* lse, const float* gO, const float* glse, int64_t chunk, void* gh,
                 int gh_dtype, void* gW, int gW_dtype, void* gE, int gE_dtype, float* gb, void* workspace,
                 size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  if (D > 128) return fail(SWVR_EDTYPE, "D=%lld exceeds the maximum 128 of the e4m3 scores", (long long)D);
  if (K8 < K || K8 % 16 != 0 || ldhq < K8 || ldhq % 16 != 0 || ldwq < K8 || ldwq % 16 != 0)
    return fail(SWVR_EINVAL, "K8=%lld (>= K), ldhq=%lld and ldwq=%lld (>= K8) must be multiples of 16",
                (long long)K8, (long long)ldhq, (long long)ldwq);
  if (K8 > ((int64_t)1 << 22)) return fail(SWVR_EINVAL, "K8=%lld too large", (long long)K8);
  if (N > 0 && V > 0 && (!hq || !Wq || !h_scale || !w_scale || !aligned16(hq) || !aligned16(Wq)))
    return fail(SWVR_EINVAL, "hq, Wq (16-byte aligned), h_scale and w_scale must be non-null");
  return bwd_common(SWVR_BF16, SWVR_BF16, SWVR_BF16, N, K, V, D, h, ldh, W, ldw, E, lde, bias, logit_scale, O, lse,
                    gO, glse, chunk, gh, gh_dtype, gW, gW_dtype, gE, gE_dtype, gb, workspace, workspace_bytes, stream,
                    hq, K8, ldhq, h_scale, Wq, ldwq, w_scale);
}

int swvr_bwd(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, const void* h, int64_t ldh, const void* W,
             int64_t ldw, const void* E, int64_t lde, const float* bias, float logit_scale, const float* O,
             const float* lse, const float* gO, const float* glse, int64_t chunk, void* gh, int gh_dtype, void* gW,
             int gW_dtype, void* gE, int gE_dtype, float* gb, void* workspace, size_t workspace_bytes,
             void* stream) {
  return swvr_bwd_mixed(dtype, dtype, dtype, N, K, V, D, h, ldh, W, ldw, E, lde, bias, logit_scale, O, lse, gO, glse,
                        chunk, gh, gh_dtype, gW, gW_dtype, gE, gE_dtype, gb, workspace, workspace_bytes, stream);
}

int swvr_timing_enable(int on) {
  std::lock_guard<std::mutex> lk(g_tmu);
  g_timing = on != 0;
  return SWVR_OK;
}

int swvr_timing_collect(double* total_ms, int64_t* launches, int max_kinds) {
  std::lock_guard<std::mutex> lk(g_tmu);
  std::vector<double> ms(kNumKinds, 0.0);
  std::vector<int64_t> cnt(kNumKinds, 0);
  int rc = SWVR_OK;
  for (const TimedLaunch& t : g_launches) {
    hipError_t e = hipEventSynchronize(t.stop);
    float f = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&f, t.start, t.stop);
    if (e != hipSuccess && rc == SWVR_OK) rc = hip_fail(e, "timing event");
    ms[t.kind] += f;
    cnt[t.kind] += 1;
    g_pool.push_back(t.start);
    g_pool.push_back(t.stop);
  }
  g_launches.clear();
  if (rc != SWVR_OK) return rc;
  const int n = max_kinds < kNumKinds ? max_kinds : kNumKinds;
  for (int k = 0; k < n; ++k) {
    if (total_ms) total_ms[k] = ms[k];
    if (launches) launches[k] = cnt[k];
  }
  return kNumKinds;
}

size_t swvr_fwd_fp8_workspace_size(int64_t N, int64_t K, int64_t V, int64_t D) {
  if (N < 0 || K < 0 || V < 0 || D < 0 || K % 16 != 0 || N > INT32_MAX || V > INT32_MAX) return 0;
  FwdPlan plan;
  if (!fwd_plan(kFwdFP8, N, K / 2, V, D, &plan)) return 0;
  return plan.ws_bytes;
}

int swvr_fwd_fp8(int64_t N, int64_t K, int64_t V, int64_t D, const void* h, int64_t ldh, const float* h_scale,
                 const void* W, int64_t ldw, const float* w_scale, const void* E, int64_t lde, const float* bias,
                 float logit_scale, float* O, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  if (D > 128) return fail(SWVR_EDTYPE, "D=%lld exceeds the maximum 128 of the e4m3 forward", (long long)D);
  if (K % 16 != 0 || ldh % 16 != 0 || ldw % 16 != 0)
    return fail(SWVR_EINVAL, "K=%lld, ldh=%lld and ldw=%lld must be multiples of 16 (e4m3 bytes)", (long long)K,
                (long long)ldh, (long long)ldw);
  // the e4m3 rows travel as bf16 rows of K / 2 elements
  int rc = check_common(SWVR_BF16, N, K / 2, V, D, h, ldh / 2, W, ldw / 2, E, lde);
  if (rc != SWVR_OK) return rc;
  if (N > 0 && (!O || !lse)) return fail(SWVR_EINVAL, "O and lse must be non-null");
  if (N > 0 && V > 0 && (!h_scale || !w_scale)) return fail(SWVR_EINVAL, "h_scale and w_scale must be non-null");
  FwdPlan plan;
  if (!fwd_plan(kFwdFP8, N, K / 2, V, D, &plan)) return fail(SWVR_EDTYPE, "no e4m3 forward kernel for D=%lld", (long long)D);
  if (N == 0) return SWVR_OK;
  if (!workspace || workspace_bytes < plan.ws_bytes)
    return fail(SWVR_EWORKSPACE, "forward workspace of %zu bytes needed, %zu given", plan.ws_bytes, workspace_bytes);
  FwdParams p{};
  p.h = h;
  p.ldh = ldh / 2;
  p.W = W;
  p.ldw = ldw / 2;
  p.E = E;
  p.lde = lde;
  p.bias = bias;
  p.scale = logit_scale;
  p.N = (int)N;
  p.K = (int)(K / 2);
  p.V = (int)V;
  p.D = (int)D;
  p.h_scale = h_scale;
  p.w_scale = w_scale;
  hipError_t e = fwd_launch(kFwdFP8, plan, p, static_cast<char*>(workspace), O, lse, nullptr, nullptr,
                            static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "forward launch");
  return SWVR_OK;
}

static int check_f64(int64_t N, int64_t K, int64_t V, int64_t D, const double* h, int64_t ldh, const double* W,
                     int64_t ldw, const double* E, int64_t lde, int64_t chunk) {
  if (N < 0 || K < 0 || V < 0 || D < 0) return fail(SWVR_EINVAL, "negative size N=%lld K=%lld V=%lld D=%lld",
                                                    (long long)N, (long long)K, (long long)V, (long long)D);
  if (N > INT32_MAX || K > INT32_MAX || V > INT32_MAX || D > SWVR_MAX_D)
    return fail(SWVR_EINVAL, "sizes must fit in 32 bits and D in SWVR_MAX_D");
  if (K >= ((int64_t)1 << 22)) return fail(SWVR_EINVAL, "K=%lld must be below 2^22", (long long)K);
  if (chunk <= 0) return fail(SWVR_EINVAL, "chunk must be positive, got %lld", (long long)chunk);
  if (ldh < K || ldw < K || lde < D) return fail(SWVR_EINVAL, "ldh, ldw must be >= K and lde >= D");
  if (N > 0 && K > 0 && !h) return fail(SWVR_EINVAL, "h must be non-null");
  if (V > 0 && K > 0 && !W) return fail(SWVR_EINVAL, "W must be non-null");
  if (V > 0 && D > 0 && !E) return fail(SWVR_EINVAL, "E must be non-null");
  return SWVR_OK;
}

size_t swvr_fwd_f64_workspace_size(int64_t N, int64_t V, int64_t D, int64_t chunk) {
  if (N < 0 || V < 0 || D < 0 || chunk <= 0) return 0;
  int64_t C;
  size_t fb;
  swvr::f64_plan(N, V, D, chunk, &C, &fb, nullptr);
  return fb;
}

int swvr_fwd_f64(int64_t N, int64_t K, int64_t V, int64_t D, const double* h, int64_t ldh, const double* W,
                 int64_t ldw, const double* E, int64_t lde, const double* bias, double logit_scale, int64_t chunk,
                 double* O, double* lse, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check_f64(N, K, V, D, h, ldh, W, ldw, E, lde, chunk);
  if (rc != SWVR_OK) return rc;
  if (N == 0) return SWVR_OK;
  if (!lse || (D > 0 && !O)) return fail(SWVR_EINVAL, "O and lse must be non-null");
  const size_t need = swvr_fwd_f64_workspace_size(N, V, D, chunk);
  if (!workspace || workspace_bytes < need)
    return fail(SWVR_EWORKSPACE, "fp64 forward workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  swvr::F64Params p{};
  p.h = h;
  p.ldh = ldh;
  p.W = W;
  p.ldw = ldw;
  p.E = E;
  p.lde = lde;
  p.bias = bias;
  p.scale = logit_scale;
  p.N = (int)N;
  p.K = (int)K;
  p.V = (int)V;
  p.D = (int)D;
  p.chunk = chunk;
  p.O = O;
  p.lse = lse;
  p.ws = static_cast<char*>(workspace);
  hipError_t e = swvr::f64_fwd(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "fp64 forward launch");
  return SWVR_OK;
}

size_t swvr_bwd_f64_workspace_size(int64_t N, int64_t V, int64_t D, int64_t chunk) {
  if (N < 0 || V < 0 || D < 0 || chunk <= 0) return 0;
  int64_t C;
  size_t bb;
  swvr::f64_plan(N, V, D, chunk, &C, nullptr, &bb);
  return bb;
}

int swvr_bwd_f64(int64_t N, int64_t K, int64_t V, int64_t D, const double* h, int64_t ldh, const double* W,
                 int64_t ldw, const double* E, int64_t lde, const double* bias, double logit_scale, const double* O,
                 const double* lse, const double* gO, const double* glse, int64_t chunk, double* gh, double* gW,
                 double* gE, double* gb, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check_f64(N, K, V, D, h, ldh, W, ldw, E, lde, chunk);
  if (rc != SWVR_OK) return rc;
  if (gb && !bias) return fail(SWVR_EINVAL, "gb requested without a bias");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (N > 0 && (!lse || !glse || (D > 0 && (!O || !gO))))
    return fail(SWVR_EINVAL, "O, lse, gO and glse must be non-null");
  const size_t need = swvr_bwd_f64_workspace_size(N, V, D, chunk);
  if (N > 0 && (!workspace || workspace_bytes < need))
    return fail(SWVR_EWORKSPACE, "fp64 backward workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  swvr::F64Params p{};
  p.h = h;
  p.ldh = ldh;
  p.W = W;
  p.ldw = ldw;
  p.E = E;
  p.lde = lde;
  p.bias = bias;
  p.scale = logit_scale;
  p.N = (int)N;
  p.K = (int)K;
  p.V = (int)V;
  p.D = (int)D;
  p.chunk = chunk;
  p.O = const_cast<double*>(O);
  p.lse = const_cast<double*>(lse);
  p.gO = gO;
  p.glse = glse;
  p.gh = gh;
  p.gW = gW;
  p.gE = gE;
  p.gb = gb;
  p.ws = static_cast<char*>(workspace);
  hipError_t e = swvr::f64_bwd(p, s);
  if (e != hipSuccess) return hip_fail(e, "fp64 backward launch");
  return SWVR_OK;
}

int swvr_probe_mfma(int64_t workgroups, int64_t iters, int mode, float* out, void* stream) {
  g_err[0] = 0;
  if (workgroups < 1 || workgroups > (1 << 20) || iters < 1 || iters > (1 << 24) || mode < 0 || mode > 8)
    return fail(SWVR_EINVAL, "probe: workgroups in [1, 2^20], iters in [1, 2^24], mode 0 to 8");
  if (!out) return fail(SWVR_EINVAL, "out must be non-null");
  hipError_t e = swvr::probe_mfma((int)workgroups, (int)iters, mode, out, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "probe launch");
  return SWVR_OK;
}

size_t swvr_quantize_e4m3_workspace_size(int64_t R, int per_row) {
  if (R < 0 || R > INT32_MAX) return 0;
  return per_row ? 0 : (size_t)R * sizeof(float);
}

int swvr_quantize_e4m3(int64_t R, int64_t K, int64_t Kp, const void* x, int64_t ld, int x_dtype, int per_row,
                       void* out, int64_t ldo, float* scale, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  if (R < 0 || K < 0 || Kp < K || R > INT32_MAX || Kp > INT32_MAX)
    return fail(SWVR_EINVAL, "bad sizes R=%lld K=%lld Kp=%lld", (long long)R, (long long)K, (long long)Kp);
  if (Kp % 16 != 0) return fail(SWVR_EINVAL, "Kp=%lld must be a multiple of 16", (long long)Kp);
  if (!is_dtype(x_dtype)) return fail(SWVR_EDTYPE, "unsupported input dtype tag %d", x_dtype);
  if (ld < K || ldo < Kp || ldo % 16 != 0)
    return fail(SWVR_EINVAL, "ld=%lld must be >= K, ldo=%lld >= Kp and a multiple of 16", (long long)ld,
                (long long)ldo);
  if (R == 0) return SWVR_OK;
  if ((K > 0 && !x) || !out || !scale || !aligned16(out)) return fail(SWVR_EINVAL, "x, out (16-byte aligned) and scale must be non-null");
  const size_t need = swvr_quantize_e4m3_workspace_size(R, per_row);
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(SWVR_EWORKSPACE, "quantisation workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  swvr::QuantParams q{};
  q.x = x;
  q.ld = ld;
  q.x_dtype = x_dtype;
  q.R = (int)R;
  q.K = (int)K;
  q.Kp = (int)Kp;
  q.per_row = per_row != 0;
  q.out = out;
  q.ldo = ldo;
  q.scale = scale;
  q.amax = static_cast<float*>(workspace);
  hipError_t e = swvr::quant_launch(q, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "quantisation launch");
  return SWVR_OK;
}

size_t swvr_mse_loss_workspace_size(int64_t N) {
  if (N < 0 || N > INT32_MAX) return 0;
  return swvr::mse_workspace_bytes((int)N);
}

int swvr_mse_loss(int64_t N, int64_t D, const float* O, const float* lse, const void* target, int target_dtype,
                  int64_t ldt, const float* weight, float z_loss_weight, int reduction, float* out, float* scale,
                  float* gO, float* glse, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  if (N < 0 || D < 1) return fail(SWVR_EINVAL, "bad sizes N=%lld D=%lld", (long long)N, (long long)D);
  if (N > INT32_MAX || D > INT32_MAX || N * D > ((int64_t)1 << 40)) return fail(SWVR_EINVAL, "sizes too large");
  if (!is_dtype(target_dtype)) return fail(SWVR_EDTYPE, "unsupported target dtype tag %d", target_dtype);
  if (reduction < SWVR_REDUCE_NONE || reduction > SWVR_REDUCE_MEAN)
    return fail(SWVR_EINVAL, "unknown reduction %d", reduction);
  if (ldt < D) return fail(SWVR_EINVAL, "ldt=%lld must be >= D", (long long)ldt);
  if (reduction == SWVR_REDUCE_NONE && N == 0) return SWVR_OK;  // nothing to write
  if (!out) return fail(SWVR_EINVAL, "out must be non-null");
  if ((gO == nullptr) != (glse == nullptr)) return fail(SWVR_EINVAL, "gO and glse must both be given or both NULL");
  if (N > 0 && (!O || !lse || !target)) return fail(SWVR_EINVAL, "O, lse and target must be non-null");
  const size_t need = reduction == SWVR_REDUCE_NONE ? 0 : swvr::mse_workspace_bytes((int)N);
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(SWVR_EWORKSPACE, "loss workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  swvr::MseParams p{};
  p.O = O;
  p.lse = lse;
  p.target = target;
  p.ldt = ldt;
  p.target_dtype = target_dtype;
  p.weight = weight;
  p.N = (int)N;
  p.D = (int)D;
  p.z = z_loss_weight;
  p.reduce = reduction;
  p.per_tok = reduction == SWVR_REDUCE_NONE ? out : nullptr;
  p.out = reduction == SWVR_REDUCE_NONE ? nullptr : out;
  p.scale = scale;
  p.gO = gO;
  p.glse = glse;
  hipError_t e = swvr::mse_launch(p, workspace, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "loss launch");
  return SWVR_OK;
}

int swvr_mse_loss_noalloc(int64_t N, int64_t D, const float* O, const float* lse, const void* target,
                          int target_dtype, int64_t ldt, const float* weight, float z_loss_weight, int reduction,
                          float* out, float* scale, float* gO, float* glse, void* stream) {
  g_err[0] = 0;
  static_assert(SWVR_MSE_NOALLOC_MAX_N == swvr::kMseNoAllocMaxTokens, "one limit");
  if (N > SWVR_MSE_NOALLOC_MAX_N)
    return fail(SWVR_EINVAL, "N=%lld exceeds the maximum %d of swvr_mse_loss_noalloc (use swvr_mse_loss)",
                (long long)N, SWVR_MSE_NOALLOC_MAX_N);
  void* ws = nullptr;
  size_t ws_bytes = 0;
  if (N > 0 && reduction != SWVR_REDUCE_NONE) {
    const hipError_t e = swvr::mse_noalloc_scratch(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return hip_fail(e, "scratch address");
    ws_bytes = swvr::mse_workspace_bytes((int)N);
  }
  return swvr_mse_loss(N, D, O, lse, target, target_dtype, ldt, weight, z_loss_weight, reduction, out, scale, gO,
                       glse, ws, ws_bytes, stream);
}

const char* swvr_kernel_name(int kind) {
  if (kind < 0 || kind >= kNumKinds) return "";
  return kKindNames[kind];
}

}  // extern "C"
