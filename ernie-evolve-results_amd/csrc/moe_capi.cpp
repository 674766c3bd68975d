// extern "C" entry points of libmoe_route.so (declared in include/moe_route.h).
//
// Every entry point validates its arguments on the host -- the role
// TORCH_CHECK plays in the reference's run() (K:4088, K:4331-4338) -- and
// only then enqueues kernels on the caller's stream.  Nothing here allocates
// device memory or synchronises: scratch space is the caller's workspace
// (the reference's per-call arena, K:4197-4268, becomes a caller-owned
// buffer whose size moe_*_workspace_bytes reports).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/moe_route.h"
#include "moe_common.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return MOE_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess)
    return fail(MOE_ERR_LAUNCH, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return ok();
}

bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Largest T*H / 8 (16-byte vectors per tensor) the 32-bit element loops take.
constexpr long long kMaxVectors = (1ll << 31) - (1ll << 25);

bool supported_e(int E) {
  return E == 8 || E == 16 || E == 32 || E == 64 || E == 128 || E == 256;
}

int check_cfg(const moe_route_cfg* cfg, int E, int k) {
  if (!cfg) return fail(MOE_ERR_NULL_POINTER, "cfg is NULL");
  if (cfg->scoring < MOE_SCORING_SOFTMAX || cfg->scoring > MOE_SCORING_SOFTMAX_BIAS)
    return fail(MOE_ERR_INVALID_ARG, "unknown scoring rule %d", cfg->scoring);
  if (cfg->scoring == MOE_SCORING_SIGMOID_GROUP && cfg->n_group > 1) {
    const int ng = cfg->n_group;
    if (!pow2(ng) || E % ng != 0)
      return fail(MOE_ERR_INVALID_ARG, "n_group=%d must be a power of two dividing E=%d", ng, E);
    const int gs = E / ng;
    const int V = moe::topk_lane_width(E, cfg->scoring, ng);
    if (gs < 2 || E / V > 64)
      return fail(MOE_ERR_UNSUPPORTED, "group size %d (E=%d, n_group=%d) below %d experts", gs,
                  E, ng, gs < 2 ? 2 : E / 64);
    if (cfg->topk_group < 1 || cfg->topk_group > ng)
      return fail(MOE_ERR_INVALID_ARG, "topk_group=%d not in [1, n_group=%d]", cfg->topk_group,
                  ng);
    if ((long long)cfg->topk_group * gs < k)
      return fail(MOE_ERR_INVALID_ARG, "topk_group*group_size=%d < k=%d", cfg->topk_group * gs,
                  k);
  } else if (cfg->n_group < 1) {
    return fail(MOE_ERR_INVALID_ARG, "n_group=%d < 1", cfg->n_group);
  }
  return MOE_OK;
}

int check_topk_shape(int T, int E, int k) {
  if (T < 0) return fail(MOE_ERR_INVALID_ARG, "T=%d < 0", T);
  if (!supported_e(E))
    return fail(MOE_ERR_UNSUPPORTED, "E=%d not in {8,16,32,64,128,256}", E);
  if (k < 1 || k > 8 || k > E) return fail(MOE_ERR_INVALID_ARG, "k=%d not in [1, min(8,E)]", k);
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_version(void) { return MOE_ROUTE_VERSION; }

const char* moe_last_error_string(void) { return g_err; }

// Partial-logit blocks per row the route path produces: 2 for an fp32 weight
// (hi/lo halves) times the GEMM's K partitions.
static int route_parts(int T, int H, int E, int w_dtype) {
  const int N = w_dtype == MOE_DTYPE_FP32 ? 2 * E : E;
  return (N / E) * moe::router_gemm_ksplit(T, H, N);
}

size_t moe_route_workspace_bytes(int T, int H, int E, int w_dtype) {
  if (T < 0 || H < 0 || E <= 0) return 0;
  if (w_dtype != MOE_DTYPE_BF16 && w_dtype != MOE_DTYPE_FP32) return 0;
  // E = 8 or 16 (8 with fp32 weights): the small-E GEMM + scoring kernel, no
  // workspace (it splits an fp32 weight itself)
  if (moe::route_small_supported(E, H, w_dtype == MOE_DTYPE_FP32)) return 0;
  const int parts = route_parts(T, H, E, w_dtype);
  size_t b = 0;
  if (w_dtype == MOE_DTYPE_FP32) b += round256((size_t)2 * E * H * 2);
  if (parts > 1) b += round256((size_t)T * parts * E * 4);
  // E = 256, H = 7168 and E = 128, H = 2048 with bf16 weights: the fused GEMM +
  // scoring kernel (used unless the scoring rule needs narrower lanes) keeps a
  // fragment-major weight copy
  if (w_dtype == MOE_DTYPE_BF16 && ((E == 256 && H == 7168) || (E == 128 && H == 2048))) {
    const size_t f = round256(moe::route_fused_workspace_bytes(E, H));
    if (f > b) b = f;
  }
  return b;
}

}  // extern "C"

// Argument checks of moe_route (workspace included).
static int check_route(const void* x, const void* w, int w_dtype, int T, int H, int E, int k,
                       const moe_route_cfg* cfg, float* logits, int32_t* topk_ids, float* topk_w,
                       void* ws, size_t ws_bytes) {
  int rc = check_topk_shape(T, E, k);
  if (rc) return rc;
  if ((rc = check_cfg(cfg, E, k))) return rc;
  if (w_dtype != MOE_DTYPE_BF16 && w_dtype != MOE_DTYPE_FP32)
    return fail(MOE_ERR_UNSUPPORTED, "w_dtype=%d (BF16 or FP32 only)", w_dtype);
  if (!x || !w || !logits || !topk_ids || !topk_w)
    return fail(MOE_ERR_NULL_POINTER, "x, w, logits, topk_ids and topk_w are required");
  if (H <= 0 || H % 64 != 0) return fail(MOE_ERR_UNSUPPORTED, "H=%d is not a positive multiple of 64", H);
  if (!aligned16(x) || !aligned16(w) || !aligned16(logits))
    return fail(MOE_ERR_ALIGNMENT, "x, w and logits must be 16-byte aligned");
  const size_t need = moe_route_workspace_bytes(T, H, E, w_dtype);
  if (need > 0 && (!ws || ws_bytes < need))
    return fail(MOE_ERR_WORKSPACE, "workspace %zu bytes < %zu required", ws ? ws_bytes : 0, need);
  if (need > 0 && !aligned16(ws)) return fail(MOE_ERR_ALIGNMENT, "workspace not 16-byte aligned");
  return MOE_OK;
}

// Whether route_launch takes the fused kernel (and so can write the permute's
// block histograms as well).
static bool route_is_fused(int T, int H, int E, int w_dtype, const moe_route_cfg* cfg) {
  return T > 0 && w_dtype == MOE_DTYPE_BF16 &&
         moe::route_fused_supported(E, H, cfg->scoring, cfg->n_group);
}

// Whether route_launch takes the small-E kernel (E = 8 or 16 with bf16
// weights, E = 8 with fp32 weights; any scoring rule).
static bool route_is_small(int T, int H, int E, int w_dtype) {
  return T > 0 && moe::route_small_supported(E, H, w_dtype == MOE_DTYPE_FP32);
}

// What the route can hand the permute instead of its histogram launch.
enum RouteHist {
  kHistNone,    // nothing: the permute counts its blocks itself
  kHistBlocks,  // the raw block histograms [E, nblk], at the permute's workspace
  kHistSub,     // the small-E kernel's 32-token histograms [E, ceil(T/32)], in
                // route_sub_hist_bytes after the permute's workspace
};

// kHistSub: every permute block of 256 / k tokens is whole 32-token columns
// and the columns are few enough for the index kernel to sum them itself.
static bool route_sub_hist(int T, int H, int E, int k, int w_dtype) {
  if (!route_is_small(T, H, E, w_dtype)) return false;
  const int st = moe::route_small_tokens();
  if (k < 1 || k > 8 || moe::kPairsPerBlock % k != 0 || (moe::kPairsPerBlock / k) % st != 0)
    return false;
  return moe::dispatch_sum_path(E, (T + st - 1) / st);
}

static size_t route_sub_hist_bytes(int T, int H, int E, int k, int w_dtype) {
  if (!route_sub_hist(T, H, E, k, w_dtype)) return 0;
  const int st = moe::route_small_tokens();
  return round256((size_t)E * ((T + st - 1) / st) * 4);
}

// Which histograms route_launch can also write for the permute: the fused
// kernel's tile, or the scoring kernel's block, covering whole blocks of
// kPairsPerBlock (token, slot) pairs, or the small-E kernel's 32-token
// columns.
static RouteHist route_block_hist(int T, int H, int E, int k, int w_dtype,
                                  const moe_route_cfg* cfg) {
  if (T == 0) return kHistNone;
  if (route_is_small(T, H, E, w_dtype))
    return route_sub_hist(T, H, E, k, w_dtype) ? kHistSub : kHistNone;
  if (route_is_fused(T, H, E, w_dtype, cfg))
    return moe::route_fused_block_hist_supported(E, k) ? kHistBlocks : kHistNone;
  return moe::topk_block_hist_supported(E, k, cfg->scoring, cfg->n_group) ? kHistBlocks
                                                                           : kHistNone;
}

// The route's launches over validated arguments.  blockcnt (or NULL; see
// route_block_hist): also write the permute's raw block histograms, from the
// fused kernel's epilogue or from the scoring kernel, or (small-E kernel) its
// 32-token histograms.
static int route_launch(const void* x, const void* w, int w_dtype, const float* bias, int T, int H,
                        int E, int k, const moe_route_cfg* cfg, float* logits, int32_t* topk_ids,
                        float* topk_w, int32_t* counts, int32_t* blockcnt, void* ws,
                        hipStream_t s) {
  if (T == 0)
    return launched(moe::launch_topk(nullptr, 1, bias, 0, E, k, cfg->scoring, cfg->renormalize,
                                     cfg->n_group, cfg->topk_group, cfg->route_scale,
                                     cfg->norm_min, nullptr, topk_ids, topk_w, counts, nullptr,
                                     s),
                    "topk");
  if (route_is_small(T, H, E, w_dtype)) {
    return launched(moe::launch_route_small((const __bf16*)x, w, w_dtype == MOE_DTYPE_FP32, bias,
                                            T, E, H, k, cfg->scoring, cfg->renormalize, cfg->n_group,
                                            cfg->topk_group, cfg->route_scale, cfg->norm_min,
                                            logits, topk_ids, topk_w, counts, blockcnt, s),
                    "route_small");
  }
  if (route_is_fused(T, H, E, w_dtype, cfg))
    return launched(moe::launch_route_fused((const __bf16*)x, (const __bf16*)w, bias, T, E, H, k,
                                            cfg->scoring, cfg->renormalize, cfg->n_group,
                                            cfg->topk_group, cfg->route_scale, cfg->norm_min,
                                            logits, topk_ids, topk_w, counts, blockcnt, ws, s),
                    "route_fused");
  const int N = w_dtype == MOE_DTYPE_FP32 ? 2 * E : E;
  const int ksplit = moe::router_gemm_ksplit(T, H, N);
  const int parts = (N / E) * ksplit;
  const __bf16* wb = (const __bf16*)w;
  char* wsp = (char*)ws;
  int rc;
  if (w_dtype == MOE_DTYPE_FP32) {
    // fp32 weights: hi/lo bf16 split (K:1786-1824), one GEMM against [2E,H]
    __bf16* wpk = (__bf16*)wsp;
    wsp += round256((size_t)2 * E * H * 2);
    rc = launched(moe::launch_wsplit((const float*)w, wpk, E, H, s), "wsplit");
    if (rc) return rc;
    wb = wpk;
  }
  // parts == 1: the GEMM writes the logits; else it writes [T, parts*E]
  // partial sums and the scoring kernel adds them and writes the logits.
  float* gout = parts > 1 ? (float*)wsp : logits;
  rc = launched(moe::launch_router_gemm((const __bf16*)x, wb, T, H, N, ksplit, gout, s),
                "router_gemm");
  if (rc) return rc;
  // an fp32 weight's partials fold as (sum of hi) + (sum of lo): negative count
  const int fold = w_dtype == MOE_DTYPE_FP32 ? -parts : parts;
  return launched(moe::launch_topk(gout, fold, bias, T, E, k, cfg->scoring, cfg->renormalize,
                                   cfg->n_group, cfg->topk_group, cfg->route_scale,
                                   cfg->norm_min, parts > 1 ? logits : nullptr, topk_ids, topk_w,
                                   counts, blockcnt, s),
                  "topk");
}

extern "C" {

int moe_router_gemm(const void* x, const void* w, int T, int H, int E, float* logits,
                    void* stream) {
  if (!x || !w || !logits) return fail(MOE_ERR_NULL_POINTER, "x, w and logits are required");
  if (T < 0 || H <= 0) return fail(MOE_ERR_INVALID_ARG, "T=%d, H=%d", T, H);
  if (H % 64 != 0) return fail(MOE_ERR_UNSUPPORTED, "H=%d is not a multiple of 64", H);
  if (!supported_e(E)) return fail(MOE_ERR_UNSUPPORTED, "E=%d not in {8,...,256}", E);
  if (!aligned16(x) || !aligned16(w)) return fail(MOE_ERR_ALIGNMENT, "x/w not 16-byte aligned");
  if (T == 0) return ok();
  return launched(moe::launch_router_gemm((const __bf16*)x, (const __bf16*)w, T, H, E, 1, logits,
                                          (hipStream_t)stream),
                  "router_gemm");
}

int moe_topk(const float* logits, const float* bias, int T, int E, int k,
             const moe_route_cfg* cfg, int32_t* topk_ids, float* topk_w, int32_t* counts,
             void* stream) {
  int rc = check_topk_shape(T, E, k);
  if (rc) return rc;
  if ((rc = check_cfg(cfg, E, k))) return rc;
  if (T > 0 && (!logits || !topk_ids || !topk_w))
    return fail(MOE_ERR_NULL_POINTER, "logits, topk_ids and topk_w are required");
  if (logits && !aligned16(logits)) return fail(MOE_ERR_ALIGNMENT, "logits not 16-byte aligned");
  return launched(moe::launch_topk(logits, 1, bias, T, E, k, cfg->scoring, cfg->renormalize,
                                   cfg->n_group, cfg->topk_group, cfg->route_scale,
                                   cfg->norm_min, nullptr, topk_ids, topk_w, counts, nullptr,
                                   (hipStream_t)stream),
                  "topk");
}

int moe_route(const void* x, const void* w, int w_dtype, const float* bias, int T, int H, int E,
              int k, const moe_route_cfg* cfg, float* logits, int32_t* topk_ids, float* topk_w,
              int32_t* counts, void* ws, size_t ws_bytes, void* stream) {
  const int rc = check_route(x, w, w_dtype, T, H, E, k, cfg, logits, topk_ids, topk_w, ws,
                             ws_bytes);
  if (rc) return rc;
  return route_launch(x, w, w_dtype, bias, T, H, E, k, cfg, logits, topk_ids, topk_w, counts,
                      nullptr, ws, (hipStream_t)stream);
}

int moe_offsets(const int32_t* counts, int E, int32_t* offsets, void* stream) {
  if (!counts || !offsets) return fail(MOE_ERR_NULL_POINTER, "counts and offsets are required");
  if (E < 1 || E > 1024) return fail(MOE_ERR_INVALID_ARG, "E=%d not in [1, 1024]", E);
  return launched(moe::launch_offsets(counts, E, offsets, (hipStream_t)stream), "offsets");
}

size_t moe_permute_workspace_bytes(int T, int E, int k) {
  if (T < 0 || E < 0 || k < 0) return 0;
  const int nblk = moe::dispatch_blocks((long long)T * k);
  return round256((size_t)E * nblk * 4) + round256((size_t)E * 4);
}

// The fp8 permute's token-major scale stage, after the permute's workspace.
static size_t fp8_stage_bytes(int T, int H) {
  if (T <= 0 || H <= 0 || H % 128 != 0) return 0;
  return round256((size_t)T * (H / 128) * 4);
}

size_t moe_permute_fp8_workspace_bytes(int T, int H, int E, int k) {
  if (T < 0 || H < 0 || E < 0 || k < 0) return 0;
  return moe_permute_workspace_bytes(T, E, k) + fp8_stage_bytes(T, H);
}

}  // extern "C"

// Argument checks of moe_permute, everything except the workspace.
static int check_permute(const void* x, int x_dtype, const int32_t* topk_ids, int T, int H, int E,
                         int k, int out_dtype, void* xg, float* scales, int32_t* row_token,
                         int32_t* pair_row) {
  if (T < 0 || H <= 0) return fail(MOE_ERR_INVALID_ARG, "T=%d, H=%d", T, H);
  if (E < 1 || E > 1024) return fail(MOE_ERR_INVALID_ARG, "E=%d not in [1, 1024]", E);
  if (k < 1 || k > 8) return fail(MOE_ERR_INVALID_ARG, "k=%d not in [1, 8]", k);
  if (x_dtype != MOE_DTYPE_BF16 && x_dtype != MOE_DTYPE_FP32)
    return fail(MOE_ERR_UNSUPPORTED, "x_dtype=%d (BF16 or FP32 only)", x_dtype);
  const bool fp8 = out_dtype == MOE_DTYPE_FP8E4M3FN;
  if (!fp8 && out_dtype != x_dtype)
    return fail(MOE_ERR_UNSUPPORTED, "out_dtype=%d must equal x_dtype=%d or be FP8E4M3FN",
                out_dtype, x_dtype);
  if (fp8 && x_dtype != MOE_DTYPE_BF16)
    return fail(MOE_ERR_UNSUPPORTED, "fp8 output needs bf16 x");
  if (T > 0 && (!topk_ids || !row_token || !pair_row))
    return fail(MOE_ERR_NULL_POINTER, "topk_ids, row_token and pair_row are required");
  const int elem = x_dtype == MOE_DTYPE_BF16 ? 2 : 4;
  if (xg) {
    if (!x) return fail(MOE_ERR_NULL_POINTER, "x is required when xg is given");
    if (fp8) {
      if (H % 128 != 0) return fail(MOE_ERR_UNSUPPORTED, "fp8 permute needs H %% 128 == 0 (H=%d)", H);
      if (!scales) return fail(MOE_ERR_NULL_POINTER, "fp8 permute needs scales");
    } else if (((long long)H * elem) % 16 != 0) {
      return fail(MOE_ERR_ALIGNMENT, "row of %d bytes is not a multiple of 16", H * elem);
    }
    if (!aligned16(x) || !aligned16(xg))
      return fail(MOE_ERR_ALIGNMENT, "x and xg must be 16-byte aligned");
    if ((long long)T * H * elem / 16 > kMaxVectors)
      return fail(MOE_ERR_UNSUPPORTED, "T*H too large for one call (%lld vectors)",
                  (long long)T * H * elem / 16);
  }
  if (((long long)T * k) >= (1ll << 31))
    return fail(MOE_ERR_UNSUPPORTED, "T*k=%lld exceeds int32 rows", (long long)T * k);
  return MOE_OK;
}

// The permute's launches over a validated workspace of
// moe_permute_workspace_bytes(T, E, k) bytes.
// hist (or NULL): raw histograms a route kernel already wrote, so the
// histogram launch is skipped (T * k > 0): the block histograms [E, nblk] at
// the workspace's start (hist_tokens = 0) or [E, ceil(T / hist_tokens)]
// columns of hist_tokens tokens (launch_dispatch_from_hist).
// stage (fp8 with offsets only, else NULL): fp8_stage_bytes(T, H) bytes for
// the token-major scales.
static int permute_launch(const void* x, int x_dtype, const int32_t* topk_ids, int T, int H,
                          int E, int k, int out_dtype, void* xg, float* scales,
                          int32_t* row_token, int32_t* pair_row, int32_t* offsets,
                          int32_t* counts, void* ws, void* stream, int32_t* hist = nullptr,
                          int hist_tokens = 0, void* stage = nullptr) {
  const bool fp8 = out_dtype == MOE_DTYPE_FP8E4M3FN;
  const int elem = x_dtype == MOE_DTYPE_BF16 ? 2 : 4;
  hipStream_t s = (hipStream_t)stream;
  const int nblk = moe::dispatch_blocks((long long)T * k);
  int32_t* blockcnt = (int32_t*)ws;
  int32_t* totals = (int32_t*)((char*)ws + round256((size_t)E * nblk * 4));
  int rc = hist
               ? launched(moe::launch_dispatch_from_hist(topk_ids, T, E, k, hist, hist_tokens,
                                                         totals, row_token, pair_row, offsets,
                                                         counts, s),
                          "dispatch_from_hist")
               : launched(moe::launch_dispatch_index(topk_ids, T, E, k, blockcnt, totals,
                                                     row_token, pair_row, offsets, counts, s),
                          "dispatch_index");
  if (rc || !xg || T == 0) return rc;
  if (fp8)
    return launched(moe::launch_gather_fp8(x, pair_row, row_token, offsets ? offsets + E : nullptr,
                                           T, H, k, xg, scales,
                                           offsets ? (float*)stage : nullptr, s),
                    "gather_fp8");
  return launched(moe::launch_gather(x, elem, pair_row, T, H, k, xg, s), "gather");
}

// ---------------------------------------------------------------------------
// Fixed device scratch of moe_permute_noalloc: the per-block expert
// histograms and expert totals that moe_permute keeps in the caller's
// workspace.  One copy per GPU, held until the process ends.  Host code never
// names the array in a launch or copy: it uses the address
// hipGetSymbolAddress reports for the current device, looked up once per
// device on the first call there.
// ---------------------------------------------------------------------------
constexpr size_t kNoallocScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];

static int noalloc_scratch(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return launched(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(MOE_ERR_UNSUPPORTED, "device %d beyond the %d scratch slots", dev,
                kMaxScratchDevices);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess) return launched(e, "hipStreamGetDevice");
    if ((int)sdev != dev)
      return fail(MOE_ERR_INVALID_ARG, "stream belongs to device %d, current device is %d",
                  (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return launched(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                               "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE_OK;
}

extern "C" {

int moe_permute(const void* x, int x_dtype, const int32_t* topk_ids, int T, int H, int E, int k,
                int out_dtype, void* xg, float* scales, int32_t* row_token, int32_t* pair_row,
                int32_t* offsets, int32_t* counts, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_permute(x, x_dtype, topk_ids, T, H, E, k, out_dtype, xg, scales, row_token,
                         pair_row);
  if (rc) return rc;
  const size_t need = moe_permute_workspace_bytes(T, E, k);
  if (!ws || ws_bytes < need)
    return fail(MOE_ERR_WORKSPACE, "workspace %zu bytes < %zu required", ws ? ws_bytes : 0, need);
  // fp8 rows with room for the scale stage after the permute's workspace
  void* stage = nullptr;
  if (out_dtype == MOE_DTYPE_FP8E4M3FN && fp8_stage_bytes(T, H) > 0 &&
      ws_bytes >= moe_permute_fp8_workspace_bytes(T, H, E, k))
    stage = (char*)ws + need;
  return permute_launch(x, x_dtype, topk_ids, T, H, E, k, out_dtype, xg, scales, row_token,
                        pair_row, offsets, counts, ws, stream, nullptr, 0, stage);
}

size_t moe_permute_noalloc_max_scratch_bytes(void) { return kNoallocScratchBytes; }

int moe_permute_noalloc(const void* x, int x_dtype, const int32_t* topk_ids, int T, int H, int E,
                        int k, int out_dtype, void* xg, float* scales, int32_t* row_token,
                        int32_t* pair_row, int32_t* offsets, int32_t* counts, void* stream) {
  int rc = check_permute(x, x_dtype, topk_ids, T, H, E, k, out_dtype, xg, scales, row_token,
                         pair_row);
  if (rc) return rc;
  const size_t need = moe_permute_workspace_bytes(T, E, k);
  if (need > kNoallocScratchBytes)
    return fail(MOE_ERR_UNSUPPORTED,
                "T=%d, E=%d, k=%d needs %zu bytes of scratch, above the fixed %zu "
                "(use moe_permute with a workspace)",
                T, E, k, need, kNoallocScratchBytes);
  void* ws = nullptr;
  if ((rc = noalloc_scratch(stream, &ws))) return rc;
  return permute_launch(x, x_dtype, topk_ids, T, H, E, k, out_dtype, xg, scales, row_token,
                        pair_row, offsets, counts, ws, stream);
}

size_t moe_route_permute_workspace_bytes(int T, int H, int E, int k, int w_dtype) {
  if (T < 0 || H < 0 || E <= 0 || k < 0) return 0;
  return round256(moe_route_workspace_bytes(T, H, E, w_dtype)) +
         moe_permute_fp8_workspace_bytes(T, H, E, k) + route_sub_hist_bytes(T, H, E, k, w_dtype);
}

int moe_route_permute(const void* x, const void* w, int w_dtype, const float* bias, int T, int H,
                      int E, int k, const moe_route_cfg* cfg, float* logits, int32_t* topk_ids,
                      float* topk_w, int out_dtype, void* xg, float* scales, int32_t* row_token,
                      int32_t* pair_row, int32_t* offsets, int32_t* counts, void* ws,
                      size_t ws_bytes, void* stream) {
  // every argument of both stages is checked before anything is launched
  const size_t rneed = round256(moe_route_workspace_bytes(T, H, E, w_dtype));
  const size_t need = moe_route_permute_workspace_bytes(T, H, E, k, w_dtype);
  if (!ws || ws_bytes < need)
    return fail(MOE_ERR_WORKSPACE, "workspace %zu bytes < %zu required", ws ? ws_bytes : 0, need);
  if (!aligned16(ws)) return fail(MOE_ERR_ALIGNMENT, "workspace not 16-byte aligned");
  int rc = check_route(x, w, w_dtype, T, H, E, k, cfg, logits, topk_ids, topk_w, ws, rneed);
  if (rc) return rc;
  if ((rc = check_permute(x, MOE_DTYPE_BF16, topk_ids, T, H, E, k, out_dtype, xg, scales,
                          row_token, pair_row)))
    return rc;
  hipStream_t s = (hipStream_t)stream;
  void* pws = (char*)ws + rneed;
  // Where the route's fused kernel (its epilogue) or its scoring kernel covers
  // whole permute blocks, it writes the permute's block histograms and the
  // histogram launch is skipped.  The route never writes counts here: the
  // index kernel writes them from the scanned totals.
  const RouteHist handoff = route_block_hist(T, H, E, k, w_dtype, cfg);
  void* stage = (char*)pws + moe_permute_workspace_bytes(T, E, k);
  int32_t* sub = (int32_t*)((char*)pws + moe_permute_fp8_workspace_bytes(T, H, E, k));
  int32_t* hist = handoff == kHistSub ? sub : handoff == kHistBlocks ? (int32_t*)pws : nullptr;
  rc = route_launch(x, w, w_dtype, bias, T, H, E, k, cfg, logits, topk_ids, topk_w, nullptr, hist,
                    ws, s);
  if (rc) return rc;
  return permute_launch(x, MOE_DTYPE_BF16, topk_ids, T, H, E, k, out_dtype, xg, scales, row_token,
                        pair_row, offsets, counts, pws, stream, hist,
                        handoff == kHistSub ? moe::route_small_tokens() : 0,
                        fp8_stage_bytes(T, H) > 0 ? stage : nullptr);
}

int moe_combine(const void* y, int y_dtype, const int32_t* pair_row, const float* topk_w,
                const void* shared, int T, int H, int k, void* out, void* stream) {
  if (T < 0 || H <= 0) return fail(MOE_ERR_INVALID_ARG, "T=%d, H=%d", T, H);
  if (k < 1 || k > 8) return fail(MOE_ERR_INVALID_ARG, "k=%d not in [1, 8]", k);
  if (y_dtype != MOE_DTYPE_BF16 && y_dtype != MOE_DTYPE_FP32)
    return fail(MOE_ERR_UNSUPPORTED, "y_dtype=%d (BF16 or FP32 only)", y_dtype);
  if (T == 0) return ok();
  if (!y || !pair_row || !topk_w || !out)
    return fail(MOE_ERR_NULL_POINTER, "y, pair_row, topk_w and out are required");
  const int elem = y_dtype == MOE_DTYPE_BF16 ? 2 : 4;
  if (((long long)H * elem) % 16 != 0)
    return fail(MOE_ERR_ALIGNMENT, "row of %d bytes is not a multiple of 16", H * elem);
  if (!aligned16(y) || !aligned16(out) || (shared && !aligned16(shared)))
    return fail(MOE_ERR_ALIGNMENT, "y, out and shared must be 16-byte aligned");
  if ((long long)T * H * elem / 16 > kMaxVectors)
    return fail(MOE_ERR_UNSUPPORTED, "T*H too large for one call");
  return launched(moe::launch_combine(y, y_dtype == MOE_DTYPE_BF16 ? 0 : 1, pair_row, topk_w,
                                      shared, T, H, k, out, (hipStream_t)stream),
                  "combine");
}

size_t moe_grouped_gemm_workspace_bytes(int G) {
  if (G < 0) return 0;
  return round256((size_t)(G + 1) * 4);
}

static int grouped_common(const void* a, const float* a_scales, const int32_t* a_rows,
                          const void* w0, const void* w1, const int32_t* offs, int G, int M,
                          int N, int K, const void* ident_a, int ident_m, void* out, void* ws,
                          size_t ws_bytes, void* stream, bool swiglu, bool fp8, bool rows) {
  if (G < 1 || G > 65536) return fail(MOE_ERR_INVALID_ARG, "G=%d not in [1, 65536]", G);
  if (M < 0 || N < 1 || K < 1) return fail(MOE_ERR_INVALID_ARG, "M=%d, N=%d, K=%d", M, N, K);
  if (K % 64 != 0) return fail(MOE_ERR_UNSUPPORTED, "K=%d is not a multiple of 64", K);
  if (fp8) {
    if (K % 128 != 0)
      return fail(MOE_ERR_UNSUPPORTED, "fp8 A needs K %% 128 == 0 (one scale per 128), K=%d", K);
    if (M > 0 && !a_scales) return fail(MOE_ERR_NULL_POINTER, "fp8 A needs a_scales");
    if (a_scales && ((uintptr_t)a_scales & 3u))
      return fail(MOE_ERR_ALIGNMENT, "a_scales not 4-byte aligned");
    if ((long long)M * (K / 128) >= (1ll << 31))
      return fail(MOE_ERR_UNSUPPORTED, "a_scales of %lld entries exceeds int32 indexing",
                  (long long)M * (K / 128));
  }
  if (ident_m < 0) return fail(MOE_ERR_INVALID_ARG, "ident_m=%d < 0", ident_m);
  if (!offs || !ws) return fail(MOE_ERR_NULL_POINTER, "offs and ws are required");
  if (M > 0 && (!a || !w0 || !w1 || !out))
    return fail(MOE_ERR_NULL_POINTER, "a, the weights and the output are required");
  if (ident_m > 0 && !ident_a) return fail(MOE_ERR_NULL_POINTER, "ident_m > 0 needs ident_a");
  if (rows && M > 0 && !a_rows) return fail(MOE_ERR_NULL_POINTER, "a_rows is required");
  if (a_rows && ((uintptr_t)a_rows & 3u))
    return fail(MOE_ERR_ALIGNMENT, "a_rows not 4-byte aligned");
  if ((a && !aligned16(a)) || (w0 && !aligned16(w0)) || (w1 && !aligned16(w1)) ||
      (ident_a && !aligned16(ident_a)))
    return fail(MOE_ERR_ALIGNMENT, "a, ident_a and the weights must be 16-byte aligned");
  if ((long long)M * K >= (1ll << 40) || (long long)G * N * K >= (1ll << 40))
    return fail(MOE_ERR_UNSUPPORTED, "operands too large");
  const size_t need = moe_grouped_gemm_workspace_bytes(G);
  if (ws_bytes < need)
    return fail(MOE_ERR_WORKSPACE, "workspace %zu bytes < %zu required", ws_bytes, need);
  if (!aligned16(ws)) return fail(MOE_ERR_ALIGNMENT, "workspace not 16-byte aligned");
  // row tiles are 128 or 256 rows: bound by the 128-row count
  const long long blocks = (((long long)M + 127) / 128 + G) *
                           moe::grouped_gemm_n_tiles(N, swiglu);
  if (blocks >= (1ll << 31)) return fail(MOE_ERR_UNSUPPORTED, "too many tiles (%lld)", blocks);
  return launched(moe::launch_grouped_gemm(a, fp8 ? a_scales : nullptr, a_rows, ident_a, ident_m,
                                           w0, w1, offs, G, M, N, K, swiglu, out, (int32_t*)ws,
                                           (hipStream_t)stream),
                  swiglu ? "grouped_swiglu" : "grouped_gemm");
}

int moe_grouped_gemm(const void* a, const void* w, const int32_t* offs, int G, int M, int N,
                     int K, const void* ident_a, int ident_m, void* out, void* ws,
                     size_t ws_bytes, void* stream) {
  return grouped_common(a, nullptr, nullptr, w, w, offs, G, M, N, K, ident_a, ident_m, out, ws,
                        ws_bytes, stream, false, false, false);
}

int moe_grouped_swiglu(const void* a, const void* wg, const void* wu, const int32_t* offs,
                       int G, int M, int N, int K, const void* ident_a, int ident_m, void* h,
                       void* ws, size_t ws_bytes, void* stream) {
  return grouped_common(a, nullptr, nullptr, wg, wu, offs, G, M, N, K, ident_a, ident_m, h, ws,
                        ws_bytes, stream, true, false, false);
}

int moe_grouped_gemm_rows(const void* a, const int32_t* a_rows, const void* w,
                          const int32_t* offs, int G, int M, int N, int K, void* out, void* ws,
                          size_t ws_bytes, void* stream) {
  return grouped_common(a, nullptr, a_rows, w, w, offs, G, M, N, K, nullptr, 0, out, ws,
                        ws_bytes, stream, false, false, true);
}

int moe_grouped_swiglu_rows(const void* a, const int32_t* a_rows, const void* wg, const void* wu,
                            const int32_t* offs, int G, int M, int N, int K, void* h, void* ws,
                            size_t ws_bytes, void* stream) {
  return grouped_common(a, nullptr, a_rows, wg, wu, offs, G, M, N, K, nullptr, 0, h, ws,
                        ws_bytes, stream, true, false, true);
}

int moe_grouped_gemm_fp8(const void* a, const float* a_scales, const void* w, const int32_t* offs,
                         int G, int M, int N, int K, void* out, void* ws, size_t ws_bytes,
                         void* stream) {
  return grouped_common(a, a_scales, nullptr, w, w, offs, G, M, N, K, nullptr, 0, out, ws,
                        ws_bytes, stream, false, true, false);
}

int moe_grouped_swiglu_fp8(const void* a, const float* a_scales, const void* wg, const void* wu,
                           const int32_t* offs, int G, int M, int N, int K, void* h, void* ws,
                           size_t ws_bytes, void* stream) {
  return grouped_common(a, a_scales, nullptr, wg, wu, offs, G, M, N, K, nullptr, 0, h, ws,
                        ws_bytes, stream, true, true, false);
}

static int grouped_i8_common(const int8_t* a, const float* a_scales, const int32_t* a_rows,
                             const int8_t* w0, const float* w0s, const int8_t* w1,
                             const float* w1s, const int32_t* offs, int G, int M, int N, int K,
                             const int8_t* ident_a, const float* ident_scales, int ident_m,
                             void* out, void* ws, size_t ws_bytes, void* stream, bool swiglu) {
  if (G < 1 || G > 65536) return fail(MOE_ERR_INVALID_ARG, "G=%d not in [1, 65536]", G);
  if (M < 0 || N < 1 || K < 1) return fail(MOE_ERR_INVALID_ARG, "M=%d, N=%d, K=%d", M, N, K);
  if (K % 128 != 0) return fail(MOE_ERR_UNSUPPORTED, "int8 K=%d is not a multiple of 128", K);
  if (ident_m < 0) return fail(MOE_ERR_INVALID_ARG, "ident_m=%d < 0", ident_m);
  if (!offs || !ws) return fail(MOE_ERR_NULL_POINTER, "offs and ws are required");
  if (M > 0 && (!a || !a_scales || !w0 || !w0s || !w1 || !w1s || !out))
    return fail(MOE_ERR_NULL_POINTER, "a, the weights, their scales and the output are required");
  if (ident_m > 0 && (!ident_a || !ident_scales))
    return fail(MOE_ERR_NULL_POINTER, "ident_m > 0 needs ident_a and ident_scales");
  if ((a && !aligned16(a)) || (w0 && !aligned16(w0)) || (w1 && !aligned16(w1)) ||
      (ident_a && !aligned16(ident_a)))
    return fail(MOE_ERR_ALIGNMENT, "a, ident_a and the weights must be 16-byte aligned");
  if ((a_scales && ((uintptr_t)a_scales & 3u)) || (w0s && ((uintptr_t)w0s & 3u)) ||
      (w1s && ((uintptr_t)w1s & 3u)) || (ident_scales && ((uintptr_t)ident_scales & 3u)) ||
      (a_rows && ((uintptr_t)a_rows & 3u)))
    return fail(MOE_ERR_ALIGNMENT, "scales and a_rows must be 4-byte aligned");
  if ((long long)M * K >= (1ll << 40) || (long long)G * N * K >= (1ll << 40) ||
      (long long)G * N >= (1ll << 31))
    return fail(MOE_ERR_UNSUPPORTED, "operands too large");
  const size_t need = moe_grouped_gemm_workspace_bytes(G);
  if (ws_bytes < need)
    return fail(MOE_ERR_WORKSPACE, "workspace %zu bytes < %zu required", ws_bytes, need);
  if (!aligned16(ws)) return fail(MOE_ERR_ALIGNMENT, "workspace not 16-byte aligned");
  const long long blocks = (((long long)M + 127) / 128 + G) *
                           moe::grouped_gemm_n_tiles(N, swiglu);
  if (blocks >= (1ll << 31)) return fail(MOE_ERR_UNSUPPORTED, "too many tiles (%lld)", blocks);
  return launched(moe::launch_grouped_gemm_i8(a, a_scales, a_rows, ident_a, ident_scales,
                                              ident_m, w0, w0s, w1, w1s, offs, G, M, N, K, swiglu,
                                              out, (int32_t*)ws, (hipStream_t)stream),
                  swiglu ? "grouped_swiglu_i8" : "grouped_gemm_i8");
}

int moe_grouped_gemm_i8(const int8_t* a, const float* a_scales, const int32_t* a_rows,
                        const int8_t* w, const float* w_scales, const int32_t* offs, int G, int M,
                        int N, int K, const int8_t* ident_a, const float* ident_scales,
                        int ident_m, void* out, void* ws, size_t ws_bytes, void* stream) {
  return grouped_i8_common(a, a_scales, a_rows, w, w_scales, w, w_scales, offs, G, M, N, K,
                           ident_a, ident_scales, ident_m, out, ws, ws_bytes, stream, false);
}

int moe_grouped_swiglu_i8(const int8_t* a, const float* a_scales, const int32_t* a_rows,
                          const int8_t* wg, const float* wg_scales, const int8_t* wu,
                          const float* wu_scales, const int32_t* offs, int G, int M, int N, int K,
                          const int8_t* ident_a, const float* ident_scales, int ident_m, void* h,
                          void* ws, size_t ws_bytes, void* stream) {
  return grouped_i8_common(a, a_scales, a_rows, wg, wg_scales, wu, wu_scales, offs, G, M, N,
                           K, ident_a, ident_scales, ident_m, h, ws, ws_bytes, stream, true);
}

int moe_quant_rows_i8(const void* x, long long R, int K, int hadamard, float scale_mul,
                      int group_rows, const int32_t* group_counts, int8_t* q, float* scales,
                      void* stream) {
  if (R < 0 || K < 1) return fail(MOE_ERR_INVALID_ARG, "R=%lld, K=%d", R, K);
  if (R >= (1ll << 31)) return fail(MOE_ERR_UNSUPPORTED, "R=%lld rows exceeds the grid", R);
  if (hadamard != 0 && hadamard != 16 && hadamard != 128)
    return fail(MOE_ERR_INVALID_ARG, "hadamard=%d (0, 16 or 128)", hadamard);
  if (K % (hadamard == 128 ? 128 : 16) != 0)
    return fail(MOE_ERR_UNSUPPORTED, "K=%d is not a multiple of %d", K,
                hadamard == 128 ? 128 : 16);
  if (K > moe::quant_rows_max_k())
    return fail(MOE_ERR_UNSUPPORTED, "K=%d > %d", K, moe::quant_rows_max_k());
  if (!(scale_mul > 0.0f) || !std::isfinite(scale_mul))
    return fail(MOE_ERR_INVALID_ARG, "scale_mul must be finite and > 0");
  if (group_counts && (group_rows < 1 || R % group_rows != 0))
    return fail(MOE_ERR_INVALID_ARG, "group_rows=%d must divide R=%lld with group_counts",
                group_rows, R);
  if (group_counts && R / group_rows > moe::quant_rows_max_groups())
    return fail(MOE_ERR_UNSUPPORTED, "%lld groups > %d", R / group_rows,
                moe::quant_rows_max_groups());
  if (R > 0 && (!x || !q || !scales))
    return fail(MOE_ERR_NULL_POINTER, "x, q and scales are required");
  if ((x && !aligned16(x)) || (q && !aligned16(q)) || (scales && ((uintptr_t)scales & 3u)) ||
      (group_counts && ((uintptr_t)group_counts & 3u)))
    return fail(MOE_ERR_ALIGNMENT, "x and q must be 16-byte aligned, scales 4-byte aligned");
  return launched(moe::launch_quant_rows_i8((const __bf16*)x, R, K, hadamard, scale_mul,
                                            group_rows, group_counts, (signed char*)q, scales,
                                            (hipStream_t)stream),
                  "quant_rows_i8");
}

}  // extern "C"
