/*
 * moe_route.h -- C ABI of libmoe_route.so, the MI355X (gfx950) MoE
 * route -> dispatch -> combine path.
 *
 * Reference: sol-execbench/029_moe_sparse_routing_and_dispatch/kernel.cu
 * (abbreviated K).  The reference exposes the path as one PyTorch extension
 * function, run() (K:4067-4077, bound at K:5729-5735), whose body launches the
 * stage kernels listed beside each entry point below.  This library exposes
 * the same stages as plain C functions over raw device pointers so that any
 * host (ctypes, cgo, JNI, N-API, C++) can bind them.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers (HBM) unless stated; tensors are dense and
 *     row-major.  bf16 is IEEE bfloat16, fp8 is OCP float8 e4m3fn.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Every call only
 *     enqueues work on that stream: no host synchronisation, no allocation, no
 *     events (as the reference, K:57-58, K:4079).
 *   - Return 0 on success, a negative MOE_ERR_* code otherwise; the message
 *     is in moe_last_error_string() (thread-local).  Arguments are validated
 *     on the host before anything is launched, so every error path is
 *     testable without a GPU.
 *   - Index outputs are int32.  A pair is (token t, slot j), flat index
 *     t*k + j.  A row is a position in the expert-contiguous buffer.
 */
#ifndef MOE_ROUTE_H_
#define MOE_ROUTE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_ROUTE_VERSION 1

/* error codes */
#define MOE_OK 0
#define MOE_ERR_NULL_POINTER -1   /* a required pointer is NULL */
#define MOE_ERR_INVALID_ARG -2    /* a size or configuration value is out of range */
#define MOE_ERR_UNSUPPORTED -3    /* a valid combination this build has no kernel for */
#define MOE_ERR_WORKSPACE -4      /* workspace missing or smaller than required */
#define MOE_ERR_LAUNCH -5         /* the HIP runtime refused a launch */
#define MOE_ERR_ALIGNMENT -6      /* a pointer or row size breaks 16-byte alignment */

/* element types */
#define MOE_DTYPE_BF16 0
#define MOE_DTYPE_FP32 1
#define MOE_DTYPE_FP8E4M3FN 2

/* scoring rules (moe_route_cfg.scoring) */
#define MOE_SCORING_SOFTMAX 0       /* top-k of logit(+bias); softmax weights (Mixtral, Qwen3) */
#define MOE_SCORING_SIGMOID_GROUP 1 /* sigmoid; +bias for selection; group-limited (DeepSeek-V3) */
#define MOE_SCORING_SOFTMAX_BIAS 2  /* softmax, +bias after softmax, / max(sum, norm_min): K:1857-1909 */

/* Routing configuration.  The reference hard-wires softmax + post-softmax
 * bias with NE=64, TOPK=8 (K:1582-1583, K:1857-1909); this struct carries the
 * generalisation the benchmark configurations need. */
typedef struct moe_route_cfg {
  int scoring;       /* MOE_SCORING_* */
  int renormalize;   /* 1: selected weights are renormalised to sum 1 (before route_scale) */
  int n_group;       /* SIGMOID_GROUP: number of expert groups (1 = no group limit) */
  int topk_group;    /* SIGMOID_GROUP: groups kept per token */
  float route_scale; /* weights are multiplied by this (DeepSeek-V3: 2.5) */
  float norm_min;    /* SOFTMAX_BIAS: denominator floor, the reference's norm_min (K:1909) */
} moe_route_cfg;

/* Library version (MOE_ROUTE_VERSION). */
int moe_version(void);

/* Message of the last error on the calling thread ("" if none).
 * Replaces TORCH_CHECK's exception text (K:1771-1775, K:4088). */
const char* moe_last_error_string(void);

/* Workspace bytes moe_route needs (the K:4197-4268 arena, caller-owned).
 * Non-zero only when
 *   - w_dtype is FP32: the hi/lo split weight [2E,H] bf16, plus
 *   - the GEMM writes more than one partial logit block per row, i.e. FP32
 *     weights (hi and lo halves) or a K split (ksplit > 1, chosen when the
 *     row x expert tiles alone leave the chip's 256 CUs idle, e.g. small T):
 *     [T, parts*E] fp32 partial sums.
 *   - E = 256, H = 7168 or E = 128, H = 2048 with bf16 weights: the router
 *     GEMM and the scoring run as one kernel that reads a fragment-major copy
 *     of the weight, E*H*2 bytes (3.5 MiB / 512 KiB), rewritten by every call.
 * E = 8 or 16 with bf16 weights and H % 256 == 0 (the Mixtral shape): zero;
 * one kernel does the GEMM, with K split across the four waves of a block,
 * and the scoring (E = 8 with FP32 weights too: the kernel splits the weight
 * into its bf16 hi/lo halves itself).
 * The size does not depend on cfg; it covers whichever path the call takes. */
size_t moe_route_workspace_bytes(int T, int H, int E, int w_dtype);

/* Stage 1: router GEMM, logits[T,E] fp32 = x[T,H] bf16 . w[E,H]^T bf16, fp32
 * accumulate on MFMA.  Replaces the cublasGemmEx call K:4327-4339.
 * Needs H % 64 == 0 and E in {8,16,32,64,128,256}. */
int moe_router_gemm(const void* x, const void* w, int T, int H, int E, float* logits,
                    void* stream);

/* Stage 2 (+ histogram): scoring + top-k on fp32 logits.  Replaces
 * topk_kernel K:1829-1920 (selection, weights, LDS histogram + global flush).
 * bias: [E] fp32 or NULL.  Outputs topk_ids [T,k], topk_w [T,k], counts [E]
 * (counts may be NULL).  Slots are ordered by descending selection score,
 * ties to the lower expert index (K:1886).  1 <= k <= 8. */
int moe_topk(const float* logits, const float* bias, int T, int E, int k,
             const moe_route_cfg* cfg, int32_t* topk_ids, float* topk_w, int32_t* counts,
             void* stream);

/* Stages 1+2: router GEMM + scoring + top-k + histogram (run() K:4323-4354).
 * w_dtype BF16: w is [E,H] bf16.  w_dtype FP32: w is [E,H] fp32 and is split
 * into bf16 hi/lo on the device (wsplit_kernel K:1786-1824) so the bf16 GEMM
 * yields fp32-accurate logits.  logits [T,E] fp32 (the reference's
 * router_logits output), counts may be NULL.  With bf16 weights at E = 256,
 * H = 7168 or E = 128, H = 2048 the GEMM and the scoring are one kernel
 * (unless a group-limited rule's groups are not multiples of 32 experts at
 * E = 256, 16 at E = 128: then the two-kernel path, same results). */
int moe_route(const void* x, const void* w, int w_dtype, const float* bias, int T, int H,
              int E, int k, const moe_route_cfg* cfg, float* logits, int32_t* topk_ids,
              float* topk_w, int32_t* counts, void* ws, size_t ws_bytes, void* stream);

/* Exclusive prefix sum of counts[E] into offsets[E+1] (offsets[E] = total).
 * offsets + 1 is the reference's inclusive group-end array offs
 * (offsets_kernel scan K:2069-2086; moe_gemm.h:66-69).  E <= 1024. */
int moe_offsets(const int32_t* counts, int E, int32_t* offsets, void* stream);

/* Workspace bytes moe_permute needs (per-block expert histograms). */
size_t moe_permute_workspace_bytes(int T, int E, int k);

/* Workspace bytes with which moe_permute's fp8 output writes its scales
 * through a token-major stage (T * H/128 fp32 after the histograms) and
 * copies whole destination rows of scales afterwards, instead of k scattered
 * 32-byte runs per token (C5: 0.07 ms less per step).  Same outputs either
 * way; the stage is used when ws_bytes reaches this size, out_dtype is
 * FP8E4M3FN, H % 128 == 0 and offsets is given.  No counterpart in the
 * reference, which has no routed fp8 permute. */
size_t moe_permute_fp8_workspace_bytes(int T, int H, int E, int k);

/* Stages 3+4: stable expert-major permutation and row gather.  Replaces
 * offsets_kernel (scan part) + dispatch_kernel + gather_kernel
 * (K:1922-2238).  Pairs are placed in the order argsort(topk_ids.flatten(),
 * stable): by expert, then ascending token -- deterministic, unlike the
 * reference's atomic order (K:2155-2158).
 *   x        [T,H] of x_dtype (BF16 or FP32)
 *   out_dtype == x_dtype: xg[T*k,H] rows are copies of x rows;
 *   out_dtype FP8E4M3FN (x BF16 only): xg[T*k,H] bytes, scales[T*k,H/128] fp32,
 *     q = e4m3fn(clamp(x / s, +-448)), s = max(amax over 128, 1e-10) / 448.
 *   row_token[T*k]: token of each row (the reference's tok, K:2179)
 *   pair_row[T*k] : row of each pair  (the reference's inv, K:2178)
 *   offsets[E+1]  : exclusive expert offsets (may be NULL)
 *   counts[E]     : per-expert row counts (may be NULL)
 * xg may be NULL (index work only).  An id outside [0,E) gets pair_row -1 and
 * no row.  Needs H*elem % 16 == 0 (FP8: H % 128 == 0). */
int moe_permute(const void* x, int x_dtype, const int32_t* topk_ids, int T, int H, int E,
                int k, int out_dtype, void* xg, float* scales, int32_t* row_token,
                int32_t* pair_row, int32_t* offsets, int32_t* counts, void* ws,
                size_t ws_bytes, void* stream);

/* moe_permute without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts
 * that forbid hipMalloc).  No counterpart in the reference (whose run()
 * takes scratch from a per-call arena, K:4197-4268).  Same arguments,
 * results and errors as moe_permute; the per-block histograms live in a
 * fixed device array of moe_permute_noalloc_max_scratch_bytes() (4 MiB) per
 * GPU, held until the process ends, so moe_permute_workspace_bytes(T, E, k)
 * must not exceed it (E=256, k=8: T up to 131040) -- larger calls return
 * MOE_ERR_UNSUPPORTED.  Nothing in it needs clearing between calls (every
 * call writes all it reads).  The array is shared by every call on one GPU:
 * calls that overlap on one GPU (two streams, two threads) race.  stream
 * must belong to the calling thread's current device. */
size_t moe_permute_noalloc_max_scratch_bytes(void);
int moe_permute_noalloc(const void* x, int x_dtype, const int32_t* topk_ids, int T, int H, int E,
                        int k, int out_dtype, void* xg, float* scales, int32_t* row_token,
                        int32_t* pair_row, int32_t* offsets, int32_t* counts, void* stream);

/* Stages 1-4 in one call: moe_route, then moe_permute on its ids (bf16 x;
 * out_dtype BF16 or FP8E4M3FN; xg NULL = index only), with the same outputs
 * bit for bit as the two calls.  Replaces run()'s sequence K:4323-4431
 * (wsplit, router GEMM, topk_kernel, offsets_kernel, dispatch and gather).
 * Where a route kernel covers whole permute blocks of 256 (token, slot)
 * pairs, it also writes the permute's per-block expert histograms into the
 * workspace and the permute's histogram launch is skipped: the fused kernel
 * (see moe_route) when 256 / k tokens fit its token tile (k in {2, 4, 8} at
 * E = 256, {4, 8} at E = 128), else the scoring kernel when 256 / k is a
 * multiple of the tokens one of its passes scores (k in {1, 2, 4, 8}: 32
 * tokens per pass at E <= 128, 16 at E = 256, fewer with expert groups
 * narrower than 16).  The small-E route kernel (E = 8 or 16, see
 * moe_route) writes one histogram per 32 tokens instead, which the index
 * kernel sums per permute block, when 256 / k is a multiple of 32 (k in
 * {1, 2, 4, 8}) and E * ceil(T / 32) <= 8192.  Otherwise the two stages run
 * as moe_route and moe_permute would.  counts: the permute's.
 * ws: moe_route_permute_workspace_bytes(T, H, E, k, w_dtype) bytes, 16-byte
 * aligned (the route's workspace, rounded up to 256 bytes, then the
 * permute's with its fp8 scale stage, moe_permute_fp8_workspace_bytes, then,
 * for the small-E kernel's handoff, E * ceil(T / 32) int32 rounded up to 256
 * bytes).
 * Every argument of both stages is checked before any launch. */
size_t moe_route_permute_workspace_bytes(int T, int H, int E, int k, int w_dtype);
int moe_route_permute(const void* x, const void* w, int w_dtype, const float* bias, int T, int H,
                      int E, int k, const moe_route_cfg* cfg, float* logits, int32_t* topk_ids,
                      float* topk_w, int out_dtype, void* xg, float* scales, int32_t* row_token,
                      int32_t* pair_row, int32_t* offsets, int32_t* counts, void* ws,
                      size_t ws_bytes, void* stream);

/* Stage 5: weighted combine.  Replaces combine_kernel K:2365-2428:
 *   out[t] = cast(shared[t] + sum_j topk_w[t,j] * y[pair_row[t,j]])
 * accumulated in fp32 in slot order.  y [R,H] and out [T,H] of y_dtype (BF16
 * or FP32); shared [T,H] of y_dtype or NULL; pairs with pair_row < 0 are
 * skipped. */
int moe_combine(const void* y, int y_dtype, const int32_t* pair_row, const float* topk_w,
                const void* shared, int T, int H, int k, void* out, void* stream);

/* Workspace bytes moe_grouped_gemm / moe_grouped_swiglu need: the device
 * tile plan, (G+1) int32.  It is always required; the kernels only write and
 * read it for G > 256 (below, every block scans the group ends itself). */
size_t moe_grouped_gemm_workspace_bytes(int G);

/* Expert grouped GEMM over expert-contiguous rows.  Replaces grouped_mm
 * (moe_gemm.h:66-85) and its device plan (plan_kernel, moe_gemm.cu:616-650):
 *   out[r, :] = a[r, :] . w[g]^T  for every row r of group g,
 * group g = rows [offs[g-1], offs[g]) (offs[-1] = 0): offs[G] int32 are the
 * INCLUSIVE group ends on the device -- moe_permute's `offsets + 1`.
 *   a   [M, K] bf16 row-major;  w [G, N, K] bf16 (K-contiguous, the
 *       reference's expert_*_proj layout);  out [M, N] bf16.
 *   ident_a / ident_m: identity shortcut (moe_gemm.h:72-77): a group with
 *       exactly ident_m rows reads row i from ident_a [ident_m, K] instead of
 *       a.  ident_m = 0 disables it (ident_a may then be NULL).
 * fp32 accumulation on MFMA.  offs must be non-decreasing and <= M; values
 * outside [0, M] are clamped, never dereferenced.  Needs K % 64 == 0, N >= 1. */
int moe_grouped_gemm(const void* a, const void* w, const int32_t* offs, int G, int M, int N,
                     int K, const void* ident_a, int ident_m, void* out, void* ws,
                     size_t ws_bytes, void* stream);

/* SwiGLU expert projection: grouped_mm_pair (moe_gemm.h:87-95) with the
 * silu*mul of the gate and up outputs fused into the epilogue (the
 * reference's int8 gate+up GEMM emits h itself, kernel.cu:61-62):
 *   h[r, :] = silu(a[r, :] . wg[g]^T) * (a[r, :] . wu[g]^T)
 * wg, wu [G, N, K] bf16; h [M, N] bf16; the rest as moe_grouped_gemm. */
int moe_grouped_swiglu(const void* a, const void* wg, const void* wu, const int32_t* offs,
                       int G, int M, int N, int K, const void* ident_a, int ident_m, void* h,
                       void* ws, size_t ws_bytes, void* stream);

/* The same two GEMMs with a row map instead of gathered rows: operand row r is
 * row a_rows[r] of a (e.g. a = the tokens x and a_rows = moe_permute's
 * row_token, so the permute runs index-only and no gathered copy is
 * written).  This generalises the reference plan's identity shortcut, which
 * aims A at x when a group holds all T tokens (moe_gemm.cu:616-650), to any
 * group.  a_rows [M] int32 (values must be rows of a), out / h [M, N]. */
int moe_grouped_gemm_rows(const void* a, const int32_t* a_rows, const void* w,
                          const int32_t* offs, int G, int M, int N, int K, void* out, void* ws,
                          size_t ws_bytes, void* stream);
int moe_grouped_swiglu_rows(const void* a, const int32_t* a_rows, const void* wg, const void* wu,
                            const int32_t* offs, int G, int M, int N, int K, void* h, void* ws,
                            size_t ws_bytes, void* stream);

/* fp8 dispatch into the expert GEMMs: the A operand is moe_permute's fp8
 * output (e4m3fn bytes a [M, K] plus fp32 scales a_scales [M, K/128]) and is
 * dequantised in the GEMM's A load as bf16(q * s) -- the fp8 row permute
 * feeding the grouped GEMM without a bf16 copy of the routed rows (the
 * reference quantises activations for its int8 expert GEMMs the same way,
 * per row, in xquant: kernel.cu:2542-2596).  Otherwise as moe_grouped_gemm /
 * moe_grouped_swiglu; needs K % 128 == 0; no identity shortcut. */
int moe_grouped_gemm_fp8(const void* a, const float* a_scales, const void* w, const int32_t* offs,
                         int G, int M, int N, int K, void* out, void* ws, size_t ws_bytes,
                         void* stream);
int moe_grouped_swiglu_fp8(const void* a, const float* a_scales, const void* wg, const void* wu,
                           const int32_t* offs, int G, int M, int N, int K, void* h, void* ws,
                           size_t ws_bytes, void* stream);

/* int8 expert path (the reference's int8 experts: xquant / hquant / wquant,
 * kernel.cu:61-66 and kernel.cu:125-129, the int8 grouped GEMMs
 * moe_int8.h:27-45 / moe_int8.cu:391-393, the quantiser moe_wq.h:150-188).
 *
 * Per-row symmetric int8 quantisation of R rows of K bf16 values:
 *   v = the row (hadamard == 16 or 128: rotated in blocks of that size along
 *       the row by the unnormalised Walsh-Hadamard transform, butterfly stages
 *       1, 2, ..., hadamard / 2),
 *   q = clamp(rint(v * (127 / max|v|)), -127, 127), 0 for an all-zero row,
 *   scales[r] = (max|v| / 127) * scale_mul.
 * group_counts (may be NULL): row r is skipped (q and scales untouched) when
 * group_counts[r / group_rows] == 0; group_rows must divide R, at most 4096
 * groups.  K % 16 == 0 (K % 128 with the
 * 128-point rotation), K <= 16384. */
int moe_quant_rows_i8(const void* x, long long R, int K, int hadamard, float scale_mul,
                      int group_rows, const int32_t* group_counts, int8_t* q, float* scales,
                      void* stream);

/* int8 grouped GEMM: groups as moe_grouped_gemm over M operand rows; w
 * [G, N, K] int8; int32 accumulation (exact), then
 *   out[r, n] = bf16(float(acc) * (sa(r) * w_scales[g, n])).
 * Operand row r is row a_rows[r] of a (a_rows NULL: row r; a_rows lets the
 * GEMM read token rows through moe_permute's row_token instead of a gather)
 * and sa(r) its scale a_scales[a_rows[r]]; a row i of an identity group
 * reads ident_a[i] and ident_scales[i].  a_rows values must be rows of a.
 * K % 128 == 0. */
int moe_grouped_gemm_i8(const int8_t* a, const float* a_scales, const int32_t* a_rows,
                        const int8_t* w, const float* w_scales, const int32_t* offs, int G, int M,
                        int N, int K, const int8_t* ident_a, const float* ident_scales,
                        int ident_m, void* out, void* ws, size_t ws_bytes, void* stream);

/* int8 SwiGLU grouped GEMM: h[r, n] = bf16(silu(g) * u) with g and u the
 * dequantised int8 products of a with wg[g] and wu[g] (scales as above). */
int moe_grouped_swiglu_i8(const int8_t* a, const float* a_scales, const int32_t* a_rows,
                          const int8_t* wg, const float* wg_scales, const int8_t* wu,
                          const float* wu_scales, const int32_t* offs, int G, int M, int N, int K,
                          const int8_t* ident_a, const float* ident_scales, int ident_m, void* h,
                          void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_ROUTE_H_ */
