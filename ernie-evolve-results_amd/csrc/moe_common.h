// Shared types and launch helpers of libmoe_route (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;  // CDNA wavefront width

// bf16 <-> fp32 without library help: bf16 is the top half of an fp32.
__device__ __forceinline__ float bf16lo(unsigned int u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16hi(unsigned int u) { return __uint_as_float(u & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (inputs here are finite).
__device__ __forceinline__ unsigned int f2bf(float f) {
  unsigned int u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ unsigned int pack_bf16x2(float lo, float hi) {
  return f2bf(lo) | (f2bf(hi) << 16);
}

// Streaming (non-temporal) 16-byte global load / store: every byte of the
// routed rows is touched once, so they should not displace reusable lines.
__device__ __forceinline__ u32x4 ld_nt(const u32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_nt(u32x4* p, u32x4 v) { __builtin_nontemporal_store(v, p); }

// 16-byte global store with the gfx950 sc1 cache-policy bit (device scope)
// and without nt; no compiler builtin sets it on a global store.  Used for
// the combine's output rows: at the DeepSeek-V3 shape the C4 step took 1.658
// against 1.680 ms with the nt store (same process, builds alternated, each
// step after a 1 GiB rewrite), 1.640 against 1.662 ms back to back.
__device__ __forceinline__ void st_sc1(u32x4* p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

}  // namespace moe

// ---------------------------------------------------------------------------
// Host-side launch wrappers, one per stage.  Each returns hipSuccess or the
// runtime's error; argument validation happens in moe_capi.hip before them.
// ---------------------------------------------------------------------------
namespace moe {

hipError_t launch_wsplit(const float* w, __bf16* wpk, int E, int H, hipStream_t s);
hipError_t launch_router_gemm(const __bf16* x, const __bf16* w, int T, int H, int N,
                              int ksplit, float* out, hipStream_t s);
int router_gemm_ksplit(int T, int H, int N);
// blockcnt (or NULL; needs topk_block_hist_supported): also the permute's raw
// block histograms [E, dispatch_blocks(T*k)], every entry written.
hipError_t launch_topk(const float* logits, int nparts, const float* bias, int T, int E, int k,
                       int scoring, int renorm, int n_group, int topk_group, float route_scale,
                       float norm_min, float* logits_out, int32_t* ids, float* w,
                       int32_t* counts, int32_t* blockcnt, hipStream_t s);
bool topk_block_hist_supported(int E, int k, int scoring, int n_group);
// Router GEMM + scoring in one kernel (E = 256, H = 7168 or E = 128, H = 2048,
// 16 experts per scoring lane); ws holds route_fused_workspace_bytes(E, H) bytes.
bool route_fused_supported(int E, int H, int scoring, int n_group);
size_t route_fused_workspace_bytes(int E, int H);
// Whether the fused kernel can also write the permute's block histograms
// (blocks of kPairsPerBlock pairs = whole tokens, whole blocks per tile).
bool route_fused_block_hist_supported(int E, int k);
// blockcnt (or NULL): raw block histograms [E, dispatch_blocks(T*k)].
hipError_t launch_route_fused(const __bf16* x, const __bf16* w, const float* bias, int T, int E,
                              int H, int k, int scoring, int renorm, int n_group, int topk_group,
                              float route_scale, float norm_min, float* logits, int32_t* ids,
                              float* wout, int32_t* counts, int32_t* blockcnt, void* ws,
                              hipStream_t s);
// The router GEMM + scoring for few experts (route_small.hip): w bf16 [E, H]
// with E = 8 or 16, or (wf32) fp32 [E, H] with E = 8, split hi/lo in the
// kernel; H % 256 == 0.  subcnt (or NULL): the block histograms of its
// route_small_tokens()-token tiles, [E, ceil(T / route_small_tokens())].
bool route_small_supported(int E, int H, bool wf32);
int route_small_tokens();
hipError_t launch_route_small(const __bf16* x, const void* w, bool wf32, const float* bias,
                              int T, int E, int H, int k, int scoring, int renorm, int n_group,
                              int topk_group, float route_scale, float norm_min, float* logits,
                              int32_t* ids, float* wout, int32_t* counts, int32_t* subcnt,
                              hipStream_t s);
hipError_t launch_offsets(const int32_t* counts, int E, int32_t* offsets, hipStream_t s);
hipError_t launch_dispatch_index(const int32_t* ids, int T, int E, int k, int32_t* blockcnt,
                                 int32_t* totals, int32_t* row_token, int32_t* pair_row,
                                 int32_t* offsets, int32_t* counts, hipStream_t s);
// launch_dispatch_index without its histogram launch: blockcnt already holds
// the raw block histograms, [E, dispatch_blocks(T*k)] (sub_tokens = 0) or
// [E, ceil(T / sub_tokens)] of sub_tokens-token columns.  T * k > 0.
hipError_t launch_dispatch_from_hist(const int32_t* ids, int T, int E, int k, int32_t* blockcnt,
                                     int sub_tokens, int32_t* totals, int32_t* row_token,
                                     int32_t* pair_row, int32_t* offsets, int32_t* counts,
                                     hipStream_t s);
hipError_t launch_gather(const void* x, int elem_bytes, const int32_t* pair_row, int T, int H,
                         int k, void* xg, hipStream_t s);
// stage (or NULL): T * (H/128) fp32 of workspace for the token-major scales,
// then copied to the destination rows r < *nrows (offsets[E]) through row_token.
hipError_t launch_gather_fp8(const void* x, const int32_t* pair_row, const int32_t* row_token,
                             const int32_t* nrows, int T, int H, int k, void* xg, float* scales,
                             float* stage, hipStream_t s);
hipError_t launch_combine(const void* y, int y_dtype, const int32_t* pair_row, const float* w,
                          const void* shared, int T, int H, int k, void* out, hipStream_t s);

// Column tiles of the grouped GEMM for N output columns.
int grouped_gemm_n_tiles(int N, bool swiglu);
// Expert grouped GEMM (plain or SwiGLU epilogue); tile_start is [G+1] ints of
// workspace (used only for G > 256); a_scales != NULL selects an e4m3fn A with [M, K/128] fp32 scales;
// a_rows (bf16 A, may be NULL) maps operand row r to row a_rows[r] of a.
hipError_t launch_grouped_gemm(const void* a, const float* a_scales, const int32_t* a_rows,
                               const void* ident_a, int ident_m, const void* w0, const void* w1,
                               const int32_t* offs, int G, int M, int N, int K, bool swiglu,
                               void* out, int32_t* tile_start, hipStream_t s);

// int8 grouped GEMM: a / ident_a / w0 / w1 int8, per-row scales a_rs (through
// a_rs_idx when not NULL) and ident_rs, per-weight-row scales w0s / w1s [G, N].
hipError_t launch_grouped_gemm_i8(const void* a, const float* a_rs, const int32_t* a_rs_idx,
                                  const void* ident_a, const float* ident_rs, int ident_m,
                                  const void* w0, const float* w0s, const void* w1,
                                  const float* w1s, const int32_t* offs, int G, int M, int N, int K,
                                  bool swiglu, void* out, int32_t* tile_start, hipStream_t s);
// Per-row int8 quantisation, optional 16- or 128-block Walsh-Hadamard rotation
// (had = 0, 16, 128).
int quant_rows_max_k();
int quant_rows_max_groups();
hipError_t launch_quant_rows_i8(const __bf16* x, long long R, int K, int had, float scale_mul,
                                int group_rows, const int* counts, signed char* q, float* s,
                                hipStream_t st);


// Experts per lane of the scoring kernel for (E, scoring, n_group).
int topk_lane_width(int E, int scoring, int n_group);

// Number of pairs one dispatch block ranks (per-block expert bitmasks).
constexpr int kPairsPerBlock = 256;
inline int dispatch_blocks(long long npairs) {
  return (int)((npairs + kPairsPerBlock - 1) / kPairsPerBlock);
}
// Histogram columns up to which every index block sums the raw columns itself
// (no scan launch): E * ncol <= kDispatchSumMax.
constexpr long long kDispatchSumMax = 8192;
inline bool dispatch_sum_path(int E, long long ncol) { return (long long)E * ncol <= kDispatchSumMax; }

}  // namespace moe
