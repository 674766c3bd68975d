// Stage 5: weighted combine (un-permute), fp32 accumulate.
//
// Replaces combine_kernel (K:2365-2428):
//   out[t] = cast(shared[t] + sum_j w[t,j] * y[pair_row[t,j]])
// Each thread produces one 16-byte vector of one output row.  All k row
// loads are issued before the reduction (the reference found serialising them
// cost ~12% of bandwidth, K:2358-2363) and use non-temporal hints, since every
// byte of y is read exactly once (K:2391-2404).
#include "moe_common.h"

namespace moe {

// bf16 vector: 8 elements; fp32 vector: 4 elements.
template <bool BF16>
struct Vec;
template <>
struct Vec<true> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(u32x4 v, float (&f)[8]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) { f[2 * q] = bf16lo(v[q]); f[2 * q + 1] = bf16hi(v[q]); }
  }
  static __device__ __forceinline__ u32x4 pack(const float (&f)[8]) {
    u32x4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = pack_bf16x2(f[2 * q], f[2 * q + 1]);
    return v;
  }
};
template <>
struct Vec<false> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void unpack(u32x4 v, float (&f)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) f[q] = __uint_as_float(v[q]);
  }
  static __device__ __forceinline__ u32x4 pack(const float (&f)[4]) {
    u32x4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = __float_as_uint(f[q]);
    return v;
  }
};

template <int K, bool BF16>
__global__ __launch_bounds__(256) void combine_kernel(const u32x4* __restrict__ y,
                                                      const int* __restrict__ pair_row,
                                                      const float* __restrict__ w,
                                                      const u32x4* __restrict__ shared,
                                                      int total, int nvec,
                                                      u32x4* __restrict__ out) {
  using VT = Vec<BF16>;
  constexpr int NE = VT::N;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const int t = i / nvec;
    const int v = i - t * nvec;
    int r[K];
    float wk[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      r[j] = pair_row[(long long)t * K + j];
      wk[j] = w[(long long)t * K + j];
    }
    // All k loads are unconditional so they issue back to back; a pair
    // without a row (pair_row < 0) loads this thread's own output vector
    // instead (valid memory) and the value is discarded by the select below.
    u32x4 yv[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const u32x4* src = r[j] >= 0 ? y + (long long)r[j] * nvec + v : out + i;
      yv[j] = ld_nt(src);
    }
#pragma unroll
    for (int j = 0; j < K; ++j)
      if (r[j] < 0) yv[j] = (u32x4){0u, 0u, 0u, 0u};
    float acc[NE];
    if (shared) {
      VT::unpack(ld_nt(shared + i), acc);
    } else {
#pragma unroll
      for (int e = 0; e < NE; ++e) acc[e] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
      float f[NE];
      VT::unpack(yv[j], f);
      const float wj = r[j] >= 0 ? wk[j] : 0.0f;
#pragma unroll
      for (int e = 0; e < NE; ++e) acc[e] += wj * f[e];
    }
    st_nt(out + i, VT::pack(acc));
  }
}

// Wave-chunk variant: a wavefront owns VPW * 64 consecutive vectors of ONE
// output row (needs nvec % (VPW*64) == 0, e.g. H % 512 == 0 for bf16 at
// VPW = 1), so the row's k indices and weights are wave-uniform (scalar
// registers) and each lane keeps VPW * k independent 16-byte loads in flight,
// every one part of a 1 KB contiguous wave access.  Measured on MI355X at the
// DeepSeek-V3 shape: within ~3% of a synthetic kernel with the same byte mix
// (8 sequential read streams + 1 write stream, 731 us).
template <int K, bool BF16, int VPW>
__global__ __launch_bounds__(256) void combine_wave_kernel(const u32x4* __restrict__ y,
                                                           const int* __restrict__ pair_row,
                                                           const float* __restrict__ w,
                                                           const u32x4* __restrict__ shared,
                                                           int total, int nvec,
                                                           u32x4* __restrict__ out) {
  using VT = Vec<BF16>;
  constexpr int NE = VT::N;
  const int lane = threadIdx.x & 63;
  const int nw = gridDim.x * 4;
  for (int c = (blockIdx.x * 256 + threadIdx.x) >> 6; c * VPW * 64 < total; c += nw) {
    const int i0 = c * VPW * 64;
    const int t = i0 / nvec;
    const int v0 = i0 - t * nvec + lane;
    int r[K];
    float wk[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      r[j] = __builtin_amdgcn_readfirstlane(pair_row[(long long)t * K + j]);
      wk[j] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(w[(long long)t * K + j])));
    }
    // Unconditional loads (see combine_kernel): all VPW*k issue back to back.
    u32x4 yv[VPW][K];
#pragma unroll
    for (int j = 0; j < K; ++j)
#pragma unroll
      for (int q = 0; q < VPW; ++q) {
        const u32x4* src = r[j] >= 0 ? y + (long long)r[j] * nvec + v0 + q * 64
                                     : out + i0 + q * 64 + lane;
        yv[q][j] = ld_nt(src);
      }
#pragma unroll
    for (int j = 0; j < K; ++j)
      if (r[j] < 0)
#pragma unroll
        for (int q = 0; q < VPW; ++q) yv[q][j] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < VPW; ++q) {
      float acc[NE];
      if (shared) {
        VT::unpack(ld_nt(shared + i0 + q * 64 + lane), acc);
      } else {
#pragma unroll
        for (int e = 0; e < NE; ++e) acc[e] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < K; ++j) {
        float f[NE];
        VT::unpack(yv[q][j], f);
        const float wj = r[j] >= 0 ? wk[j] : 0.0f;
#pragma unroll
        for (int e = 0; e < NE; ++e) acc[e] += wj * f[e];
      }
      st_sc1(out + i0 + q * 64 + lane, VT::pack(acc));
    }
  }
}

template <bool BF16>
static hipError_t launch_combine_t(const void* y, const int32_t* pair_row, const float* w,
                                   const void* shared, int total, int nvec, int k, void* out,
                                   hipStream_t s) {
  long long g = (total + 255) / 256;
  if (g > (1ll << 24)) g = 1ll << 24;
  const dim3 grid((unsigned)g), blk(256);
  const u32x4* ys = (const u32x4*)y;
  const u32x4* sh = (const u32x4*)shared;
  u32x4* o = (u32x4*)out;
  // one 64-vector chunk per wave, one pass of blocks over the rows (a grid
  // capped at 65536 blocks, each wave looping ~1.75 times, measured 15 us
  // slower at the DeepSeek-V3 shape: 749 vs 734 us in the step)
  const bool wave = nvec % 64 == 0;
  long long wg = ((long long)total / 64 + 3) / 4;
  if (wg > (1ll << 24)) wg = 1ll << 24;
  const dim3 wgrid((unsigned)(wg < 1 ? 1 : wg));
#define MOE_COMBINE_CASE(KK)                                                                   \
  case KK:                                                                                     \
    if (wave)                                                                                  \
      hipLaunchKernelGGL((combine_wave_kernel<KK, BF16, 1>), wgrid, blk, 0, s, ys, pair_row, w,  \
                         sh, total, nvec, o);                                                  \
    else                                                                                       \
      hipLaunchKernelGGL((combine_kernel<KK, BF16>), grid, blk, 0, s, ys, pair_row, w, sh,       \
                         total, nvec, o);                                                      \
    break;
  switch (k) {
    MOE_COMBINE_CASE(1)
    MOE_COMBINE_CASE(2)
    MOE_COMBINE_CASE(3)
    MOE_COMBINE_CASE(4)
    MOE_COMBINE_CASE(5)
    MOE_COMBINE_CASE(6)
    MOE_COMBINE_CASE(7)
    MOE_COMBINE_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef MOE_COMBINE_CASE
  return hipGetLastError();
}

// y_dtype: 0 = bf16, 1 = fp32 (checked by the caller)
hipError_t launch_combine(const void* y, int y_dtype, const int32_t* pair_row, const float* w,
                          const void* shared, int T, int H, int k, void* out, hipStream_t s) {
  const int elem = y_dtype == 0 ? 2 : 4;
  const int nvec = (int)((long long)H * elem / 16);
  const int total = T * nvec;
  if (total == 0) return hipSuccess;
  if (y_dtype == 0) return launch_combine_t<true>(y, pair_row, w, shared, total, nvec, k, out, s);
  return launch_combine_t<false>(y, pair_row, w, shared, total, nvec, k, out, s);
}

}  // namespace moe
