// Stage 4: permute / gather token rows into the expert-contiguous buffer.
//
// Replaces gather_kernel (K:2206-2238).  The reference walks the ROWS of the
// permuted buffer and copies x[tok[row]] into each, so a token row is read k
// times.  Here the walk is over TOKENS: each x row is read from HBM once and
// written to its k rows (pair_row[t*k + j]), which is the algorithmic minimum
// T*H + T*k*H bytes.  Every thread moves one 16-byte vector, so a wavefront
// reads 1 KB of one token row and writes k 1 KB runs.  x is loaded with
// ordinary (temporal) loads, which hit the part of x the router GEMM left in
// the memory-side cache (MALL); the k rows are written non-temporal.
//
// fp8 variant (the reference has no routed fp8 permute): a 16-lane group owns
// one 1x128 block of a token row (8 bf16 per lane), reduces |x| max over the
// group with xor shuffles, and writes e4m3fn(clamp(x / s, +-448)) with
// s = max(amax, 1e-10) / 448 into all k rows, plus the scale.
#include "moe_common.h"

namespace moe {

template <int K>
__global__ __launch_bounds__(256) void gather_kernel(const u32x4* __restrict__ x,
                                                     const int* __restrict__ pair_row,
                                                     int total, int nvec, int k_rt,
                                                     u32x4* __restrict__ xg) {
  const int k = K > 0 ? K : k_rt;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const int t = i / nvec;
    const int v = i - t * nvec;
    const u32x4 val = x[i];
    const int* pr = pair_row + (long long)t * k;
    // all k row indices first (one wait), then the k stores
    int r[K > 0 ? K : 8];
#pragma unroll
    for (int j = 0; j < (K > 0 ? K : 8); ++j) r[j] = (K > 0 || j < k) ? pr[j] : -1;
#pragma unroll
    for (int j = 0; j < (K > 0 ? K : 8); ++j)
      if (r[j] >= 0) st_nt(xg + (long long)r[j] * nvec + v, val);
  }
}

static int grid_for(long long work) {
  long long g = (work + 255) / 256;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

hipError_t launch_gather(const void* x, int elem_bytes, const int32_t* pair_row, int T, int H,
                         int k, void* xg, hipStream_t s) {
  const int nvec = (int)((long long)H * elem_bytes / 16);
  const int total = T * nvec;  // < 2^31, checked by the caller
  if (total == 0) return hipSuccess;
  const dim3 grid(grid_for(total)), blk(256);
  const u32x4* xs = (const u32x4*)x;
  u32x4* xd = (u32x4*)xg;
  switch (k) {
    case 1: hipLaunchKernelGGL(gather_kernel<1>, grid, blk, 0, s, xs, pair_row, total, nvec, k, xd); break;
    case 2: hipLaunchKernelGGL(gather_kernel<2>, grid, blk, 0, s, xs, pair_row, total, nvec, k, xd); break;
    case 4: hipLaunchKernelGGL(gather_kernel<4>, grid, blk, 0, s, xs, pair_row, total, nvec, k, xd); break;
    case 8: hipLaunchKernelGGL(gather_kernel<8>, grid, blk, 0, s, xs, pair_row, total, nvec, k, xd); break;
    default: hipLaunchKernelGGL(gather_kernel<0>, grid, blk, 0, s, xs, pair_row, total, nvec, k, xd); break;
  }
  return hipGetLastError();
}

// e4m3fn conversion of two floats already inside [-448, 448]: the gfx950
// converter rounds to nearest even (OCP e4m3fn encoding).
__device__ __forceinline__ unsigned int cvt_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (unsigned int)w;
}

__global__ __launch_bounds__(256) void gather_fp8_kernel(const u32x4* __restrict__ x,
                                                         const int* __restrict__ pair_row,
                                                         int ngroups, int nb, int H, int k,
                                                         unsigned char* __restrict__ xg,
                                                         float* __restrict__ scales) {
  // One 16-lane group per (token, 128-block).  The 16 lanes of a group share
  // g, so they enter and leave the loop together and the xor shuffles below
  // only read lanes of their own group.
  const int lane16 = threadIdx.x & 15;
  for (int g = (blockIdx.x * 256 + threadIdx.x) >> 4; g < ngroups; g += gridDim.x * 16) {
    const int t = g / nb;
    const int blk = g - t * nb;
    const u32x4 raw = x[((long long)t * H + blk * 128) / 8 + lane16];
    float f[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f[2 * q] = bf16lo(raw[q]);
      f[2 * q + 1] = bf16hi(raw[q]);
    }
    float amax = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) amax = fmaxf(amax, fabsf(f[q]));
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float scale = __fdiv_rn(fmaxf(amax, 1e-10f), 448.0f);
    float qv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) qv[q] = fminf(fmaxf(__fdiv_rn(f[q], scale), -448.0f), 448.0f);
    u32x2 packed;
    packed[0] = cvt_fp8x4(qv[0], qv[1], qv[2], qv[3]);
    packed[1] = cvt_fp8x4(qv[4], qv[5], qv[6], qv[7]);
    const int* pr = pair_row + (long long)t * k;
    for (int j = 0; j < k; ++j) {
      const int r = pr[j];
      if (r < 0) continue;
      u32x2* dst = reinterpret_cast<u32x2*>(xg + (long long)r * H + blk * 128) + lane16;
      __builtin_nontemporal_store(packed, dst);
      if (lane16 == 0) scales[(long long)r * nb + blk] = scale;
    }
  }
}

hipError_t launch_gather_fp8(const void* x, const int32_t* pair_row, int T, int H, int k,
                             void* xg, float* scales, hipStream_t s) {
  const int nb = H / 128;
  const int ngroups = T * nb;
  if (ngroups == 0) return hipSuccess;
  const long long threads = (long long)ngroups * 16;
  hipLaunchKernelGGL(gather_fp8_kernel, dim3(grid_for(threads)), dim3(256), 0, s,
                     (const u32x4*)x, pair_row, ngroups, nb, H, k, (unsigned char*)xg, scales);
  return hipGetLastError();
}

}  // namespace moe
