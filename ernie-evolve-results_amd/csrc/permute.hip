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
// fp8 variant (the reference has no routed fp8 permute): an 8-lane group owns
// one 1x128 block of a token row (16 bf16 per lane), reduces |x| max over the
// group with xor shuffles, and writes e4m3fn(clamp(x / s, +-448)) with
// s = max(amax, 1e-10) / 448 into all k rows (16 bytes per lane), plus the
// scale.
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

// One pass: a 256-thread block per 256 work items (the kernels still loop, so
// any grid is correct).  A grid capped at 65536 blocks, each thread looping
// ~1.75 times, measured 20 us slower for the C4 gather (801 vs 821 us in the
// step).
static int grid_for(long long work) {
  long long g = (work + 255) / 256;
  if (g > (1ll << 24)) g = 1ll << 24;
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

// One lane per 16 consecutive elements (two 16-byte loads, one 16-byte e4m3fn
// store per destination row); the 8 lanes of a 1x128 block reduce |x| max
// with xor shuffles, and the block's first lane writes the scale -- the 8
// blocks of a wavefront's 1 KB of fp8 row land as 8 consecutive scales, one
// 32-byte run per store instruction.
__global__ __launch_bounds__(256) void gather_fp8_kernel(const u32x4* __restrict__ x,
                                                         const int* __restrict__ pair_row,
                                                         long long nchunks, int cpr, int nb,
                                                         int k, u32x4* __restrict__ xg,
                                                         float* __restrict__ scales) {
  // chunk c = t * cpr + v: 16 elements of token t; cpr = H / 16 is a multiple
  // of 8, so the 8 lanes of a block share t and leave the loop together
  const int lane8 = threadIdx.x & 7;
  for (long long c = (long long)blockIdx.x * 256 + threadIdx.x; c < nchunks;
       c += (long long)gridDim.x * 256) {
    const int t = (int)(c / cpr);
    const int v = (int)(c - (long long)t * cpr);
    const u32x4 r0 = x[2 * c], r1 = x[2 * c + 1];
    float f[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f[2 * q] = bf16lo(r0[q]);
      f[2 * q + 1] = bf16hi(r0[q]);
      f[8 + 2 * q] = bf16lo(r1[q]);
      f[8 + 2 * q + 1] = bf16hi(r1[q]);
    }
    float amax = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) amax = fmaxf(amax, fabsf(f[q]));
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float scale = __fdiv_rn(fmaxf(amax, 1e-10f), 448.0f);
    float qv[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) qv[q] = fminf(fmaxf(__fdiv_rn(f[q], scale), -448.0f), 448.0f);
    u32x4 packed;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      packed[q] = cvt_fp8x4(qv[4 * q], qv[4 * q + 1], qv[4 * q + 2], qv[4 * q + 3]);
    const int* pr = pair_row + (long long)t * k;
    const int blk = v >> 3;
    for (int j = 0; j < k; ++j) {
      const int r = pr[j];
      if (r < 0) continue;
      st_nt(xg + (long long)r * cpr + v, packed);
      if (lane8 == 0) scales[(long long)r * nb + blk] = scale;
    }
  }
}

hipError_t launch_gather_fp8(const void* x, const int32_t* pair_row, int T, int H, int k,
                             void* xg, float* scales, hipStream_t s) {
  const int cpr = H / 16;  // 16-element chunks per row (H % 128 == 0: a multiple of 8)
  const long long nchunks = (long long)T * cpr;
  if (nchunks == 0) return hipSuccess;
  hipLaunchKernelGGL(gather_fp8_kernel, dim3(grid_for(nchunks)), dim3(256), 0, s,
                     (const u32x4*)x, pair_row, nchunks, cpr, H / 128, k, (u32x4*)xg, scales);
  return hipGetLastError();
}

}  // namespace moe
