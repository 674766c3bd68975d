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
#include <type_traits>

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
// 32-byte run per store instruction.  With `stage`, the scale goes once into
// the token-major stage[t * nb + blk] instead of into the k destination rows
// (a 256-thread block writes 32 consecutive scales: one whole 128-byte line),
// and scatter_scales_kernel copies whole destination rows afterwards: the k
// scattered 32-byte runs per token cost more than the fp8 rows they describe
// (C5: gather 438 against 403 us and the combine after it 762 against 732 us
// with and without them).
// One 16-element chunk c of x: its e4m3fn bytes and its 1x128 block's scale.
// The 8 lanes of a block (consecutive, 8-aligned) must all call it.
__device__ __forceinline__ void quant_chunk(const u32x4* __restrict__ x, long long c,
                                            u32x4& packed, float& scale) {
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
  scale = __fdiv_rn(fmaxf(amax, 1e-10f), 448.0f);
  float qv[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) qv[q] = fminf(fmaxf(__fdiv_rn(f[q], scale), -448.0f), 448.0f);
#pragma unroll
  for (int q = 0; q < 4; ++q)
    packed[q] = cvt_fp8x4(qv[4 * q], qv[4 * q + 1], qv[4 * q + 2], qv[4 * q + 3]);
}

__global__ __launch_bounds__(256) void gather_fp8_kernel(const u32x4* __restrict__ x,
                                                         const int* __restrict__ pair_row,
                                                         long long nchunks, int cpr, int nb,
                                                         int k, u32x4* __restrict__ xg,
                                                         float* __restrict__ scales,
                                                         float* __restrict__ stage) {
  // chunk c = t * cpr + v: 16 elements of token t; cpr = H / 16 is a multiple
  // of 8, so the 8 lanes of a block share t and leave the loop together
  const int lane8 = threadIdx.x & 7;
  for (long long c = (long long)blockIdx.x * 256 + threadIdx.x; c < nchunks;
       c += (long long)gridDim.x * 256) {
    const int t = (int)(c / cpr);
    const int v = (int)(c - (long long)t * cpr);
    u32x4 packed;
    float scale;
    quant_chunk(x, c, packed, scale);
    const int* pr = pair_row + (long long)t * k;
    const int blk = v >> 3;
    if (stage && lane8 == 0) stage[(long long)t * nb + blk] = scale;
    for (int j = 0; j < k; ++j) {
      const int r = pr[j];
      if (r < 0) continue;
      st_nt(xg + (long long)r * cpr + v, packed);
      if (!stage && lane8 == 0) scales[(long long)r * nb + blk] = scale;
    }
  }
}

// scales[r] = stage[row_token[r]] for the rows r < offsets[E] that exist, as
// whole rows in destination order: consecutive lanes write consecutive
// 16-byte pieces (nb % 4 == 0) or floats, so every store is part of a
// contiguous run and the lines go out whole.
// Each thread moves kScatterItems pieces, 256 * gridDim apart (a block's
// pieces of one round are contiguous), all loads before the stores: the stage
// is read from L2 or the memory-side cache, and one load in flight per lane
// left the kernel latency-bound.
constexpr int kScatterItems = 4;
template <int W>
__global__ __launch_bounds__(256) void scatter_scales_kernel(const float* __restrict__ stage,
                                                             const int* __restrict__ row_token,
                                                             const int* __restrict__ nrows_p,
                                                             long long nitems, int nb, int T,
                                                             float* __restrict__ scales) {
  using Piece = typename std::conditional<W == 4, u32x4, float>::type;
  const int per_row = nb / W;
  const long long nrows = *nrows_p;
  const long long stride = (long long)gridDim.x * 256;
  const long long q0 = (long long)blockIdx.x * 256 + threadIdx.x;
  Piece v[kScatterItems];
  long long dst[kScatterItems];
#pragma unroll
  for (int i = 0; i < kScatterItems; ++i) {
    const long long q = q0 + i * stride;
    const long long r = q / per_row;
    dst[i] = -1;
    if (q < nitems && r < nrows) {
      const int p = (int)(q - r * per_row);
      const long long t = row_token[r];
      if (t >= 0 && t < T) {  // a row the index pass dropped holds no token
        v[i] = reinterpret_cast<const Piece*>(stage + t * nb)[p];
        dst[i] = r * per_row + p;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kScatterItems; ++i) {
    if (dst[i] < 0) continue;
    if constexpr (W == 4) st_nt(reinterpret_cast<u32x4*>(scales) + dst[i], v[i]);
    else scales[dst[i]] = v[i];
  }
}

hipError_t launch_gather_fp8(const void* x, const int32_t* pair_row, const int32_t* row_token,
                             const int32_t* nrows, int T, int H, int k, void* xg, float* scales,
                             float* stage, hipStream_t s) {
  const int cpr = H / 16;  // 16-element chunks per row (H % 128 == 0: a multiple of 8)
  const int nb = H / 128;
  const long long nchunks = (long long)T * cpr;
  if (nchunks == 0) return hipSuccess;
  hipLaunchKernelGGL(gather_fp8_kernel, dim3(grid_for(nchunks)), dim3(256), 0, s,
                     (const u32x4*)x, pair_row, nchunks, cpr, nb, k, (u32x4*)xg, scales, stage);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !stage) return e;
  // 16-byte pieces only where every piece is 16-byte aligned in both buffers
  // (scales needs only 4-byte alignment at the C ABI)
  const bool vec = nb % 4 == 0 && ((uintptr_t)scales & 15u) == 0 && ((uintptr_t)stage & 15u) == 0;
  const long long nitems = (long long)T * k * (vec ? nb / 4 : nb);
  const dim3 sgrid((unsigned)((nitems + 256LL * kScatterItems - 1) / (256LL * kScatterItems)));
  if (vec)
    hipLaunchKernelGGL(scatter_scales_kernel<4>, sgrid, dim3(256), 0, s, stage, row_token, nrows,
                       nitems, nb, T, scales);
  else
    hipLaunchKernelGGL(scatter_scales_kernel<1>, sgrid, dim3(256), 0, s, stage, row_token, nrows,
                       nitems, nb, T, scales);
  return hipGetLastError();
}

}  // namespace moe
