// Measurement aid (no counterpart in the reference): plain streaming kernels
// that move the byte mixes of the path's HBM-bound stages with sequential
// addresses, so the rate this MI355X sustains for each mix can be measured
// beside the real kernels.  The gather writes 8 bytes for every byte it reads
// (token rows to their k expert rows); the combine reads 8 for every byte it
// writes; the router reads x once.  Each probe uses the cache policy of the
// stage it models (gather: ordinary loads, non-temporal stores; combine:
// non-temporal loads and stores), one 16-byte vector per lane.
//
// Two launch shapes, since neither is fastest for every mix on this GPU: one
// pass (a block per 256 vectors; the shape the real gather and combine use)
// or a grid-stride loop over at most 65536 blocks.  GS (the shape) is a
// template argument only so that a kernel trace tells the two apart.
#include "moe_common.h"

namespace moe {

constexpr long long kProbeStrideGrid = 1 << 16;

// W = the number of streams (template: each (pattern, W) pair is its own
// kernel symbol, so a kernel trace tells the probes apart); W = 0: runtime.
template <int W, bool GS>
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4* __restrict__ src,
                                                         long long n, int ways,
                                                         u32x4* __restrict__ sink) {
  const int nw = W > 0 ? W : ways;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (long long)gridDim.x * 256)
    for (int j = 0; j < nw; ++j) acc ^= ld_nt(src + (long long)j * n + i);
  // never true for the probe's inputs; keeps the loads alive
  if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0xf39cc060u) sink[0] = acc;
}

template <int W, bool GS>
__global__ __launch_bounds__(256) void probe_write_kernel(u32x4* __restrict__ dst, long long n,
                                                          int ways) {
  const int nw = W > 0 ? W : ways;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (long long)gridDim.x * 256)
    for (int j = 0; j < nw; ++j)
      st_nt(dst + (long long)j * n + i, (u32x4){(unsigned)i, (unsigned)j, 0x3f803f80u, 0u});
}

// read vector i once, write it to `ways` sequential streams dst[j*n + i]
template <bool GS>
__global__ __launch_bounds__(256) void probe_gather_mix_kernel(const u32x4* __restrict__ src,
                                                               long long n, int ways,
                                                               u32x4* __restrict__ dst) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (long long)gridDim.x * 256) {
    const u32x4 v = src[i];
    for (int j = 0; j < ways; ++j) st_nt(dst + (long long)j * n + i, v);
  }
}

// read `ways` sequential streams src[j*n + i], add them as bf16 in fp32, write
// one bf16 vector dst[i]
template <bool GS>
__global__ __launch_bounds__(256) void probe_combine_mix_kernel(const u32x4* __restrict__ src,
                                                                long long n, int ways,
                                                                u32x4* __restrict__ dst) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (long long)gridDim.x * 256) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = j < ways ? ld_nt(src + (long long)j * n + i) : (u32x4){0u, 0u, 0u, 0u};
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] += bf16lo(v[j][q]);
        acc[2 * q + 1] += bf16hi(v[j][q]);
      }
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
    st_nt(dst + i, o);
  }
}

template <bool GS>
__global__ __launch_bounds__(256) void probe_copy_kernel(const u32x4* __restrict__ src,
                                                         long long n, u32x4* __restrict__ dst) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (long long)gridDim.x * 256)
    dst[i] = src[i];
}

template <bool GS>
static void launch_probe(int pattern, const u32x4* in, u32x4* out, long long nvec, int ways,
                         hipStream_t s) {
  long long g = (nvec + 255) / 256;
  if (GS && g > kProbeStrideGrid) g = kProbeStrideGrid;
  const dim3 grid((unsigned)g), blk(256);
  switch (pattern) {
    case 0:
      if (ways == 1) hipLaunchKernelGGL((probe_read_kernel<1, GS>), grid, blk, 0, s, in, nvec, 1, out);
      else if (ways == 8) hipLaunchKernelGGL((probe_read_kernel<8, GS>), grid, blk, 0, s, in, nvec, 8, out);
      else hipLaunchKernelGGL((probe_read_kernel<0, GS>), grid, blk, 0, s, in, nvec, ways, out);
      break;
    case 1:
      if (ways == 1) hipLaunchKernelGGL((probe_write_kernel<1, GS>), grid, blk, 0, s, out, nvec, 1);
      else if (ways == 8) hipLaunchKernelGGL((probe_write_kernel<8, GS>), grid, blk, 0, s, out, nvec, 8);
      else hipLaunchKernelGGL((probe_write_kernel<0, GS>), grid, blk, 0, s, out, nvec, ways);
      break;
    case 2: hipLaunchKernelGGL(probe_gather_mix_kernel<GS>, grid, blk, 0, s, in, nvec, ways, out); break;
    case 3: hipLaunchKernelGGL(probe_combine_mix_kernel<GS>, grid, blk, 0, s, in, nvec, ways, out); break;
    default: hipLaunchKernelGGL(probe_copy_kernel<GS>, grid, blk, 0, s, in, nvec, out); break;
  }
}

// pattern: 0..4 (read, write, gather mix, combine mix, copy), plus 0x100 for
// the grid-stride shape; the caller has checked both and the sizes
hipError_t launch_stream_probe(int pattern, const void* src, void* dst, long long nvec, int ways,
                               hipStream_t s) {
  const int p = pattern & 0xff;
  if (p > 4 || nvec < 1 || (nvec + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
  if (pattern & 0x100) launch_probe<true>(p, (const u32x4*)src, (u32x4*)dst, nvec, ways, s);
  else launch_probe<false>(p, (const u32x4*)src, (u32x4*)dst, nvec, ways, s);
  return hipGetLastError();
}

}  // namespace moe
