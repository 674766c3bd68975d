// Stage 3: expert offsets and the stable expert-major permutation.
//
// Replaces the scan half of offsets_kernel (K:2069-2086) and dispatch_body
// (K:2109-2189).  The reference reserves positions with one global atomicAdd
// per expert per block, so a row's place inside its expert segment depends on
// which block got there first (K:2155-2158).  Here the order is fixed: pairs
// are ranked by their flat index t*k + j, giving exactly
// argsort(topk_ids.flatten(), stable) -- by expert, then ascending token.
//
// Three launches (two when E * blocks <= kDispatchSumMax: the index kernel then sums
// the block histograms itself), all integer work over the T*k ids (1 MB at
// T=32768, k=8):
//   1. pair_hist:   per block of 256 pairs, one 64-bit LDS bitmask word per
//                   (expert, wave) marks which pairs chose the expert; the
//                   popcounts are the block's expert histogram.
//   2. block_scan:  one workgroup per expert scans its column of block
//                   histograms (exclusive, in place) and writes its total.
//   3. index:       each block rebuilds its bitmasks, scans the E totals into
//                   offsets in LDS, and places every pair at
//                   offsets[e] + (rows of e in earlier blocks) + (popcount of
//                   earlier pairs of this block that chose e).
#include "moe_common.h"

namespace moe {

constexpr int kMaskWords = kPairsPerBlock / 64;  // one word per wave

__device__ __forceinline__ void build_masks(const int* __restrict__ ids, long long npairs, int E,
                                            unsigned long long* mask, int& e_out) {
  const int tid = threadIdx.x;
  const long long p = (long long)blockIdx.x * kPairsPerBlock + tid;
  int e = -1;
  if (p < npairs) {
    e = ids[p];
    if (e < 0 || e >= E) e = -1;
  }
  if (e >= 0) atomicOr(&mask[e * kMaskWords + (tid >> 6)], 1ull << (tid & 63));
  e_out = e;
}

__global__ __launch_bounds__(kPairsPerBlock) void pair_hist_kernel(
    const int* __restrict__ ids, long long npairs, int E, int nblk, int* __restrict__ blockcnt) {
  extern __shared__ unsigned long long mask[];
  const int tid = threadIdx.x;
  for (int i = tid; i < E * kMaskWords; i += kPairsPerBlock) mask[i] = 0ull;
  __syncthreads();
  int e;
  build_masks(ids, npairs, E, mask, e);
  __syncthreads();
  for (int x = tid; x < E; x += kPairsPerBlock) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < kMaskWords; ++w) c += __popcll(mask[x * kMaskWords + w]);
    blockcnt[(long long)x * nblk + blockIdx.x] = c;
  }
}

// Exclusive scan of 256 ints held one per thread; returns the exclusive prefix
// and the block total.  Wave scans by __shfl_up, then a 4-entry carry.
__device__ __forceinline__ int block_exclusive_scan(int v, int* sh4, int& total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(inc, o, 64);
    if (lane >= o) inc += n;
  }
  if (lane == 63) sh4[wave] = inc;
  __syncthreads();
  int carry = 0;
  for (int w = 0; w < wave; ++w) carry += sh4[w];
  total = sh4[0] + sh4[1] + sh4[2] + sh4[3];
  __syncthreads();
  return carry + inc - v;
}

constexpr int kScanPerThread = 4;

__global__ __launch_bounds__(256) void block_scan_kernel(int* __restrict__ blockcnt, int nblk,
                                                         int* __restrict__ totals) {
  __shared__ int sh4[4];
  int* col = blockcnt + (long long)blockIdx.x * nblk;
  const int tid = threadIdx.x;
  int carry = 0;
  for (int base = 0; base < nblk; base += 256 * kScanPerThread) {
    int v[kScanPerThread];
    int s = 0;
#pragma unroll
    for (int i = 0; i < kScanPerThread; ++i) {
      const int idx = base + tid * kScanPerThread + i;
      v[i] = idx < nblk ? col[idx] : 0;
      s += v[i];
    }
    int total;
    int ex = block_exclusive_scan(s, sh4, total) + carry;
#pragma unroll
    for (int i = 0; i < kScanPerThread; ++i) {
      const int idx = base + tid * kScanPerThread + i;
      if (idx < nblk) col[idx] = ex;
      ex += v[i];
    }
    carry += total;
  }
  if (tid == 0) totals[blockIdx.x] = carry;
}

// Exclusive scan of cnt[0..E) into offs[0..E] held in LDS (E <= 1024).
__device__ __forceinline__ void lds_offsets(const int* __restrict__ cnt, int E, int* offs,
                                            int* sh4) {
  const int tid = threadIdx.x;
  int v[4];
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid * 4 + i;
    v[i] = idx < E ? cnt[idx] : 0;
    s += v[i];
  }
  int total;
  int ex = block_exclusive_scan(s, sh4, total);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid * 4 + i;
    if (idx < E) offs[idx] = ex;
    ex += v[i];
  }
  if (tid == 0) offs[E] = total;
}

// Small problems (E * ncol <= kDispatchSumMax): dispatch_index_kernel reads
// the raw block histograms itself -- each block sums, per expert, the counts
// of the blocks before it and of all blocks -- so block_scan_kernel is not
// launched.  The histograms may be finer than the index blocks: ncol columns
// of sub-blocks, sub of them per index block (the small-E route kernel's
// 32-token tiles), summed the same way.
// P = 256 / E lanes (a power of two, at most 64) share one expert's column.
constexpr int kColBatch = 8;
__device__ __forceinline__ void column_sums(const int* __restrict__ blockcnt, int ncol, int sub,
                                            int E, int* base_out, int* tot_out) {
  const int tid = threadIdx.x;
  int P = 64;
  while (P > 1 && P * E > kPairsPerBlock) P >>= 1;
  const int per = kPairsPerBlock / P;  // experts handled per pass
  for (int e0 = 0; e0 < E; e0 += per) {
    const int e = e0 + tid / P, j = tid % P;
    int before = 0, all = 0;
    if (tid / P < per && e < E) {
      const int* col = blockcnt + (long long)e * ncol;
      const int first = (int)blockIdx.x * sub;  // this block's first column
      // kColBatch independent loads per lane before any add: a lane sums up
      // to ncol / P columns, and one load at a time would pay the memory
      // latency per column
      for (int i0 = j; i0 < ncol; i0 += P * kColBatch) {
        int c[kColBatch];
#pragma unroll
        for (int u = 0; u < kColBatch; ++u) {
          const int i = i0 + u * P;
          c[u] = i < ncol ? col[i] : 0;
        }
#pragma unroll
        for (int u = 0; u < kColBatch; ++u) {
          all += c[u];
          if (i0 + u * P < first) before += c[u];
        }
      }
    }
    // reduce over the P lanes of the expert (P divides 64: groups never straddle a wave)
    for (int o = P >> 1; o > 0; o >>= 1) {
      before += __shfl_xor(before, o, 64);
      all += __shfl_xor(all, o, 64);
    }
    if (tid / P < per && e < E && j == 0) {
      base_out[e] = before;
      tot_out[e] = all;
    }
  }
}

// SUM = false: blockbase is block_scan_kernel's scanned columns [E, nblk] and
// totals its per-expert totals.  SUM = true: blockbase is raw histograms
// [E, ncol], sub columns per block (pair_hist_kernel's: ncol = nblk, sub = 1),
// summed here (totals unused).
template <bool SUM>
__global__ __launch_bounds__(kPairsPerBlock) void dispatch_index_kernel(
    const int* __restrict__ ids, long long npairs, int E, int k, int nblk, int ncol, int sub,
    const int* __restrict__ blockbase, const int* __restrict__ totals,
    int* __restrict__ row_token, int* __restrict__ pair_row, int* __restrict__ offsets_out,
    int* __restrict__ counts_out) {
  extern __shared__ unsigned long long mask[];
  int* offs = reinterpret_cast<int*>(mask + E * kMaskWords);  // [E + 1]
  int* sbase = offs + E + 1;                                   // SUM: [E] rows of e before this block
  int* stot = sbase + E;                                       // SUM: [E] totals
  __shared__ int sh4[4];
  const int tid = threadIdx.x;
  for (int i = tid; i < E * kMaskWords; i += kPairsPerBlock) mask[i] = 0ull;
  if (SUM) {
    column_sums(blockbase, ncol, sub, E, sbase, stot);
    __syncthreads();
    totals = stot;
  }
  lds_offsets(totals, E, offs, sh4);  // contains __syncthreads
  int e;
  build_masks(ids, npairs, E, mask, e);
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int i = tid; i <= E; i += kPairsPerBlock) {
      if (offsets_out) offsets_out[i] = offs[i];
      if (counts_out && i < E) counts_out[i] = totals[i];
    }
  }
  const long long p = (long long)blockIdx.x * kPairsPerBlock + tid;
  if (p >= npairs) return;
  if (e < 0) {
    pair_row[p] = -1;
    return;
  }
  const int wv = tid >> 6, bit = tid & 63;
  const unsigned long long* me = mask + e * kMaskWords;
  int rank = __popcll(me[wv] & ((1ull << bit) - 1ull));
  for (int w = 0; w < wv; ++w) rank += __popcll(me[w]);
  const int pos = offs[e] + (SUM ? sbase[e] : blockbase[(long long)e * nblk + blockIdx.x]) + rank;
  // histograms that do not match the ids (a caller's inconsistent buffers)
  // give positions outside [0, npairs): the pair is dropped (pair_row -1, which
  // the gather and the combine skip) instead of written out of bounds
  if (pos < 0 || pos >= npairs) {
    pair_row[p] = -1;
    return;
  }
  pair_row[p] = pos;
  row_token[pos] = (int)(p / k);
}

__global__ __launch_bounds__(256) void offsets_kernel(const int* __restrict__ counts, int E,
                                                      int* __restrict__ offsets) {
  __shared__ int offs[1025];
  __shared__ int sh4[4];
  lds_offsets(counts, E, offs, sh4);
  __syncthreads();
  for (int i = threadIdx.x; i <= E; i += 256) offsets[i] = offs[i];
}

hipError_t launch_offsets(const int32_t* counts, int E, int32_t* offsets, hipStream_t s) {
  hipLaunchKernelGGL(offsets_kernel, dim3(1), dim3(256), 0, s, counts, E, offsets);
  return hipGetLastError();
}

// blockcnt: [E, nblk] int32 workspace; totals: [E] int32 workspace.
hipError_t launch_dispatch_index(const int32_t* ids, int T, int E, int k, int32_t* blockcnt,
                                 int32_t* totals, int32_t* row_token, int32_t* pair_row,
                                 int32_t* offsets, int32_t* counts, hipStream_t s) {
  const long long npairs = (long long)T * k;
  const int nblk = dispatch_blocks(npairs);
  if (nblk == 0) {
    // No pairs: offsets and counts are all zero.
    hipLaunchKernelGGL(block_scan_kernel, dim3(E), dim3(256), 0, s, blockcnt, 0, totals);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (offsets) {
      hipLaunchKernelGGL(offsets_kernel, dim3(1), dim3(256), 0, s, totals, E, offsets);
      err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    if (counts) return hipMemcpyAsync(counts, totals, sizeof(int) * E, hipMemcpyDeviceToDevice, s);
    return hipSuccess;
  }
  const size_t shm_hist = sizeof(unsigned long long) * E * kMaskWords;
  hipLaunchKernelGGL(pair_hist_kernel, dim3(nblk), dim3(kPairsPerBlock), shm_hist, s, ids,
                     npairs, E, nblk, blockcnt);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  return launch_dispatch_from_hist(ids, T, E, k, blockcnt, 0, totals, row_token, pair_row,
                                   offsets, counts, s);
}

// The scan and index launches over raw block histograms already in blockcnt
// (pair_hist_kernel's, or a route kernel's epilogue).  sub_tokens = 0: one
// column per index block, [E, nblk]; else columns of sub_tokens tokens each,
// [E, ceil(T / sub_tokens)], whole columns per index block (256 / k a multiple
// of sub_tokens) and few enough for the summing path (dispatch_sum_path).
// T * k > 0.
hipError_t launch_dispatch_from_hist(const int32_t* ids, int T, int E, int k, int32_t* blockcnt,
                                     int sub_tokens, int32_t* totals, int32_t* row_token,
                                     int32_t* pair_row, int32_t* offsets, int32_t* counts,
                                     hipStream_t s) {
  const long long npairs = (long long)T * k;
  const int nblk = dispatch_blocks(npairs);
  const size_t shm_hist = sizeof(unsigned long long) * E * kMaskWords;
  hipError_t err;
  const int ncol = sub_tokens ? (T + sub_tokens - 1) / sub_tokens : nblk;
  const int sub = sub_tokens ? kPairsPerBlock / k / sub_tokens : 1;
  if (sub_tokens || dispatch_sum_path(E, nblk)) {
    // few block histograms: every index block sums them itself, no scan launch
    const size_t shm_sum = shm_hist + sizeof(int) * (3 * E + 1);
    hipLaunchKernelGGL(dispatch_index_kernel<true>, dim3(nblk), dim3(kPairsPerBlock), shm_sum, s,
                       ids, npairs, E, k, nblk, ncol, sub, blockcnt, totals, row_token, pair_row,
                       offsets, counts);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(block_scan_kernel, dim3(E), dim3(256), 0, s, blockcnt, nblk, totals);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  const size_t shm_idx = shm_hist + sizeof(int) * (E + 1);
  hipLaunchKernelGGL(dispatch_index_kernel<false>, dim3(nblk), dim3(kPairsPerBlock), shm_idx, s,
                     ids, npairs, E, k, nblk, nblk, 1, blockcnt, totals, row_token, pair_row,
                     offsets, counts);
  return hipGetLastError();
}

}  // namespace moe
