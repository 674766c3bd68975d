// Stage 2: per-token scoring + top-k + expert histogram.
//
// Replaces the reference's topk_kernel (K:1829-1920).  That kernel gives each
// token one 32-lane warp with NE=64 experts as two scores per lane.  Here a
// token gets G = E/V lanes of a 64-lane wavefront, each holding V <= 16
// contiguous experts (G = 16 at E = 256: four tokens per wavefront), so the
// cross-lane levels of every reduction are DPP moves within a 16-lane row
// rather than LDS-routed shuffles, and 16 tokens per 256-thread block give
// the chip ~8 wavefronts per SIMD at T = 32768.
//
// Selection is k rounds of a group argmax with ties to the lower expert index
// (K:1872-1901), the winner's owner lane masking it out.  Every value feeding
// a comparison is computed by the same fp32 operation sequence as the CPU
// restatement (det_exp / det_sigmoid, pairwise sums in butterfly order), so
// the selected ids are bit-identical to it on identical logits.
//
// The histogram is an LDS atomic per selected pair, flushed with one global
// atomic per expert per block (K:1912-1919).  Integer atomics commute, so the
// counts are deterministic.  With blockcnt, a block scores the 256 / k tokens
// of one of the permute's blocks of 256 (token, slot) pairs (NPASS passes of
// its tokens per pass) and also writes that block's expert histogram, every
// entry, so the permute needs no histogram launch.
#include "score_token.h"

namespace moe {

// One token per G = E/V lanes; V contiguous experts per lane; NT threads,
// (NT / 64) * (64 / G) tokens per pass, npass passes (1 without blockcnt).
template <int E, int V, int KK, int SC, int NT>
__global__ __launch_bounds__(NT) void topk_kernel(
    const float* __restrict__ logits, int nparts, const float* __restrict__ bias, int T, int k_rt,
    int renorm, int n_group, int topk_group, float route_scale, float norm_min,
    float* __restrict__ lout, int* __restrict__ ids, float* __restrict__ wout,
    int* __restrict__ counts, int* __restrict__ blockcnt, int nblk, int npass) {
#pragma clang fp contract(off)
  constexpr int G = E / V;
  constexpr int TPB = (NT / 64) * (64 / G);
  static_assert(G >= 8 && G <= 64 && V >= 1 && V <= 16, "lane shape");
  const int k = KK > 0 ? KK : k_rt;  // compile-time for the common k: the rounds unroll
  __shared__ int hist[E];
  const int tid = threadIdx.x;
  const bool hists = counts || blockcnt;
  if (hists) {
    for (int i = tid; i < E; i += NT) hist[i] = 0;
    __syncthreads();
  }

  const int gl = tid % G;
  for (int pass = 0; pass < npass; ++pass) {
  const long long t = ((long long)blockIdx.x * npass + pass) * TPB + tid / G;
  const bool valid = t < T;
  const int e0 = gl * V;
  float l[V];
  const int np = nparts < 0 ? -nparts : nparts;
  {
    // |nparts| > 1: the row holds the partial sums of the logits side by side
    // (K partitions of the GEMM); nparts > 1: added in index order;
    // nparts < 0: (hi, lo) pairs of an fp32 weight's bf16 split per K
    // partition, folded as (sum of hi) + (sum of lo) (fold_parts)
    const int in_stride = np * E;
    if (valid) {
      const float* src = logits + t * in_stride + e0;
      load_vec<V>(src, l);
      if (nparts > 0) {
        for (int p = 1; p < np; ++p) {
          float q[V];
          load_vec<V>(src + p * E, q);
#pragma unroll
          for (int j = 0; j < V; ++j) l[j] = l[j] + q[j];
        }
      } else {
        float lo[V];
        load_vec<V>(src + E, lo);
        for (int p = 2; p < np; p += 2) {
          float q[V], r[V];
          load_vec<V>(src + p * E, q);
          load_vec<V>(src + (p + 1) * E, r);
#pragma unroll
          for (int j = 0; j < V; ++j) {
            l[j] = l[j] + q[j];
            lo[j] = lo[j] + r[j];
          }
        }
#pragma unroll
        for (int j = 0; j < V; ++j) l[j] = l[j] + lo[j];
      }
      if (lout) store_vec<V>(lout + t * E + e0, l);
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) l[j] = 0.0f;
    }
  }
  float b[V];
#pragma unroll
  for (int j = 0; j < V; ++j) b[j] = bias ? bias[e0 + j] : 0.0f;
  int my_id;
  float wv;
  score_token<E, V, KK, SC>(l, b, logits + (valid ? t : 0) * (long long)(np * E), nparts,
                            valid, gl, k_rt, renorm, n_group, topk_group, route_scale, norm_min,
                            my_id, wv);
  {
    if (valid && gl < k) {
      ids[t * k + gl] = my_id;
      wout[t * k + gl] = wv;
      if (hists) atomicAdd(&hist[my_id], 1);
    }
  }
  }
  if (hists) {
    __syncthreads();
    for (int i = tid; i < E; i += NT) {
      const int c = hist[i];
      if (counts && c) atomicAdd(counts + i, c);
      // [E, nblk]: this block is the permute's block blockIdx.x
      if (blockcnt) blockcnt[(long long)i * nblk + blockIdx.x] = c;
    }
  }
}

__global__ void zero_i32_kernel(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

template <int E, int V>
static hipError_t launch_topk_ev(const float* logits, int nparts, const float* bias, int T, int k,
                                 int scoring, int renorm, int n_group, int topk_group,
                                 float route_scale, float norm_min, float* lout, int32_t* ids,
                                 float* w, int32_t* counts, int32_t* blockcnt, hipStream_t s) {
  constexpr int TPB = 4 * (64 / (E / V));  // tokens per 256 threads
  // with blockcnt: one block per permute block of kPairsPerBlock pairs, as one
  // pass of up to 1024 threads, else in passes of 1024
  const int per_block = kPairsPerBlock / k;  // tokens
  const int npass = !blockcnt ? 1 : (per_block > 4 * TPB ? per_block / (4 * TPB) : 1);
  const int nblk = dispatch_blocks((long long)T * k);
  const dim3 grid((unsigned)(blockcnt ? nblk : (T + TPB - 1) / TPB));
  const int nt = !blockcnt ? 256 : (per_block >= 4 * TPB ? 1024 : per_block / TPB * 256);
#define MOE_TOPK_ARGS                                                                      \
  grid, dim3(nt), 0, s, logits, nparts, bias, T, k, renorm, n_group, topk_group, \
      route_scale, norm_min, lout, ids, w, counts, blockcnt, nblk, npass
#define MOE_TOPK_NT(KV, SC)                                                      \
  if (nt == 1024) hipLaunchKernelGGL((topk_kernel<E, V, KV, SC, 1024>), MOE_TOPK_ARGS); \
  else if (nt == 512) hipLaunchKernelGGL((topk_kernel<E, V, KV, SC, 512>), MOE_TOPK_ARGS); \
  else hipLaunchKernelGGL((topk_kernel<E, V, KV, SC, 256>), MOE_TOPK_ARGS);
#define MOE_TOPK_K(SC)                                        \
  if (k == 8) {                                               \
    MOE_TOPK_NT(8, SC)                                        \
  } else if (k == 2) {                                        \
    MOE_TOPK_NT(2, SC)                                        \
  } else {                                                    \
    MOE_TOPK_NT(0, SC)                                        \
  }
  if (scoring == kScoreSoftmax) {
    MOE_TOPK_K(kScoreSoftmax)
  } else if (scoring == kScoreSigmoidGroup) {
    MOE_TOPK_K(kScoreSigmoidGroup)
  } else {
    MOE_TOPK_K(kScoreSoftmaxBias)
  }
#undef MOE_TOPK_K
#undef MOE_TOPK_NT
#undef MOE_TOPK_ARGS
  return hipGetLastError();
}

// Experts per lane V = min(16, E/8, expert-group size): a token spans
// G = E/V lanes, at least 8 so every slot (k <= 8) has its own lane, at most
// 16 for E <= 256 so every reduction level is a DPP move; an expert group
// never splits a lane.
int topk_lane_width(int E, int scoring, int n_group) {
  int V = E / 8 < 16 ? E / 8 : 16;
  if (scoring == kScoreSigmoidGroup && n_group > 1) {
    const int gs = E / n_group;
    if (gs < V) V = gs;
  }
  return V < 1 ? 1 : V;
}

bool topk_block_hist_supported(int E, int k, int scoring, int n_group) {
  if (k < 1 || k > 8 || kPairsPerBlock % k != 0) return false;
  const int tpb = 4 * (64 / (E / topk_lane_width(E, scoring, n_group)));
  return (kPairsPerBlock / k) % tpb == 0;
}

hipError_t launch_topk(const float* logits, int nparts, const float* bias, int T, int E, int k,
                       int scoring, int renorm, int n_group, int topk_group, float route_scale,
                       float norm_min, float* lout, int32_t* ids, float* w, int32_t* counts,
                       int32_t* blockcnt, hipStream_t s) {
  if (counts) {
    hipLaunchKernelGGL(zero_i32_kernel, dim3((E + 255) / 256), dim3(256), 0, s, counts, E);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (T == 0) return hipSuccess;
  const int V = topk_lane_width(E, scoring, n_group);
#define MOE_TOPK_CASE(EE, VV)                                                               \
  if (E == EE && V == VV)                                                                   \
    return launch_topk_ev<EE, VV>(logits, nparts, bias, T, k, scoring, renorm, n_group,       \
                                  topk_group, route_scale, norm_min, lout, ids, w, counts,    \
                                  blockcnt, s);
  MOE_TOPK_CASE(8, 1)
  MOE_TOPK_CASE(16, 2)
  MOE_TOPK_CASE(32, 2)
  MOE_TOPK_CASE(32, 4)
  MOE_TOPK_CASE(64, 2)
  MOE_TOPK_CASE(64, 4)
  MOE_TOPK_CASE(64, 8)
  MOE_TOPK_CASE(128, 2)
  MOE_TOPK_CASE(128, 4)
  MOE_TOPK_CASE(128, 8)
  MOE_TOPK_CASE(128, 16)
  MOE_TOPK_CASE(256, 4)
  MOE_TOPK_CASE(256, 8)
  MOE_TOPK_CASE(256, 16)
#undef MOE_TOPK_CASE
  return hipErrorInvalidValue;
}

}  // namespace moe
