// Stage 2: per-token scoring + top-k + expert histogram.
//
// Replaces the reference's topk_kernel (K:1829-1920).  That kernel gives each
// token one 32-lane warp with NE=64 experts as two scores per lane.  Here a
// token gets a group of G = min(64, E) lanes of a 64-lane wavefront, each lane
// holding V = E / G contiguous experts (one float / float2 / float4 load), so
// 64/G tokens share a wavefront when E < 64.  Reductions are xor butterflies
// inside the G-lane group.
//
// Selection is k rounds of a group argmax with ties to the lower expert index
// (K:1872-1901), the winner's owner lane masking it out.  Every value feeding
// a comparison is computed by the same fp32 operation sequence as the CPU
// restatement (det_exp / det_sigmoid, pairwise sums in butterfly order), so
// the selected ids are bit-identical to it on identical logits.
//
// The histogram is an LDS atomic per selected pair, flushed with one global
// atomic per expert per block (K:1912-1919).  Integer atomics commute, so the
// counts are deterministic.
#include "moe_common.h"
#include "moe_math.h"

namespace moe {

constexpr int kScoreSoftmax = 0, kScoreSigmoidGroup = 1, kScoreSoftmaxBias = 2;
constexpr int kTopkTokensPerBlock = 64;

template <int E>
struct TopkShape {
  static constexpr int V = E <= 64 ? 1 : E / 64;  // experts per lane
  static constexpr int G = E / V;                 // lanes per token
  static constexpr int TPW = 64 / G;              // tokens per wavefront pass
  static constexpr int ITER = kTopkTokensPerBlock / (4 * TPW);
};

__device__ __forceinline__ float group_max(float v, int G) {
  for (int o = 1; o < G; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Pairwise sum over the G-lane group: lane partials are combined with xor 1,
// 2, 4, ...; a + b == b + a, so every lane ends with the same bits.
__device__ __forceinline__ float group_sum(float v, int G) {
#pragma clang fp contract(off)
  for (int o = 1; o < G; o <<= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

template <int V>
__device__ __forceinline__ float local_pairwise_sum(const float (&e)[V]) {
#pragma clang fp contract(off)
  if constexpr (V == 1) return e[0];
  else if constexpr (V == 2) return e[0] + e[1];
  else if constexpr (V == 4) return (e[0] + e[1]) + (e[2] + e[3]);
  else {
    float s[V];
#pragma unroll
    for (int j = 0; j < V; ++j) s[j] = e[j];
#pragma unroll
    for (int w = V; w > 1; w >>= 1)
#pragma unroll
      for (int j = 0; j < w / 2; ++j) s[j] = s[2 * j] + s[2 * j + 1];
    return s[0];
  }
}

template <int V>
__device__ __forceinline__ void load_row(const float* __restrict__ p, float (&v)[V]) {
  if constexpr (V == 4) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
  } else if constexpr (V == 2) {
    const float2 a = *reinterpret_cast<const float2*>(p);
    v[0] = a.x; v[1] = a.y;
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = p[j];
  }
}

template <int E, int SCORING>
__global__ __launch_bounds__(256) void topk_kernel(
    const float* __restrict__ logits, int fold, const float* __restrict__ bias, int T, int k,
    int renorm, int n_group, int topk_group, float route_scale, float norm_min,
    float* __restrict__ lout, int* __restrict__ ids, float* __restrict__ wout,
    int* __restrict__ counts) {
#pragma clang fp contract(off)
  using S = TopkShape<E>;
  constexpr int V = S::V, G = S::G, TPW = S::TPW;
  constexpr float NEG_INF = -__builtin_inff();
  __shared__ int hist[E];
  const int tid = threadIdx.x;
  for (int i = tid; i < E; i += 256) hist[i] = 0;
  __syncthreads();

  const int lane = tid & 63, wave = tid >> 6;
  const int sub = lane / G, gl = lane % G;
  const int e0 = gl * V;  // first expert of this lane
  float b[V];
#pragma unroll
  for (int j = 0; j < V; ++j) b[j] = bias ? bias[e0 + j] : 0.0f;
  const int in_stride = fold ? 2 * E : E;

  for (int it = 0; it < S::ITER; ++it) {
    const long long t =
        (long long)blockIdx.x * kTopkTokensPerBlock + (it * 4 + wave) * TPW + sub;
    const bool valid = t < T;
    float l[V];
    if (valid) {
      load_row<V>(logits + t * in_stride + e0, l);
      if (fold) {
        float lo[V];
        load_row<V>(logits + t * in_stride + E + e0, lo);
#pragma unroll
        for (int j = 0; j < V; ++j) l[j] = l[j] + lo[j];
      }
      if (lout) {
#pragma unroll
        for (int j = 0; j < V; ++j) lout[t * E + e0 + j] = l[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) l[j] = 0.0f;
    }

    // ---- scores: sel (what is ranked) and aux (what the weight is made of)
    float sel[V], aux[V];
    float m0 = 0.0f, fullsum = 1.0f;
    if constexpr (SCORING == kScoreSoftmax) {
#pragma unroll
      for (int j = 0; j < V; ++j) { sel[j] = l[j] + b[j]; aux[j] = sel[j]; }
      if (!renorm) {
        float m = sel[0];
#pragma unroll
        for (int j = 1; j < V; ++j) m = fmaxf(m, sel[j]);
        m = group_max(m, G);
        float e[V];
#pragma unroll
        for (int j = 0; j < V; ++j) e[j] = det_exp(sel[j] - m);
        fullsum = group_sum(local_pairwise_sum<V>(e), G);
      }
    } else if constexpr (SCORING == kScoreSoftmaxBias) {
      // K:1857-1866: e = exp(l - max), p = e * (1/sum), c = p + bias
      float m = l[0];
#pragma unroll
      for (int j = 1; j < V; ++j) m = fmaxf(m, l[j]);
      m = group_max(m, G);
      float e[V];
#pragma unroll
      for (int j = 0; j < V; ++j) e[j] = det_exp(l[j] - m);
      const float rs = __fdiv_rn(1.0f, group_sum(local_pairwise_sum<V>(e), G));
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float p = e[j] * rs;
        sel[j] = p + b[j];
        aux[j] = sel[j];
      }
    } else {  // sigmoid + selection bias, group-limited
#pragma unroll
      for (int j = 0; j < V; ++j) {
        aux[j] = det_sigmoid(l[j]);
        sel[j] = aux[j] + b[j];
      }
      if (n_group > 1) {
        const int L = (E / n_group) / V;  // lanes per group (>= 1, power of two)
        float t1 = NEG_INF, t2 = NEG_INF;
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const float v = sel[j];
          if (v > t1) { t2 = t1; t1 = v; }
          else if (v > t2) t2 = v;
        }
        for (int o = 1; o < L; o <<= 1) {
          const float o1 = __shfl_xor(t1, o, 64), o2 = __shfl_xor(t2, o, 64);
          const float n1 = fmaxf(t1, o1);
          const float n2 = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
          t1 = n1;
          t2 = n2;
        }
        const float gscore = t1 + t2;
        const int g = gl / L;
        bool kept = false;
        for (int r = 0; r < topk_group; ++r) {
          float bv = kept ? NEG_INF : gscore;
          int bg = g;
          for (int o = L; o < G; o <<= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int og = __shfl_xor(bg, o, 64);
            if (ov > bv || (ov == bv && og < bg)) { bv = ov; bg = og; }
          }
          if (bg == g) kept = true;
        }
        if (!kept) {
#pragma unroll
          for (int j = 0; j < V; ++j) sel[j] = NEG_INF;
        }
      }
    }

    // ---- k rounds of group argmax (ties -> lower index, K:1886)
    int my_id = 0;
    float my_sel = 0.0f, my_aux = 0.0f;
    float acc = 0.0f;  // sequential slot-order sum the weights divide by
    for (int r = 0; r < k; ++r) {
      float bv = sel[0], ba = aux[0];
      int bi = e0;
#pragma unroll
      for (int j = 1; j < V; ++j)
        if (sel[j] > bv) { bv = sel[j]; ba = aux[j]; bi = e0 + j; }
      for (int o = 1; o < G; o <<= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        const float oa = __shfl_xor(ba, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; ba = oa; }
      }
      if (gl == r) { my_id = bi; my_sel = bv; my_aux = ba; }
#pragma unroll
      for (int j = 0; j < V; ++j)
        if (e0 + j == bi) sel[j] = NEG_INF;
      if constexpr (SCORING == kScoreSoftmax) {
        if (r == 0) m0 = bv;
        const float e = det_exp(bv - m0);
        acc = (r == 0) ? e : acc + e;
      } else if constexpr (SCORING == kScoreSigmoidGroup) {
        acc = (r == 0) ? ba : acc + ba;
      } else {
        acc = (r == 0) ? bv : acc + bv;
      }
    }

    if (valid && gl < k) {
      float wv;
      if constexpr (SCORING == kScoreSoftmax) {
        const float e = det_exp(my_sel - m0);
        wv = __fdiv_rn(e, renorm ? acc : fullsum) * route_scale;
      } else if constexpr (SCORING == kScoreSigmoidGroup) {
        wv = (renorm ? __fdiv_rn(my_aux, acc + 1e-20f) : my_aux) * route_scale;
      } else {
        wv = __fdiv_rn(my_sel, fmaxf(acc, norm_min));  // K:1909
      }
      ids[t * k + gl] = my_id;
      wout[t * k + gl] = wv;
      atomicAdd(&hist[my_id], 1);
    }
  }
  __syncthreads();
  if (counts) {
    for (int i = tid; i < E; i += 256) {
      const int c = hist[i];
      if (c) atomicAdd(counts + i, c);
    }
  }
}

__global__ void zero_i32_kernel(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

template <int E>
static hipError_t launch_topk_e(const float* logits, int fold, const float* bias, int T, int k,
                                int scoring, int renorm, int n_group, int topk_group,
                                float route_scale, float norm_min, float* lout, int32_t* ids,
                                float* w, int32_t* counts, hipStream_t s) {
  const dim3 grid((unsigned)((T + kTopkTokensPerBlock - 1) / kTopkTokensPerBlock));
#define MOE_TOPK_ARGS                                                                      \
  grid, dim3(256), 0, s, logits, fold, bias, T, k, renorm, n_group, topk_group, route_scale, \
      norm_min, lout, ids, w, counts
  if (scoring == kScoreSoftmax)
    hipLaunchKernelGGL((topk_kernel<E, kScoreSoftmax>), MOE_TOPK_ARGS);
  else if (scoring == kScoreSigmoidGroup)
    hipLaunchKernelGGL((topk_kernel<E, kScoreSigmoidGroup>), MOE_TOPK_ARGS);
  else
    hipLaunchKernelGGL((topk_kernel<E, kScoreSoftmaxBias>), MOE_TOPK_ARGS);
#undef MOE_TOPK_ARGS
  return hipGetLastError();
}

hipError_t launch_topk(const float* logits, int fold, const float* bias, int T, int E, int k,
                       int scoring, int renorm, int n_group, int topk_group, float route_scale,
                       float norm_min, float* lout, int32_t* ids, float* w, int32_t* counts,
                       hipStream_t s) {
  if (counts) {
    hipLaunchKernelGGL(zero_i32_kernel, dim3((E + 255) / 256), dim3(256), 0, s, counts, E);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (T == 0) return hipSuccess;
#define MOE_TOPK_CASE(EE)                                                                   \
  case EE:                                                                                  \
    return launch_topk_e<EE>(logits, fold, bias, T, k, scoring, renorm, n_group, topk_group, \
                             route_scale, norm_min, lout, ids, w, counts, s);
  switch (E) {
    MOE_TOPK_CASE(8)
    MOE_TOPK_CASE(16)
    MOE_TOPK_CASE(32)
    MOE_TOPK_CASE(64)
    MOE_TOPK_CASE(128)
    MOE_TOPK_CASE(256)
    default:
      return hipErrorInvalidValue;
  }
#undef MOE_TOPK_CASE
}

}  // namespace moe
