// Per-token scoring + top-k of the routing head, shared by the scoring
// kernel (topk.hip) and the fused GEMM + scoring kernel (route_fused.hip).
//
// Selection is k rounds of a group argmax with ties to the lower expert index
// (K:1872-1901), the winner's owner lane masking it out.  Every value feeding
// a comparison is computed by the same fp32 operation sequence as the CPU
// restatement (det_exp / det_sigmoid, pairwise sums in butterfly order), so
// the selected ids are bit-identical to it on identical logits.
#pragma once
#include "moe_common.h"
#include "moe_math.h"

namespace moe {

constexpr int kScoreSoftmax = 0, kScoreSigmoidGroup = 1, kScoreSoftmaxBias = 2;

// Partner value at butterfly level `lvl` inside aligned groups of 2^(lvl+1)
// lanes.  Levels 0-3 are DPP moves (quad_perm xor1, xor2; row_half_mirror;
// row_mirror) -- a mirror pairs lane i with the lane holding the other half
// of its 2^(lvl+1) block, exactly like an xor, so pairwise sums keep the
// adjacent-pair tree order.  Levels 4-5 cross DPP rows: xor shuffle.
template <int LVL>
__device__ __forceinline__ int partner_i(int v) {
  if constexpr (LVL == 0) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  else if constexpr (LVL == 1) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  else if constexpr (LVL == 2) return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  else if constexpr (LVL == 3) return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
  else return __shfl_xor(v, 1 << LVL, 64);
}
template <int LVL>
__device__ __forceinline__ float partner_f(float v) {
  return __int_as_float(partner_i<LVL>(__float_as_int(v)));
}

// Runtime level -> compile-time partner (levels are uniform across the wave).
#define MOE_FOR_LEVELS(LO, HI, ...)                                     \
  {                                                                     \
    if (0 >= (LO) && 0 < (HI)) { constexpr int L_ = 0; __VA_ARGS__ }   \
    if (1 >= (LO) && 1 < (HI)) { constexpr int L_ = 1; __VA_ARGS__ }   \
    if (2 >= (LO) && 2 < (HI)) { constexpr int L_ = 2; __VA_ARGS__ }   \
    if (3 >= (LO) && 3 < (HI)) { constexpr int L_ = 3; __VA_ARGS__ }   \
    if (4 >= (LO) && 4 < (HI)) { constexpr int L_ = 4; __VA_ARGS__ }   \
    if (5 >= (LO) && 5 < (HI)) { constexpr int L_ = 5; __VA_ARGS__ }   \
  }

template <int V>
__device__ __forceinline__ float local_pairwise_sum(const float (&e)[V]) {
#pragma clang fp contract(off)
  float s[V];
#pragma unroll
  for (int j = 0; j < V; ++j) s[j] = e[j];
#pragma unroll
  for (int w = V; w > 1; w >>= 1)
#pragma unroll
    for (int j = 0; j < w / 2; ++j) s[j] = s[2 * j] + s[2 * j + 1];
  return s[0];
}

// Largest of V values (a max tree: independent ops, not one dependent
// chain) and the lowest index holding it (a scan from the top, so ties keep
// the lower index).
template <int V>
__device__ __forceinline__ void local_argmax(const float (&v)[V], int e0, float& bv, int& bi) {
  float m[V];
#pragma unroll
  for (int j = 0; j < V; ++j) m[j] = v[j];
#pragma unroll
  for (int w = V; w > 1; w >>= 1)
#pragma unroll
    for (int j = 0; j < w / 2; ++j) m[j] = fmaxf(m[2 * j], m[2 * j + 1]);
  bv = m[0];
  int ix = V - 1;
#pragma unroll
  for (int j = V - 2; j >= 0; --j) ix = v[j] == bv ? j : ix;
  bi = e0 + ix;
}

// local_argmax for values that are never NaN: the max tree in IEEE
// maximum, which gfx950 issues as v_maximum3_f32 with no canonicalisation of
// operands (fmaxf quiets each operand not known to be canonical first).  For
// non-NaN inputs the result and the index are local_argmax's.
template <int V>
__device__ __forceinline__ void local_argmax_nn(const float (&v)[V], int e0, float& bv, int& bi) {
  float m[V];
#pragma unroll
  for (int j = 0; j < V; ++j) m[j] = v[j];
  // a ternary tree: each node one three-operand maximum
#pragma unroll
  for (int w = V; w > 1; w = (w + 2) / 3)
#pragma unroll
    for (int j = 0; j < (w + 2) / 3; ++j) {
      const float a = m[3 * j];
      const float b = 3 * j + 1 < w ? m[3 * j + 1] : a;
      const float c = 3 * j + 2 < w ? m[3 * j + 2] : b;
      m[j] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
    }
  bv = m[0];
  int ix = V - 1;
#pragma unroll
  for (int j = V - 2; j >= 0; --j) ix = v[j] == bv ? j : ix;
  bi = e0 + ix;
}

constexpr int ilog2c(int v) { return v <= 1 ? 0 : 1 + ilog2c(v / 2); }

// V contiguous floats; 16-byte accesses when V is a multiple of 4 (a lane's
// first expert is V-aligned and rows are E floats, so they are aligned).
template <int V>
__device__ __forceinline__ void load_vec(const float* __restrict__ p, float (&v)[V]) {
  if constexpr (V % 4 == 0) {
#pragma unroll
    for (int j = 0; j < V; j += 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p + j);
      v[j] = a[0]; v[j + 1] = a[1]; v[j + 2] = a[2]; v[j + 3] = a[3];
    }
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = p[j];
  }
}
template <int V>
__device__ __forceinline__ void store_vec(float* __restrict__ p, const float (&v)[V]) {
  if constexpr (V % 4 == 0) {
#pragma unroll
    for (int j = 0; j < V; j += 4)
      *reinterpret_cast<f32x4*>(p + j) = (f32x4){v[j], v[j + 1], v[j + 2], v[j + 3]};
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) p[j] = v[j];
  }
}

// One logit from its partial blocks (E floats apart).  nparts > 0: the
// blocks added in index order.  nparts < 0: -nparts blocks of an fp32
// weight's bf16 hi/lo split, a (hi, lo) pair per K partition; the logit is
// (sum of the hi blocks) + (sum of the lo blocks), each in K order: the
// reference's fold of the two whole half products (K:1786-1824).
template <int E>
__device__ __forceinline__ float fold_parts(const float* src, int nparts) {
#pragma clang fp contract(off)
  if (nparts > 0) {
    float v = src[0];
    for (int p = 1; p < nparts; ++p) v = v + src[p * E];
    return v;
  }
  float hi = src[0], lo = src[E];
  for (int p = 2; p < -nparts; p += 2) {
    hi = hi + src[p * E];
    lo = lo + src[(p + 1) * E];
  }
  return hi + lo;
}

// NT tokens' scores at once, each held by G = E/V consecutive lanes (lane gl
// of a token owns experts [gl*V, gl*V + V)).  Token n: l[n] the lane's
// logits, row[n] its logit row (|nparts| partial blocks of E floats side by
// side, folded by fold_parts; read only to recompute a selected expert's
// sigmoid weight), valid[n]
// false for a padding token; b: the lane's bias.  Lanes gl < k return slot
// gl's expert in id_out[n] and its weight in w_out[n].  Every lane of the
// token's G must call it (cross-lane reductions).
//
// Each token gets exactly the operation sequence of a lone token (so the
// result does not depend on NT); NT > 1 only interleaves independent
// tokens' instructions, which hides the latency of the DPP / shuffle chains.
template <int E, int V, int KK, int SC, int NT>
__device__ __forceinline__ void score_tokens(const float (&l)[NT][V], const float (&b)[V],
                                             const float* const (&row)[NT], int nparts,
                                             const bool (&valid)[NT], int gl, int k_rt,
                                             int renorm, int n_group, int topk_group,
                                             float route_scale, float norm_min,
                                             int (&id_out)[NT], float (&w_out)[NT]) {
#pragma clang fp contract(off)
  constexpr int G = E / V;
  constexpr int LG = ilog2c(G);
  constexpr float NEG_INF = -__builtin_inff();
  const int k = KK > 0 ? KK : k_rt;
  const int e0 = gl * V;
  // ---- scores: sel (what is ranked) and aux (what the weight is made of)
  float sel[NT][V];
  float fullsum[NT];
  bool kept_grp[NT];  // sigmoid rule: the lane's expert group survived the group selection
#pragma unroll
  for (int n = 0; n < NT; ++n) fullsum[n] = 1.0f;
  if constexpr (SC == kScoreSoftmax) {
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int j = 0; j < V; ++j) sel[n][j] = l[n][j] + b[j];
    if (!renorm) {
      float m[NT], sum[NT];
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        m[n] = sel[n][0];
#pragma unroll
        for (int j = 1; j < V; ++j) m[n] = fmaxf(m[n], sel[n][j]);
      }
      MOE_FOR_LEVELS(0, LG, {
        for (int n = 0; n < NT; ++n) m[n] = fmaxf(m[n], partner_f<L_>(m[n]));
      })
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        float e[V];
#pragma unroll
        for (int j = 0; j < V; ++j) e[j] = det_exp(sel[n][j] - m[n]);
        sum[n] = local_pairwise_sum<V>(e);
      }
      MOE_FOR_LEVELS(0, LG, {
        for (int n = 0; n < NT; ++n) sum[n] = sum[n] + partner_f<L_>(sum[n]);
      })
#pragma unroll
      for (int n = 0; n < NT; ++n) fullsum[n] = sum[n];
    }
  } else if constexpr (SC == kScoreSoftmaxBias) {
    // K:1857-1866: e = exp(l - max), p = e * (1/sum), c = p + bias
    float m[NT], sum[NT], e[NT][V];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      m[n] = l[n][0];
#pragma unroll
      for (int j = 1; j < V; ++j) m[n] = fmaxf(m[n], l[n][j]);
    }
    MOE_FOR_LEVELS(0, LG, {
      for (int n = 0; n < NT; ++n) m[n] = fmaxf(m[n], partner_f<L_>(m[n]));
    })
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
      for (int j = 0; j < V; ++j) e[n][j] = det_exp(l[n][j] - m[n]);
      sum[n] = local_pairwise_sum<V>(e[n]);
    }
    MOE_FOR_LEVELS(0, LG, {
      for (int n = 0; n < NT; ++n) sum[n] = sum[n] + partner_f<L_>(sum[n]);
    })
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const float rs = __fdiv_rn(1.0f, sum[n]);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float p = e[n][j] * rs;
        sel[n][j] = p + b[j];
      }
    }
  } else {  // sigmoid + selection bias, group-limited
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int j = 0; j < V; ++j) sel[n][j] = det_sigmoid(l[n][j]) + b[j];
#pragma unroll
    for (int n = 0; n < NT; ++n) kept_grp[n] = false;
    if (n_group > 1) {
      const int lgl = ilog2c((E / n_group) / V);  // log2(lanes per group), V divides the group
      float t1[NT], t2[NT], gscore[NT];
      bool kept[NT];
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        t1[n] = NEG_INF;
        t2[n] = NEG_INF;
#pragma unroll
        for (int j = 0; j < V; ++j) {
          // running top two: (t1, t2) <- top2(t1, t2, v).  sel is never NaN
          // (det_sigmoid clamps its argument), so IEEE maximum / minimum give
          // fmaxf / fminf's values without canonicalising the operands
          t2[n] = __builtin_elementwise_maximum(t2[n], __builtin_elementwise_minimum(t1[n], sel[n][j]));
          t1[n] = __builtin_elementwise_maximum(t1[n], sel[n][j]);
        }
      }
      MOE_FOR_LEVELS(0, lgl, {
        for (int n = 0; n < NT; ++n) {
          const float o1 = partner_f<L_>(t1[n]), o2 = partner_f<L_>(t2[n]);
          const float n1 = fmaxf(t1[n], o1);
          const float n2 = fmaxf(fminf(t1[n], o1), fmaxf(t2[n], o2));
          t1[n] = n1;
          t2[n] = n2;
        }
      })
      const int g = gl >> lgl;
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        gscore[n] = t1[n] + t2[n];
        kept[n] = false;
      }
      for (int r = 0; r < topk_group; ++r) {
        float bv[NT];
        int bg[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          bv[n] = kept[n] ? NEG_INF : gscore[n];
          bg[n] = g;
        }
        MOE_FOR_LEVELS(lgl, LG, {
          for (int n = 0; n < NT; ++n) {
            const float ov = partner_f<L_>(bv[n]);
            const int og = partner_i<L_>(bg[n]);
            const bool take = (ov > bv[n]) | ((ov == bv[n]) & (og < bg[n]));
            bv[n] = take ? ov : bv[n];
            bg[n] = take ? og : bg[n];
          }
        })
#pragma unroll
        for (int n = 0; n < NT; ++n) kept[n] = kept[n] | (bg[n] == g);
      }
#pragma unroll
      for (int n = 0; n < NT; ++n) kept_grp[n] = kept[n];
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int j = 0; j < V; ++j) sel[n][j] = kept[n] ? sel[n][j] : NEG_INF;
    }
  }

  // ---- k rounds of group argmax (ties -> lower index, K:1886).  Only the
  // ranked value and its index travel; the sigmoid weight of a winner is
  // recomputed from its logit afterwards (same operations, same bits).
  int my_id[NT];
  float my_sel[NT], m0[NT], acc[NT];  // acc: sequential slot-order sum the weights divide by
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    my_id[n] = 0;
    my_sel[n] = 0.0f;
    m0[n] = 0.0f;
    acc[n] = 0.0f;
  }
  // Compacted rounds (sigmoid rule, 8 lanes of 32 experts per token, one lane
  // per expert group, at most 4 groups kept, two tokens per lane group): the
  // kept groups of token 0 move to lanes 0-3 and those of token 1 to lanes
  // 4-7 (ds_bpermute, in group order), so each lane ranks one group of one
  // token and a round reduces over 4 lanes -- half the rounds' work.  The
  // winners are the same: each round takes the best remaining kept entry
  // under (value desc, index asc), and the entries of dropped groups were
  // -inf, which never win while a kept entry remains (k <= 32).
  bool compact = false;
  if constexpr (SC == kScoreSigmoidGroup && NT == 2 && G == 8 && V == 32) {
    compact = n_group == G && topk_group >= 1 && topk_group <= 4 && k <= 8;
    if (compact) {
      const int lane = (int)(threadIdx.x & 63);
      const int gb = lane & ~7;  // the lane group's first lane in the wave
      const unsigned long long kb0 = __ballot(kept_grp[0]), kb1 = __ballot(kept_grp[1]);
      const int half = gl >> 2, c = gl & 3;
      const unsigned m = (unsigned)(((half ? kb1 : kb0) >> gb) & 0xFFull);
      // the c-th (from 0) set bit of m: drop the c lowest set bits
      const unsigned m1 = m & (m - 1u), m2 = m1 & (m1 - 1u), m3 = m2 & (m2 - 1u);
      const unsigned mc = c == 0 ? m : (c == 1 ? m1 : (c == 2 ? m2 : m3));
      const bool has = mc != 0u;
      const int src = has ? (int)__builtin_ctz(mc) : gl;
      const int addr = (gb + src) * 4;
      const int ce0 = src * V;  // the first expert of the group this lane ranks
      float cs[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float a = __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(sel[0][j])));
        const float d = __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(sel[1][j])));
        // canonical once here, so the rounds' max trees need no per-use
        // canonicalisation (a value that came through an integer move is
        // not known to be)
        cs[j] = has ? __builtin_canonicalizef(half ? d : a) : NEG_INF;
      }
#pragma unroll
      for (int r = 0; r < (KK > 0 ? KK : 8); ++r) {
        if (KK == 0 && r >= k) break;
        float bv;
        int bi;
        local_argmax_nn<V>(cs, ce0, bv, bi);
        MOE_FOR_LEVELS(0, 2, {
          const float ov = partner_f<L_>(bv);
          const int oi = partner_i<L_>(bi);
          const bool take = (ov > bv) | ((ov == bv) & (oi < bi));
          bv = take ? ov : bv;
          bi = take ? oi : bi;
        })
        // the other token's winner, from the mirrored half of the 8 lanes
        const float xv = partner_f<2>(bv);
        const int xi = partner_i<2>(bi);
        const int i0 = half ? xi : bi, i1 = half ? bi : xi;
        const float v0 = half ? xv : bv, v1 = half ? bv : xv;
        my_id[0] = gl == r ? i0 : my_id[0];
        my_id[1] = gl == r ? i1 : my_id[1];
        my_sel[0] = gl == r ? v0 : my_sel[0];
        my_sel[1] = gl == r ? v1 : my_sel[1];
        const int wj = bi - ce0;  // the winner's place in this lane's group, if it is here
#pragma unroll
        for (int j = 0; j < V; ++j) cs[j] = j == wj ? NEG_INF : cs[j];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < (KK > 0 ? KK : 8); ++r) {
    if (compact) break;
    if (KK == 0 && r >= k) break;
    float bv[NT];
    int bi[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) local_argmax<V>(sel[n], e0, bv[n], bi[n]);
    MOE_FOR_LEVELS(0, LG, {
      for (int n = 0; n < NT; ++n) {
        const float ov = partner_f<L_>(bv[n]);
        const int oi = partner_i<L_>(bi[n]);
        // non-short-circuit: a select, not a branch
        const bool take = (ov > bv[n]) | ((ov == bv[n]) & (oi < bi[n]));
        bv[n] = take ? ov : bv[n];
        bi[n] = take ? oi : bi[n];
      }
    })
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      my_id[n] = gl == r ? bi[n] : my_id[n];
      my_sel[n] = gl == r ? bv[n] : my_sel[n];
#pragma unroll
      for (int j = 0; j < V; ++j) sel[n][j] = e0 + j == bi[n] ? NEG_INF : sel[n][j];
      if constexpr (SC == kScoreSoftmax) {
        if (r == 0) m0[n] = bv[n];
        const float e = det_exp(bv[n] - m0[n]);
        acc[n] = (r == 0) ? e : acc[n] + e;
      } else if constexpr (SC == kScoreSoftmaxBias) {
        acc[n] = (r == 0) ? bv[n] : acc[n] + bv[n];
      }
    }
  }
  if constexpr (SC == kScoreSigmoidGroup) {
    // a slot's weight is the sigmoid of its expert's logit; the divisor is
    // the sequential slot-order sum of those, read lane by lane from the
    // token's first k lanes
    float my_aux[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      my_aux[n] = 0.0f;
      if (valid[n] && gl < k) {
        my_aux[n] = det_sigmoid(fold_parts<E>(row[n] + my_id[n], nparts));
      }
    }
    const int base = (threadIdx.x & 63) - gl;
    for (int r = 0; r < k; ++r) {
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const float a = __shfl(my_aux[n], base + r, 64);
        acc[n] = (r == 0) ? a : acc[n] + a;
      }
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) my_sel[n] = my_aux[n];  // the weight numerator below
  }

  // lane gl < k holds slot gl (G >= 8 >= k)
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    id_out[n] = my_id[n];
    w_out[n] = 0.0f;
    if (valid[n] && gl < k) {
      float wv;
      if constexpr (SC == kScoreSoftmax) {
        const float e = det_exp(my_sel[n] - m0[n]);
        wv = __fdiv_rn(e, renorm ? acc[n] : fullsum[n]) * route_scale;
      } else if constexpr (SC == kScoreSigmoidGroup) {
        wv = (renorm ? __fdiv_rn(my_sel[n], acc[n] + 1e-20f) : my_sel[n]) * route_scale;
      } else {
        wv = __fdiv_rn(my_sel[n], fmaxf(acc[n], norm_min));  // K:1909
      }
      w_out[n] = wv;
    }
  }
}

// One token (score_tokens with NT = 1).
template <int E, int V, int KK, int SC>
__device__ __forceinline__ void score_token(const float (&l)[V], const float (&b)[V],
                                            const float* row, int nparts, bool valid, int gl,
                                            int k_rt, int renorm, int n_group, int topk_group,
                                            float route_scale, float norm_min, int& id_out,
                                            float& w_out) {
  const float(&l1)[1][V] = *reinterpret_cast<const float(*)[1][V]>(&l);
  const float* const rows[1] = {row};
  const bool v1[1] = {valid};
  int id1[1];
  float w1[1];
  score_tokens<E, V, KK, SC, 1>(l1, b, rows, nparts, v1, gl, k_rt, renorm, n_group, topk_group,
                                route_scale, norm_min, id1, w1);
  id_out = id1[0];
  w_out = w1[0];
}

}  // namespace moe
