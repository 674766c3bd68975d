// Stages 1-2 fused for few experts (E = 8 or 16, bf16 weights): the router
// GEMM and the scoring in one kernel.
//
// Replaces, for the Mixtral-like shapes, the reference's cublasGemmEx router
// GEMM (K:4327-4339) followed by topk_kernel (K:1829-1920).  With E <= 16 the
// router GEMM is an x stream: 8 or 16 weight rows (64-128 KB at H = 4096,
// resident in L2) against every token row.  The two-kernel path needs the K
// range split over four blocks to fill the chip, and a second kernel to add
// the partial logits and score them.  Here a 256-thread block owns 32 tokens
// and its four waves split K instead (a quarter each), so the partial sums
// meet in LDS and the same block scores its tokens:
//
//   K loop   each wave streams its quarter of K through its own LDS ring:
//            64-wide K steps of the 32 token rows and the E weight rows,
//            brought in by the gfx950 LDS DMA (8 rows x 128 B per wave
//            instruction, XOR-swizzled 16-byte chunks), 2 steps in flight,
//            then two v_mfma_f32_16x16x32_bf16 (one per 16-row half) per
//            32 k.  Only the wave that loads a ring reads it, so the loop
//            has no barrier.  The weight fragment's 16 columns hold expert
//            fr % E (at E = 8 columns 8..15 repeat 0..7 and are dropped).
//            Measured at C2, slower alternatives: the fragments loaded
//            straight into registers (16 rows x 64 B per load instruction,
//            no LDS) 16.5 us; the standalone GEMM's pipeline (two waves per
//            quarter sharing a ring, one block-wide barrier per step)
//            15.5 us; 16 weight rows loaded at E = 8 13.2 us; shipped 13.0 us,
//            against 12.2 + 4.8 us for the two-kernel path's GEMM and scoring.
//   epilogue the four partial tiles go to LDS (over the rings) as
//            [token][quarter][expert]; the logits are their sum in quarter
//            order ((p0 + p1) + p2) + p3 -- the order the scoring kernel adds
//            the two-kernel path's four K partitions in, with the same K steps
//            and the same MFMA lane-to-k mapping, so the logits equal that
//            path's where it splits K in four (C2) -- and G = E/V lanes per
//            token score them with the scoring kernel's per-token routine
//            (bit-identical selection on identical logits).  The block's
//            expert histogram goes to counts and, with subcnt, to column
//            blockIdx.x of the [E, ceil(T/32)] 32-token histograms the
//            permute's index kernel sums (no histogram launch).
#include "moe_common.h"
#include "score_token.h"

namespace moe {

namespace rs {
constexpr int TB = 32;  // tokens per block (two 16-row MFMA fragments)
// K parts (one wave each) and ring stages per wave.  Measured at C2 (T = 8192,
// H = 4096, E = 8; kernel-trace medians): 4 waves x 3 stages 13.0 us, x 4-6
// stages 13.1-13.3, 8 waves x 3 stages 14.1, 2 waves x 8-12 stages 19-20;
// 16-token blocks (512 of them, each reading the weight for half as many
// tokens) 12.6 us with the C2 step unchanged (0.0819-0.0823 ms).
constexpr int NG = 4, NS = 3;
constexpr int BK = 64, ROWB = BK * 2, CH = 8, RPI = 8;  // K step, LDS row bytes, 16-byte chunks
__device__ __forceinline__ int swz(int r) { return (r >> 1) & (CH - 1); }
}  // namespace rs

// NG waves, wave g owning K part g (H / NG, whole 64-wide steps) of all 32
// tokens, each on its own NS-stage LDS ring.  HL = 1: w is the bf16 weight
// [E, H].  HL = 2 (E = 8): w is an fp32 weight [E, H]; its rows come into the
// ring as fp32 and each lane splits its 8 k into hi = bf16(w) and
// lo = bf16(w - hi) (the reference's wsplit_kernel, K:1786-1824), so the 16
// fragment columns are the 8 hi then the 8 lo rows, and a logit is
// (sum of the NG hi partials) + (sum of the NG lo partials), each in K order:
// the reference's fold of the full hi and lo products.
template <int E, int V, int KK, int SC, int NG, int NS, int HL>
__global__ __launch_bounds__(64 * NG) void route_small_kernel(
    const __bf16* __restrict__ x, const void* __restrict__ w, const float* __restrict__ bias,
    int T, int H, int k_rt, int renorm, int n_group, int topk_group, float route_scale,
    float norm_min, float* __restrict__ logits, int* __restrict__ ids, float* __restrict__ wout,
    int* __restrict__ counts, int* __restrict__ subcnt, int nsub) {
#pragma clang fp contract(off)
  using namespace rs;
  constexpr int NT = 64 * NG;
  static_assert((E == 8 || E == 16) && (HL == 1 || HL == 2) && HL * E <= 16,
                "one 16-column weight fragment");
  constexpr int NW = HL * E;    // weight fragment columns in use
  constexpr int NP = NG * HL;   // partial logit blocks per token
  constexpr int NPF = HL == 2 ? -NP : NP;  // their fold (fold_parts): hi sum + lo sum
  // a stage: TB token rows (128 B each), then the E weight rows of one K step,
  // 128 B of bf16 (HL = 1) or 256 B of fp32 (HL = 2) each; 1 KB per DMA
  // instruction (8 token rows, 8 bf16 or 4 fp32 weight rows)
  constexpr int WROWB = HL == 2 ? 2 * ROWB : ROWB;
  constexpr int STAGE_B = TB * ROWB + E * WROWB;
  constexpr int NQX = TB / RPI;
  constexpr int NQ = NQX + E * WROWB / 1024;
  static_assert(E * WROWB % 1024 == 0, "whole DMA instructions");
  constexpr int RING_B = NG * NS * STAGE_B;
  constexpr int PART_B = TB * NP * E * 4;
  // the partial tiles reuse the rings once every wave has left its K loop
  __shared__ __attribute__((aligned(1024))) char lds[RING_B > PART_B ? RING_B : PART_B];
  __shared__ int hist[E];
  float* const part = reinterpret_cast<float*>(lds);  // [token][K part][half][expert]

  const int lane = threadIdx.x & 63;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // this wave's K part
  const long long m0 = (long long)blockIdx.x * TB;
  const int kw = H / NG;
  const int KT = kw / BK;
  char* const wring = lds + g * NS * STAGE_B;

  // Per-lane source of each DMA instruction of a stage (its K step 0): token
  // rows (past T: a copy of row T-1, never stored) with 16-byte chunk p of row
  // r at physical chunk p ^ swz(r); then the weight rows, bf16 the same way, or
  // fp32 with 32-byte chunk c of row e at physical chunk c ^ e.
  const char* src[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    if (q < NQX) {
      const int r = q * RPI + lane / CH;  // stage row
      long long t = m0 + r;
      if (t >= T) t = T - 1;
      src[q] = reinterpret_cast<const char*>(x + t * H + (long long)g * kw +
                                             ((lane % CH) ^ swz(r)) * 8);
    } else if constexpr (HL == 1) {
      const int r = (q - NQX) * RPI + lane / CH;  // weight row
      src[q] = reinterpret_cast<const char*>(static_cast<const __bf16*>(w) + (long long)r * H +
                                             (long long)g * kw + ((lane % CH) ^ swz(TB + r)) * 8);
    } else {
      const int e = (q - NQX) * 4 + lane / 16;  // weight row: 16 lanes x 16 B
      const int pc = (lane % 16) / 2, hf = lane % 2;  // physical 32-byte chunk, its half
      src[q] = reinterpret_cast<const char*>(static_cast<const float*>(w) + (long long)e * H +
                                             (long long)g * kw + (pc ^ e) * 8 + hf * 4);
    }
  }
  auto issue = [&](int kt, int st) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      auto* dst = (__attribute__((address_space(3))) void*)(wring + st * STAGE_B + q * 1024);
      const int step_b = (q < NQX || HL == 1) ? BK * 2 : BK * 4;  // bytes per K step
      __builtin_amdgcn_global_load_lds((const void*)(src[q] + (long long)kt * step_b), dst, 16, 0,
                                       0);
    }
  };

  f32x4 acc0 = (f32x4){0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
#pragma unroll
  for (int st = 0; st < NS - 1; ++st)
    if (st < KT) issue(st, st);
  const int fr = lane & 15, fc = lane >> 4;
  for (int kt = 0; kt < KT; ++kt) {
    // Stage kt is in LDS once at most NS-2 later stages are outstanding (only
    // this wave's DMA loads are in flight here, and only this wave reads its
    // ring: no barrier).  The slot refilled next held stage kt-1, whose
    // fragment reads the MFMAs of step kt-1 have consumed.
    if (kt + NS - 2 < KT)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * NQ) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (kt + NS - 1 < KT) issue(kt + NS - 1, (kt + NS - 1) % NS);
    const char* sb = wring + (kt % NS) * STAGE_B;
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      // lane (fr, fc) feeds k = kk*32 + fc*8 .. +8 of row fr: the standalone
      // GEMM's mapping, so the parts' sums are its K partitions' bit for bit
      const int c = kk * 4 + fc;
      const int r1 = 16 + fr;
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(sb + fr * ROWB + ((c ^ swz(fr)) * 16));
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(sb + r1 * ROWB + ((c ^ swz(r1)) * 16));
      const char* wb = sb + TB * ROWB;
      bf16x8 b;
      if constexpr (HL == 1) {
        // the weight fragment's 16 columns: weight row fr % E (at E = 8
        // columns 8..15 repeat 0..7 and are dropped)
        const int rb = fr % E;
        b = *reinterpret_cast<const bf16x8*>(wb + rb * ROWB + ((c ^ swz(TB + rb)) * 16));
      } else {
        // columns 0..7: hi of row fr, 8..15: lo of row fr - 8, from the same
        // 8 fp32 (lanes fr and fr + 8 read one address)
        const int e = fr & 7;
        const f32x4* pv = reinterpret_cast<const f32x4*>(wb + e * WROWB + (c ^ e) * 32);
        const f32x4 v0 = pv[0], v1 = pv[1];
        const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        unsigned int hv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const unsigned int h = f2bf(v[i]);
          hv[i] = fr < 8 ? h : f2bf(v[i] - __uint_as_float(h << 16));
        }
        const u32x4 pk = {hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16),
                          hv[6] | (hv[7] << 16)};
        b = __builtin_bit_cast(bf16x8, pk);
      }
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b, acc1, 0, 0, 0);
    }
  }
  __syncthreads();  // every ring is read: the partial tiles may overwrite them

  // ---- partial tiles to LDS: lane (fr, fc) holds column fr, rows fc*4 .. fc*4+3
  // of each 16-row half
  // column fr = half h, expert e; the partial block index is g * HL + h
  if (fr < NW) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      part[((fc * 4 + i) * NG + g) * NW + fr] = acc0[i];
      part[((16 + fc * 4 + i) * NG + g) * NW + fr] = acc1[i];
    }
  }
  const bool hists = counts || subcnt;
  if (threadIdx.x < E) hist[threadIdx.x] = 0;
  __syncthreads();

  // ---- scoring: G = E/V lanes per token
  constexpr int G = E / V;
  constexpr int TPP = NT / G;  // tokens per pass
  static_assert(TB % TPP == 0 || TPP % TB == 0, "token passes");
  const int gl = threadIdx.x % G;
  const int e0 = gl * V;
  float bl[V];
#pragma unroll
  for (int j = 0; j < V; ++j) bl[j] = bias ? bias[e0 + j] : 0.0f;
  const int k = KK > 0 ? KK : k_rt;
  for (int tl = threadIdx.x / G; tl < TB; tl += TPP) {
    const long long t = m0 + tl;
    const float* row = part + tl * NP * E;
    float l[1][V];
#pragma unroll
    for (int j = 0; j < V; ++j) l[0][j] = fold_parts<E>(row + e0 + j, NPF);
    const bool valid[1] = {t < T};
    if (valid[0]) {
#pragma unroll
      for (int j = 0; j < V; ++j) logits[t * E + e0 + j] = l[0][j];
    }
    const float* const rows[1] = {row};
    int my_id[1];
    float wv[1];
    score_tokens<E, V, KK, SC, 1>(l, bl, rows, NPF, valid, gl, k_rt, renorm, n_group, topk_group,
                                  route_scale, norm_min, my_id, wv);
    if (valid[0] && gl < k) {
      ids[t * k + gl] = my_id[0];
      wout[t * k + gl] = wv[0];
      if (hists) atomicAdd(&hist[my_id[0]], 1);
    }
  }
  if (hists) {
    __syncthreads();
    if (threadIdx.x < E) {
      const int c = hist[threadIdx.x];
      if (counts && c) atomicAdd(counts + threadIdx.x, c);
      if (subcnt) subcnt[(long long)threadIdx.x * nsub + blockIdx.x] = c;
    }
  }
}

__global__ void rs_zero_kernel(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// H a multiple of 256 (four parts of whole 64-wide K steps); E = 8 or 16 with
// bf16 weights, E = 8 with fp32 weights (split hi/lo in the kernel: 16 weight
// fragment columns).
bool route_small_supported(int E, int H, bool wf32) {
  return (wf32 ? E == 8 : (E == 8 || E == 16)) && H > 0 && H % (rs::NG * rs::BK) == 0;
}

int route_small_tokens() { return rs::TB; }

template <int E, int V, int KK, int SC, int HL>
static hipError_t launch_rs(const __bf16* x, const void* w, const float* bias, int T, int H,
                            int k, int renorm, int n_group, int topk_group, float route_scale,
                            float norm_min, float* logits, int32_t* ids, float* wout,
                            int32_t* counts, int32_t* subcnt, hipStream_t s) {
  const int nsub = (T + rs::TB - 1) / rs::TB;
  hipLaunchKernelGGL((route_small_kernel<E, V, KK, SC, rs::NG, rs::NS, HL>), dim3((unsigned)nsub),
                     dim3(64 * rs::NG), 0, s, x, w, bias, T, H, k, renorm, n_group, topk_group,
                     route_scale, norm_min, logits, ids, wout, counts, subcnt, nsub);
  return hipGetLastError();
}

template <int E, int V, int HL>
static hipError_t launch_rs_cfg(const __bf16* x, const void* w, const float* bias, int T, int H,
                                int k, int scoring, int renorm, int n_group, int topk_group,
                                float route_scale, float norm_min, float* logits, int32_t* ids,
                                float* wout, int32_t* counts, int32_t* subcnt, hipStream_t s) {
#define MOE_RS_ARGS x, w, bias, T, H, k, renorm, n_group, topk_group, route_scale, norm_min, \
                    logits, ids, wout, counts, subcnt, s
#define MOE_RS_K(SC)                                           \
  return k == 2 ? launch_rs<E, V, 2, SC, HL>(MOE_RS_ARGS)      \
                : launch_rs<E, V, 0, SC, HL>(MOE_RS_ARGS);
  if (scoring == kScoreSoftmax) MOE_RS_K(kScoreSoftmax)
  if (scoring == kScoreSigmoidGroup) MOE_RS_K(kScoreSigmoidGroup)
  MOE_RS_K(kScoreSoftmaxBias)
#undef MOE_RS_K
#undef MOE_RS_ARGS
}

hipError_t launch_route_small(const __bf16* x, const void* w, bool wf32, const float* bias,
                              int T, int E, int H, int k, int scoring, int renorm, int n_group,
                              int topk_group, float route_scale, float norm_min, float* logits,
                              int32_t* ids, float* wout, int32_t* counts, int32_t* subcnt,
                              hipStream_t s) {
  if (counts) {
    hipLaunchKernelGGL(rs_zero_kernel, dim3(1), dim3(64), 0, s, counts, E);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (T == 0) return hipSuccess;
  // lanes of min(2, E/8) experts: a sigmoid group holds at least two
  const int V = topk_lane_width(E, scoring, n_group);
  if (wf32) {
    if (E == 8 && V == 1)
      return launch_rs_cfg<8, 1, 2>(x, w, bias, T, H, k, scoring, renorm, n_group, topk_group,
                                    route_scale, norm_min, logits, ids, wout, counts, subcnt, s);
    return hipErrorInvalidValue;
  }
  if (E == 8 && V == 1)
    return launch_rs_cfg<8, 1, 1>(x, w, bias, T, H, k, scoring, renorm, n_group, topk_group,
                               route_scale, norm_min, logits, ids, wout, counts, subcnt, s);
  if (E == 16 && V == 2)
    return launch_rs_cfg<16, 2, 1>(x, w, bias, T, H, k, scoring, renorm, n_group, topk_group,
                                route_scale, norm_min, logits, ids, wout, counts, subcnt, s);
  return hipErrorInvalidValue;
}

}  // namespace moe
