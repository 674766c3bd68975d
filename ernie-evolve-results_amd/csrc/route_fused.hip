// Stages 1+2 in one kernel at E = 256: router GEMM + scoring + top-k +
// histogram, with the logits tile kept on chip.
//
// Replaces the reference's cublasGemmEx (K:4327-4339) followed by
// topk_kernel (K:1829-1920), which writes the [T,E] fp32 logits to HBM and
// reads them back.  Here a workgroup owns 128 tokens x all 256 experts:
//
//   weights     a small pre-pass copies w[256, H] into a fragment-major
//               layout, so every MFMA B fragment a wave loads is 1 KB
//               contiguous (the row-major rows are 14 KB apart and land on
//               few L2 channels: the weight stream ran at ~2/3 of the speed).
//   main loop   x[128, 64-wide K step] is brought into an LDS ring by the
//               gfx950 global_load_lds DMA, D = 4 steps ahead.  Each of the
//               8 waves (two per SIMD: one wave alone cannot issue MFMAs at
//               the matrix core's rate) owns 32 experts, so its weight slice
//               is private and goes straight to registers, also D steps
//               ahead.  v_mfma_f32_16x16x32_bf16, fp32 accumulate, K in the
//               same order as the standalone GEMM (identical logits).  x and
//               w loads share the in-order vmcnt counter: waiting for a
//               step's weights retires its x stage too, and a wave never has
//               more than 63 loads in flight (the counter's limit).
//   epilogue    the 128 x 256 fp32 tile goes through LDS once; its rows are
//               copied out to router_logits (1 KB per wavefront store,
//               non-temporal), then 8 lanes per token (16 at E = 128) score
//               it with the scoring kernel's per-token routine (bit-identical
//               selection) and write the ids and weights and the block's
//               expert histogram -- optionally one per 256 (token,
//               slot) pairs, the permute's block histograms, so the permute
//               needs no histogram pass.
#include "moe_common.h"
#include "score_token.h"

namespace moe {

namespace rf {
constexpr int BK = 64, ROWB = BK * 2, CH = 8;
__device__ __forceinline__ int swz(int r) { return (r >> 1) & (CH - 1); }
// BM tokens x E experts per workgroup: the x ring stage (BM rows of one 64-wide
// K step) and the epilogue's fp32 tile (row stride E + 4 floats)
constexpr int stage_bytes(int BM) { return BM * ROWB; }
constexpr int tile_ld(int E) { return E + 4; }
constexpr int tile_bytes(int BM, int E) { return BM * tile_ld(E) * 4; }
}  // namespace rf

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt
// bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima).
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// N (8 or 4) 16-byte LDS reads 2 KB apart, issued as one instruction group
// the compiler does not track (early-clobber outputs: no output may share the
// address register); the caller places the lgkmcnt wait (an asm that takes
// the registers as "+v" operands, so nothing reads them before it).
template <int N>
__device__ __forceinline__ void lds_readn(bf16x8 (&d)[N], unsigned ad) {
  static_assert(N == 8 || N == 4, "fragment count");
  if constexpr (N == 8)
    asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:2048\n\t"
        "ds_read_b128 %2, %8 offset:4096\n\tds_read_b128 %3, %8 offset:6144\n\t"
        "ds_read_b128 %4, %8 offset:8192\n\tds_read_b128 %5, %8 offset:10240\n\t"
        "ds_read_b128 %6, %8 offset:12288\n\tds_read_b128 %7, %8 offset:14336"
        : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3]), "=&v"(d[4]), "=&v"(d[5]),
          "=&v"(d[6]), "=&v"(d[7])
        : "v"(ad)
        : "memory");
  else
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:2048\n\t"
        "ds_read_b128 %2, %4 offset:4096\n\tds_read_b128 %3, %4 offset:6144"
        : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3])
        : "v"(ad)
        : "memory");
}

// wait for every outstanding LDS read; the N registers pass through the asm
template <int N>
__device__ __forceinline__ void lds_wait(bf16x8 (&d)[N]) {
  if constexpr (N == 8)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]),
                   "+v"(d[6]), "+v"(d[7])::"memory");
  else
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3])::"memory");
}

// Bytes of LDS the kernel needs: the x ring or the epilogue tile.
constexpr int route_fused_lds(int BM, int E, int D) {
  return (D + 1) * rf::stage_bytes(BM) > rf::tile_bytes(BM, E) ? (D + 1) * rf::stage_bytes(BM)
                                                                 : rf::tile_bytes(BM, E);
}

// BM tokens (128 or 64) x E experts (256 or 128) per workgroup.  NWV waves
// (64 * NWV threads, NWV / 4 per SIMD): wave w owns experts [w*WE, (w+1)*WE)
// of all BM rows, so its weight slice is its own and goes straight to
// registers; x is shared through the LDS ring.  D: K steps of loads in
// flight.  KTC: the K steps, fully unrolled.  V, KK, SC: the scoring lane
// width, k (0: runtime) and rule.  NTOK: tokens one lane group scores per pass.
// nt_from: the first tile whose x loads are non-temporal (rf_temporal_tiles).
template <int BM, int E, int NWV, int D, int KTC, int V, int KK, int SC, int NTOK>
__global__ __launch_bounds__(64 * NWV, 1) void route_fused_kernel(
    const __bf16* __restrict__ x, const __bf16* __restrict__ wf, const float* __restrict__ bias,
    int T, int H, int k_rt, int renorm, int n_group, int topk_group, float route_scale,
    float norm_min, float* __restrict__ logits, int* __restrict__ ids, float* __restrict__ wout,
    int* __restrict__ counts, int* __restrict__ blockcnt, int nblk, int pt_log2,
    int nt_from) {
  using namespace rf;
  constexpr int NT = 64 * NWV;             // threads
  constexpr int FM = BM / 16;              // 16-row fragments per K half
  constexpr int STAGE_B = stage_bytes(BM);
  constexpr int TILE_LD = tile_ld(E);
  constexpr int WE = E / NWV;              // experts per wave
  constexpr int NJ = WE / 16;              // 16-expert fragment columns per wave
  constexpr int NX = (BM / 8) / NWV;       // x DMA instructions per wave per stage
  constexpr int NWF = 2 * NJ;              // weight fragments per wave per step (two K halves)
  constexpr int NS = D + 1;                // x ring stages
  // every wave keeps at most 63 vector loads in flight (the vmcnt limit: the
  // counter does not account for more)
  static_assert(D * (NX + NWF) <= 63, "too many loads in flight per wave");
  static_assert(NX >= 1 && NJ >= 1, "tile shape");
  __shared__ __attribute__((aligned(1024))) char lds[route_fused_lds(BM, E, D)];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wg = wave;                     // expert group
  const long long m0 = (long long)blockIdx.x * BM;
  const int KT = KTC > 0 ? KTC : H / BK;
  const int fr = lane & 15, fc = lane >> 4;

  // x DMA sources (rows past T clamped: loaded, never stored)
  const __bf16* xsrc[NX];
#pragma unroll
  for (int q = 0; q < NX; ++q) {
    const int gi = wave * NX + q;
    const int r = gi * 8 + lane / 8, p = lane % 8;
    long long row = m0 + r;
    if (row >= T) row = T - 1;
    xsrc[q] = x + row * H + (p ^ swz(r)) * 8;
  }

  // x step `src_kt` into the ring slot of step `kt`
  auto issue_x = [&](int kt, int src_kt) {
    char* st = lds + (kt % NS) * STAGE_B;
#pragma unroll
    for (int q = 0; q < NX; ++q) {
      auto* dst = (__attribute__((address_space(3))) void*)(st + (wave * NX + q) * 1024);
      // tiles from nt_from on: non-temporal (aux bit 1: nt), so they do not
      // displace the rows of the earlier tiles from the memory-side cache
      const int sk = src_kt;
      if ((int)blockIdx.x >= nt_from)
        __builtin_amdgcn_global_load_lds((const void*)(xsrc[q] + sk * BK), dst, 16, 0, 2);
      else
        __builtin_amdgcn_global_load_lds((const void*)(xsrc[q] + sk * BK), dst, 16, 0, 0);
    }
  };
  bf16x8 wr[D][NWF];
  auto issue_w = [&](int kt, bf16x8 (&dst)[NWF]) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        dst[kk * NJ + j] = *reinterpret_cast<const bf16x8*>(
            wf + ((long long)((kt * 2 + kk) * (E / 16) + wg * NJ + j) * 64 + lane) * 8);
  };
  constexpr int VMW = (D - 1) * (NX + NWF);

  f32x4 acc[FM][NJ];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // prologue: steps 0 .. D-1 in flight (KT % D == 0 is required by the launcher)
#pragma unroll
  for (int u = 0; u < D; ++u) {
    issue_x(u, u);
    issue_w(u, wr[u]);
  }

  // Every step waits, computes and refills the same way: the last D steps
  // reload step KT-1 into slots nobody reads again, so the compiler sees one
  // uniform sequence and the vmcnt count below holds on every step.
  bf16x8 a0[FM], a1[FM];
#pragma unroll
  for (int kb = 0; kb < KT; kb += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int kt = kb + u;
      // stage kt and weights kt are the oldest loads once at most (D-1)
      // later steps' loads are pending.  The wait is the builtin, not asm,
      // so the compiler's own vmcnt bookkeeping knows they are retired.
      __builtin_amdgcn_s_waitcnt(vmcnt_only(VMW));
      __builtin_amdgcn_s_barrier();
      const char* sb = lds + (kt % NS) * STAGE_B;
      // refill x first: stage kt + D goes to the slot of stage kt - 1, which
      // every wave finished reading before this step's barrier, so its DMA can
      // start before this step's fragment reads and MFMAs
      const int kn = kt + D < KT ? kt + D : KT - 1;
      issue_x(kt + D, kn);
      // rows i*16 + fr share the swizzle of fr: a half step's FM fragment
      // reads are 2 KB apart
      auto frag_addr = [&](int kk) {
        return (unsigned)(uintptr_t)((__attribute__((address_space(3))) const char*)(
            sb + fr * ROWB + (((kk * 4 + fc) ^ swz(fr)) * 16)));
      };
      lds_readn<FM>(a0, frag_addr(0));
      lds_wait<FM>(a0);
      // the second half's reads go out before the first half's MFMAs and
      // land while they run
      lds_readn<FM>(a1, frag_addr(1));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[i], wr[u][j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      lds_wait<FM>(a1);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[i], wr[u][NJ + j], acc[i][j], 0, 0, 0);
      // refill the weights of step kt + D once this step's MFMAs have read them
      issue_w(kn, wr[u]);
    }
  }

  // ---- epilogue: the fp32 tile through LDS
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  float* tile = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = wg * WE + j * 16 + fr;
#pragma unroll
      for (int r = 0; r < 4; ++r) tile[(i * 16 + fc * 4 + r) * TILE_LD + col] = acc[i][j][r];
    }
  __syncthreads();

  // ---- logits: the tile's rows copied out whole, one 16-byte vector per lane
  // (a wavefront writes 1 KB of consecutive floats), non-temporal so they do
  // not take memory-side cache space from x; issued before the scoring, which
  // runs while they drain
  for (int idx = threadIdx.x; idx < BM * (E / 4); idx += NT) {
    const int row = idx / (E / 4), c4 = idx - row * (E / 4);
    if (m0 + row < T)
      __builtin_nontemporal_store(*reinterpret_cast<const f32x4*>(tile + row * TILE_LD + c4 * 4),
                                  reinterpret_cast<f32x4*>(logits + (m0 + row) * E + c4 * 4));
  }

  // ---- scoring: G = E/V lanes per token
  constexpr int G = E / V;
  constexpr int TPP = NT / G;  // tokens per pass
  // expert histograms of the tile's sub-blocks of 2^pt_log2 tokens (with
  // blockcnt: the permute's blocks of 256 pairs, 256 / k tokens each; without:
  // pt_log2 >= log2(BM), one histogram for the whole tile)
  constexpr int MAXSB = BM / 32;
  __shared__ int hist[MAXSB * E];
  const bool hists = counts || blockcnt;
  if (hists) {
    for (int i = threadIdx.x; i < MAXSB * E; i += NT) hist[i] = 0;
    __syncthreads();
  }
  const int gl = threadIdx.x % G;
  const int e0 = gl * V;
  float bl[V];
#pragma unroll
  for (int j = 0; j < V; ++j) bl[j] = bias ? bias[e0 + j] : 0.0f;
  const int k = KK > 0 ? KK : k_rt;
  // each G-lane group scores NTOK tokens per pass (tl, tl + TPP, ...); two or
  // four interleaved tokens measured no faster than one (175-180 us per call)
  static_assert(BM % (TPP * NTOK) == 0, "token passes");
  for (int tl0 = threadIdx.x / G; tl0 < BM; tl0 += TPP * NTOK) {
    float l[NTOK][V];
    const float* rows[NTOK];
    bool valid[NTOK];
#pragma unroll
    for (int n = 0; n < NTOK; ++n) {
      const int tl = tl0 + n * TPP;
      const long long t = m0 + tl;
      rows[n] = tile + tl * TILE_LD;
#pragma unroll
      for (int j = 0; j < V; j += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(rows[n] + e0 + j);
        l[n][j] = v[0]; l[n][j + 1] = v[1]; l[n][j + 2] = v[2]; l[n][j + 3] = v[3];
      }
      valid[n] = t < T;
    }
    int my_id[NTOK];
    float wv[NTOK];
    score_tokens<E, V, KK, SC, NTOK>(l, bl, rows, 1, valid, gl, k_rt, renorm, n_group,
                                     topk_group, route_scale, norm_min, my_id, wv);
#pragma unroll
    for (int n = 0; n < NTOK; ++n) {
      const long long t = m0 + tl0 + n * TPP;
      if (valid[n] && gl < k) {
        ids[t * k + gl] = my_id[n];
        wout[t * k + gl] = wv[n];
        if (hists) atomicAdd(&hist[((tl0 + n * TPP) >> pt_log2) * E + my_id[n]], 1);
      }
    }
  }
  if (hists) {
    __syncthreads();
    const int nsb = pt_log2 >= 31 ? 1 : (BM >> pt_log2 > 0 ? BM >> pt_log2 : 1);
    if (counts) {
      for (int i = threadIdx.x; i < E; i += NT) {
        int c = 0;
        for (int b = 0; b < nsb; ++b) c += hist[b * E + i];
        if (c) atomicAdd(counts + i, c);
      }
    }
    if (blockcnt) {
      // [E, nblk] layout: the tile's nsb consecutive blocks of one expert are
      // adjacent; blocks past the last pair are not written
      const int b0 = (int)(m0 >> pt_log2);
      for (int i = threadIdx.x; i < nsb * E; i += NT) {
        const int e = i / nsb, b = i - e * nsb;
        if (b0 + b < nblk) blockcnt[(long long)e * nblk + b0 + b] = hist[b * E + e];
      }
    }
  }
}

// Router weight [E, H] bf16 -> fragment-major copy: with NG = E / 16 expert
// groups, fragment f = (kt*2 + kk)*NG + g holds, for lane l, the 8 values
// w[g*16 + (l & 15)][kt*64 + kk*32 + (l >> 4)*8 ..], so each MFMA B fragment
// the GEMM loads is 1 KB contiguous.
__global__ __launch_bounds__(256) void rf_wfrag_kernel(const u32x4* __restrict__ w, int H, int ng,
                                                        u32x4* __restrict__ wf, int n) {
  const int v = blockIdx.x * 256 + threadIdx.x;
  if (v >= n) return;
  const int l = v & 63, f = v >> 6;
  const int g = f % ng, kk = (f / ng) & 1, kt = f / (2 * ng);
  const int e = g * 16 + (l & 15);
  const int k = kt * 64 + kk * 32 + (l >> 4) * 8;
  wf[v] = w[((long long)e * H + k) / 8];
}

__global__ void rf_zero_kernel(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// The configurations shipped: 8 waves (two per SIMD; one wave per SIMD issues
// MFMAs at about a third of the rate), loads D = 4 steps ahead, one token per
// lane group per scoring pass, the K loop fully unrolled (a runtime trip count
// makes the compiler merge its load bookkeeping at the loop head into a
// vmcnt(0) that drains every load in flight once per iteration):
//   E = 256, H = 7168 (DeepSeek-V3): 128-token tiles, 112 K steps;
//   E = 128, H = 2048 (Qwen3-MoE):   64-token tiles (256 of them at T = 16384),
//                                    32 K steps.
constexpr int kRfWaves = 8, kRfDepth = 4, kRfScoreTokens = 1;

// Experts per scoring lane: 32 at E = 256 (8 lanes per token; a DeepSeek-V3
// group of 32 is one lane, so its top-2 needs no lane exchange: 4-6 us less
// per call than 16), 16 at E = 128 (a 64-token tile has no room for fewer
// lanes per token).  A group-limited rule needs whole groups per lane.
constexpr int rf_lane_width(int E) { return E == 256 ? 32 : 16; }

bool route_fused_supported(int E, int H, int scoring, int n_group) {
  const bool shape = (E == 256 && H == 112 * rf::BK) || (E == 128 && H == 32 * rf::BK);
  if (!shape) return false;
  if (scoring == kScoreSigmoidGroup && n_group > 1)
    return n_group <= E && E % n_group == 0 && (E / n_group) % rf_lane_width(E) == 0;
  return true;
}

// Token tile of the shipped configuration of this shape.
static int rf_tile_tokens(int E) { return E == 256 ? 128 : 64; }

bool route_fused_block_hist_supported(int E, int k) {
  // blocks of kPairsPerBlock pairs hold whole tokens, and a tile whole blocks
  return k >= 1 && k <= 8 && kPairsPerBlock % k == 0 &&
         rf_tile_tokens(E) % (kPairsPerBlock / k) == 0;
}

size_t route_fused_workspace_bytes(int E, int H) { return (size_t)E * H * 2; }

// Memory-side cache (MALL, 256 MiB on MI355X) policy for the x stream.  The
// permute's gather reads x again right after this kernel, token by token.
// With every x load temporal, the MALL ends up holding the last-read K columns
// of every token, and the gather's own misses evict them before it gets there.
// Instead, the tiles of the first kRfMallBytes of x (in token order) load
// temporal and the rest non-temporal, so the MALL keeps whole rows of the
// tokens the gather reads first; the logits go out non-temporal, so they take
// none of it.  Measured at the DeepSeek-V3 shape (C4 step, 5 runs of 20 steps
// each, 128-token tiles): all temporal 1.700 ms, all non-temporal 1.709; with
// the logits stored temporal from registers, the first 100 / 109 / 120 tiles
// temporal 1.681 / 1.678 / 1.685; with the non-temporal row copy of the
// logits, 109 / 120 / 130 / 140 / 150 / 160 tiles 1.675 / 1.675 / 1.669 /
// 1.672 / 1.685 / 1.695.
constexpr long long kRfMallBytes = 228ll << 20;
static int rf_temporal_tiles(int BM, int H) {
  const long long t = kRfMallBytes / ((long long)BM * H * 2);
  return t > (1 << 30) ? (1 << 30) : (int)t;
}

template <int BM, int E, int KTC, int V, int KK, int SC>
static hipError_t launch_rf(const __bf16* x, const __bf16* wf, const float* bias, int T, int H,
                            int k, int renorm, int n_group, int topk_group, float route_scale,
                            float norm_min, float* logits, int32_t* ids, float* wout,
                            int32_t* counts, int32_t* blockcnt, hipStream_t s) {
  auto kern = route_fused_kernel<BM, E, kRfWaves, kRfDepth, KTC, V, KK, SC, kRfScoreTokens>;
  // blocks of 256 pairs = 2^pt_log2 tokens (k a power of two), else one
  // histogram per tile
  int pt_log2 = 31;
  if (blockcnt) {
    pt_log2 = 0;
    while ((k << pt_log2) < kPairsPerBlock) ++pt_log2;
  }
  const int nblk = dispatch_blocks((long long)T * k);
  hipLaunchKernelGGL(kern, dim3((unsigned)((T + BM - 1) / BM)), dim3(64 * kRfWaves), 0, s, x, wf,
                     bias, T, H, k, renorm, n_group, topk_group, route_scale, norm_min, logits,
                     ids, wout, counts, blockcnt, nblk, pt_log2, rf_temporal_tiles(BM, H));
  return hipGetLastError();
}

template <int BM, int E, int KTC>
static hipError_t launch_rf_cfg(const __bf16* x, const __bf16* wf, const float* bias, int T,
                                int H, int k, int scoring, int renorm, int n_group, int topk_group,
                                float route_scale, float norm_min, float* logits, int32_t* ids,
                                float* wout, int32_t* counts, int32_t* blockcnt, hipStream_t s) {
#define MOE_RF_ARGS x, wf, bias, T, H, k, renorm, n_group, topk_group, route_scale, norm_min, \
                    logits, ids, wout, counts, blockcnt, s
#define MOE_RF_SC(SCV)                                                  \
  {                                                                     \
    if (k == 8) return launch_rf<BM, E, KTC, rf_lane_width(E), 8, SCV>(MOE_RF_ARGS);  \
    return launch_rf<BM, E, KTC, rf_lane_width(E), 0, SCV>(MOE_RF_ARGS);              \
  }
  if (scoring == kScoreSoftmax) MOE_RF_SC(kScoreSoftmax)
  if (scoring == kScoreSigmoidGroup) MOE_RF_SC(kScoreSigmoidGroup)
  MOE_RF_SC(kScoreSoftmaxBias)
#undef MOE_RF_SC
#undef MOE_RF_ARGS
}

// x [T, H] bf16, w [E, H] bf16; ws: route_fused_workspace_bytes(E, H) bytes
// (the fragment-major weight copy).  Caller checked route_fused_supported.
// blockcnt (or NULL): the permute's raw block histograms [E, ceil(T*k/256)],
// every entry written; needs route_fused_block_hist_supported(E, k).
hipError_t launch_route_fused(const __bf16* x, const __bf16* w, const float* bias, int T, int E,
                              int H, int k, int scoring, int renorm, int n_group, int topk_group,
                              float route_scale, float norm_min, float* logits, int32_t* ids,
                              float* wout, int32_t* counts, int32_t* blockcnt, void* ws,
                              hipStream_t s) {
  if (counts) {
    hipLaunchKernelGGL(rf_zero_kernel, dim3((E + 255) / 256), dim3(256), 0, s, counts, E);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (T == 0) return hipSuccess;
  __bf16* wf = (__bf16*)ws;
  {
    const int n = E * H / 8;
    hipLaunchKernelGGL(rf_wfrag_kernel, dim3((n + 255) / 256), dim3(256), 0, s, (const u32x4*)w,
                       H, E / 16, (u32x4*)wf, n);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (E == 256)
    return launch_rf_cfg<128, 256, 112>(x, wf, bias, T, H, k, scoring, renorm, n_group,
                                        topk_group, route_scale, norm_min, logits, ids, wout,
                                        counts, blockcnt, s);
  return launch_rf_cfg<64, 128, 32>(x, wf, bias, T, H, k, scoring, renorm, n_group, topk_group,
                                    route_scale, norm_min, logits, ids, wout, counts, blockcnt,
                                    s);
}

}  // namespace moe
