// Stages 1+2 in one kernel at E = 256 and E = 128: router GEMM + scoring +
// top-k + histogram, with the logits tile kept on chip.
//
// Replaces the reference's cublasGemmEx (K:4327-4339) followed by
// topk_kernel (K:1829-1920), which writes the [T,E] fp32 logits to HBM and
// reads them back.  Here a workgroup owns BM tokens x all E experts (128 x 256
// at the DeepSeek-V3 shape, 64 x 128 at Qwen3-MoE's):
//
//   weights     a small pre-pass copies w[E, H] into a fragment-major
//               layout, so every MFMA B fragment a wave loads is 1 KB
//               contiguous (read row-major, the 14 KB-strided rows of one K
//               step land on few L2 channels).
//   main loop   x comes into an LDS ring by the gfx950 buffer_load ... lds
//               DMA, one stage = two 64-wide K steps (256 contiguous bytes of
//               every row), NSTG - 1 stages ahead.  Each of the 8 waves (two
//               per SIMD) owns E/8 experts, so its weight slice is private and
//               goes straight to registers, DW steps ahead.
//               v_mfma_f32_16x16x32_bf16, fp32 accumulate, K in order (the
//               logits equal the standalone GEMM's bit for bit).  x and w
//               loads share the vmcnt counter; each step's one wait
//               (rf::Sched) counts only loads issued after the ones it must
//               retire that are of the same kind, so it holds whatever order
//               the x DMA and the weight loads complete in relative to each
//               other.  Rows past T read as zeros (buffer bounds).
//   epilogue    the BM x E fp32 tile goes through LDS once; its rows are
//               copied out to router_logits (1 KB per wavefront store,
//               non-temporal), then 8 lanes per token (32 experts each at
//               E = 256, 16 at E = 128) score it with the scoring kernel's
//               per-token routine (bit-identical selection; at E = 256 two
//               tokens per 8 lanes, whose kept expert groups the selection
//               rounds compact into the 8 lanes) and write the ids and
//               weights and the block's expert histogram -- optionally one
//               per 256 (token, slot) pairs, the permute's block histograms,
//               so the permute needs no histogram pass.
#include <utility>

#include "moe_common.h"
#include "score_token.h"

namespace moe {

namespace rf {
constexpr int BK = 64;
// word 3 of a gfx9 raw buffer resource (32-bit data format, no swizzle)
constexpr int kRsrcW3 = 0x00020000;

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt
// bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima).
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// One wave's vector-memory loads in program order.  Prologue: x stages
// 0 .. DX-1 (NX DMA loads each), then the weights of steps 0 .. DW-1 (NW each).
// Step p: [at a stage start: wait, barrier, x stage p/SPS + DX] wait for the
// step's weights; MFMAs; weights of step p + DW.  wait_at(p) is the vmcnt that
// retires the loads step p needs (its weights and, at a stage start, its x
// stage) assuming only that loads of one kind complete in issue order: the x
// DMA loads (into LDS) and the weight loads (into registers) are not assumed
// to complete in order with respect to each other.  With W(p) outstanding, the
// (DW-1)*NW weight loads issued after it are outstanding too, so a count of at
// most (DW-1)*NW retires W(p); likewise (DX-1)*NX for x stage p/SPS.  (A count
// that relied on the two kinds completing in one order read stale LDS rows on
// the first, cold call of a configuration whose x ran only as far ahead as its
// weights.)
struct Sched {
  int SPS, DX, DW, NX, NW;
  constexpr int wait_at(int p) const {
    const int w = (DW - 1) * NW, xs = (DX - 1) * NX;
    return (p % SPS == 0 && xs < w) ? xs : w;
  }
};

// The kernel's shape: BM tokens x E experts, H = 64 * KT, 8 waves.
template <int BM, int E, int KT>
struct Cfg {
  static constexpr int NWV = 8, NT = 64 * NWV;
  static constexpr int SPS = 2;                     // K steps per x stage
  static constexpr int NSTG = E == 256 ? 4 : 3;     // x ring stages
  static constexpr int DW = E == 256 ? 5 : 4;       // weight steps in flight
  static constexpr int ROWB = SPS * BK * 2;         // LDS row pitch of a stage
  static constexpr int STAGE_B = BM * ROWB;
  static constexpr int DX = NSTG - 1, NST = KT / SPS;
  static constexpr int WE = E / NWV, NJ = WE / 16, NW = 2 * NJ, FM = BM / 16;
  static constexpr int NX = STAGE_B / 1024 / NWV;   // 1 KB DMA instructions per wave per stage
  static constexpr int TILE_LD = E + 4;             // epilogue tile row stride (floats)
  static constexpr int LDSB = NSTG * STAGE_B > BM * TILE_LD * 4 ? NSTG * STAGE_B : BM * TILE_LD * 4;
  static constexpr Sched S{SPS, DX, DW, NX, NW};
  static_assert(KT % SPS == 0 && NX >= 1 && NJ >= 1 && (FM == 8 || FM == 4), "tile shape");
  static_assert(DX * NX + DW * NW <= 63, "vmcnt range");
};

// 16-byte chunk c of stage row r -> its LDS slot: the 16 rows of one fragment
// read land in 16 distinct 16-byte bank groups.
__device__ __forceinline__ int xslot(int r, int c) { return c ^ (r & 15); }
}  // namespace rf

// N (8 or 4) 16-byte LDS reads 16 rows apart (row pitch RB bytes), issued as
// one instruction group the compiler does not track (early-clobber outputs:
// no output may share the address register); lds_wait places the wait.
template <int N, int RB>
__device__ __forceinline__ void lds_readn(bf16x8 (&d)[N], unsigned ad) {
  static_assert(N == 8 || N == 4, "fragment count");
  if constexpr (N == 8)
    asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:%9\n\t"
        "ds_read_b128 %2, %8 offset:%10\n\tds_read_b128 %3, %8 offset:%11\n\t"
        "ds_read_b128 %4, %8 offset:%12\n\tds_read_b128 %5, %8 offset:%13\n\t"
        "ds_read_b128 %6, %8 offset:%14\n\tds_read_b128 %7, %8 offset:%15"
        : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3]), "=&v"(d[4]), "=&v"(d[5]),
          "=&v"(d[6]), "=&v"(d[7])
        : "v"(ad), "n"(16 * RB), "n"(32 * RB), "n"(48 * RB), "n"(64 * RB), "n"(80 * RB),
          "n"(96 * RB), "n"(112 * RB)
        : "memory");
  else
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:%5\n\t"
        "ds_read_b128 %2, %4 offset:%6\n\tds_read_b128 %3, %4 offset:%7"
        : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3])
        : "v"(ad), "n"(16 * RB), "n"(32 * RB), "n"(48 * RB)
        : "memory");
}

// wait for the LDS reads: all but the last CNT issued; the N registers pass
// through the asm, so nothing reads them before it
template <int CNT, int N>
__device__ __forceinline__ void lds_wait(bf16x8 (&d)[N]) {
  if constexpr (N == 8)
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]),
                   "+v"(d[6]), "+v"(d[7])
                 : "n"(CNT)
                 : "memory");
  else
    asm volatile("s_waitcnt lgkmcnt(%4)"
                 : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3])
                 : "n"(CNT)
                 : "memory");
}

// x DMA of one 16-byte piece per lane into LDS (buffer_load_dwordx4 ... lds);
// NT: non-temporal (aux bit 1), so the line is not kept in the memory-side cache
template <bool NT>
__device__ __forceinline__ void rf_dma16(__amdgpu_buffer_rsrc_t r, char* l, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)l, 16,
                                           voff, soff, 0, NT ? 2 : 0);
}

// The K loop of one BM-token tile: acc[i][j] = the wave's 16 x 16 blocks
// (rows i*16.., experts wave*WE + j*16..), fp32.  NTX: x loads non-temporal.
// The whole loop is unrolled (one instantiation per step), so every ring slot,
// register slot and wait count is a constant.
template <int BM, int E, int KT, bool NTX>
__device__ __forceinline__ void rf_kloop(const __bf16* __restrict__ x,
                                         const __bf16* __restrict__ wf, int T, char* lds,
                                         f32x4 (&acc)[BM / 16][E / 128]) {
  using C = rf::Cfg<BM, E, KT>;
  using namespace rf;
  constexpr int H = KT * BK, ROWB = C::ROWB, STAGE_B = C::STAGE_B, NSTG = C::NSTG;
  constexpr int NJ = C::NJ, NW = C::NW, DX = C::DX, DW = C::DW, NX = C::NX, FM = C::FM;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const long long m0 = (long long)blockIdx.x * BM;
  const int fr = lane & 15, fc = lane >> 4;
  const int rows = T - m0 < BM ? (int)(T - m0) : BM;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(x + m0 * H), (short)0, rows * H * 2, kRsrcW3);
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)wf, (short)0, E * H * 2, kRsrcW3);

  // x DMA: instruction q of this wave covers stage rows (wave*NX + q)*RPI ..;
  // lane l writes the 16 bytes at LDS offset l*16 of the instruction's 1 KB
  constexpr int RPI = 1024 / ROWB, CPR = ROWB / 16;
  int voff_x[NX];
#pragma unroll
  for (int q = 0; q < NX; ++q) {
    const int r = (wave * NX + q) * RPI + lane / CPR, p = lane % CPR;
    voff_x[q] = r * H * 2 + xslot(r, p) * 16;
  }
  auto issue_x = [&](int st) {
    const int ls = st < C::NST ? st : C::NST - 1;  // past the end: reload the last stage
#pragma unroll
    for (int q = 0; q < NX; ++q)
      rf_dma16<NTX>(rx, lds + (st % NSTG) * STAGE_B + (wave * NX + q) * 1024, voff_x[q],
                    ls * ROWB);
  };
  // weights: fragment (kt*2 + kk)*(E/16) + wave*NJ + j, 1 KB each
  const int voff_w = (wave * NJ * 64 + lane) * 16;
  bf16x8 wr[DW][NW];
  auto issue_w = [&](int p, bf16x8 (&dst)[NW]) {
    if (p >= KT) p = KT - 1;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        dst[kk * NJ + j] = __builtin_bit_cast(
            bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rw, voff_w + j * 1024,
                                                          (p * 2 + kk) * E * 64, 0));
  };

#pragma unroll
  for (int st = 0; st < DX; ++st) issue_x(st);
#pragma unroll
  for (int p = 0; p < DW; ++p) issue_w(p, wr[p]);
  const unsigned fbase =
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) const char*)lds + fr * ROWB;
  bf16x8 a[FM];
  auto step = [&]<int P>(std::integral_constant<int, P>) __attribute__((always_inline)) {
    constexpr int VM = C::S.wait_at(P);
    static_assert(VM >= 0 && VM <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt(vmcnt_only(VM));
    if constexpr (P % C::SPS == 0) {
      // every wave's part of this stage has landed and every wave is done
      // with the previous stage's slot, which the new DMA refills
      __builtin_amdgcn_s_barrier();
      issue_x(P / C::SPS + DX);
    }
    constexpr int slot = (P / C::SPS) % NSTG;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const unsigned ad =
          fbase + slot * STAGE_B + xslot(fr, (P % C::SPS) * 8 + kk * 4 + fc) * 16;
      if constexpr (FM == 8) {
        // two groups of four fragments: the first group's MFMAs start while
        // the second group's reads are in flight
        bf16x8(&lo)[4] = *reinterpret_cast<bf16x8(*)[4]>(&a[0]);
        bf16x8(&hi)[4] = *reinterpret_cast<bf16x8(*)[4]>(&a[4]);
        lds_readn<4, ROWB>(lo, ad);
        lds_readn<4, ROWB>(hi, ad + 64 * ROWB);
        lds_wait<4>(lo);
      } else {
        lds_readn<FM, ROWB>(a, ad);
        lds_wait<0>(a);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if constexpr (FM == 8) {
          if (i == 4) {
            __builtin_amdgcn_sched_barrier(0);
            lds_wait<0>(*reinterpret_cast<bf16x8(*)[4]>(&a[4]));
          }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], wr[P % DW][kk * NJ + j],
                                                              acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    issue_w(P + DW, wr[P % DW]);
  };
  [&]<int... Ps>(std::integer_sequence<int, Ps...>) __attribute__((always_inline)) {
    (step(std::integral_constant<int, Ps>{}), ...);
  }(std::make_integer_sequence<int, KT>{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// BM tokens (128 or 64) x E experts (256 or 128) per workgroup, 8 waves: wave
// w owns experts [w*E/8, (w+1)*E/8) of all BM rows.  KT: the K steps.  V, KK,
// SC: the scoring lane width, k (0: runtime) and rule.  nt_from: the first
// tile whose x loads are non-temporal (rf_temporal_tiles).
template <int BM, int E, int KT, int V, int KK, int SC>
__global__ __launch_bounds__(512, 1) void route_fused_kernel(
    const __bf16* __restrict__ x, const __bf16* __restrict__ wf, const float* __restrict__ bias,
    int T, int H, int k_rt, int renorm, int n_group, int topk_group, float route_scale,
    float norm_min, float* __restrict__ logits, int* __restrict__ ids, float* __restrict__ wout,
    int* __restrict__ counts, int* __restrict__ blockcnt, int nblk, int pt_log2,
    int nt_from) {
  using C = rf::Cfg<BM, E, KT>;
  constexpr int NT = C::NT, FM = C::FM, NJ = C::NJ, WE = C::WE, TILE_LD = C::TILE_LD;
  constexpr int NTOK = E == 256 ? 2 : 1;  // tokens a lane group scores per pass
  __shared__ __attribute__((aligned(1024))) char lds[C::LDSB];
  const int lane = threadIdx.x & 63;
  const int wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // expert group
  const long long m0 = (long long)blockIdx.x * BM;
  const int fr = lane & 15, fc = lane >> 4;

  f32x4 acc[FM][NJ];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  if ((int)blockIdx.x >= nt_from)
    rf_kloop<BM, E, KT, true>(x, wf, T, lds, acc);
  else
    rf_kloop<BM, E, KT, false>(x, wf, T, lds, acc);

  // ---- epilogue: the fp32 tile through LDS (over the ring: every wave is
  // past its last fragment read once it reaches this barrier)
  __syncthreads();
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
  {
    constexpr int NCP = BM * (E / 4) / NT;  // 16-byte pieces per thread, all read before any store
    static_assert(BM * (E / 4) % NT == 0, "logits copy");
    f32x4 piece[NCP];
#pragma unroll
    for (int i = 0; i < NCP; ++i) {
      const int idx = threadIdx.x + i * NT;
      const int row = idx / (E / 4), c4 = idx - row * (E / 4);
      piece[i] = *reinterpret_cast<const f32x4*>(tile + row * TILE_LD + c4 * 4);
    }
#pragma unroll
    for (int i = 0; i < NCP; ++i) {
      const int idx = threadIdx.x + i * NT;
      const int row = idx / (E / 4), c4 = idx - row * (E / 4);
      if (m0 + row < T)
        __builtin_nontemporal_store(piece[i], reinterpret_cast<f32x4*>(logits + (m0 + row) * E + c4 * 4));
    }
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
  if (bias) {
    load_vec<V>(bias + e0, bl);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) bl[j] = 0.0f;
  }
  const int k = KK > 0 ? KK : k_rt;
  // each G-lane group scores NTOK tokens per pass (tl, tl + TPP, ...): every
  // tile finishes its K loop at about the same time, so the scoring is not
  // hidden behind other tiles' loops, and two interleaved tokens hide the
  // latency of its cross-lane chains (C4 route stage 150 -> 145 us with
  // every x load non-temporal)
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

// The configurations shipped (rf::Cfg): 8 waves (two per SIMD; one wave per
// SIMD with 128 x 64 wave tiles ran the same K loop time and a slower
// scoring), the K loop fully unrolled, two tokens per lane group per scoring
// pass at E = 256 and one at E = 128:
//   E = 256, H = 7168 (DeepSeek-V3): 128-token tiles, 112 K steps, 4 x-ring
//                                    stages of 32 KB, weights 5 steps ahead;
//   E = 128, H = 2048 (Qwen3-MoE):   64-token tiles (256 of them at T = 16384),
//                                    32 K steps, 3 stages of 16 KB, weights 4
//                                    steps ahead (route 25.4 us after a
//                                    combine, against 26.1-28.3 us for 4-8
//                                    stages and weights 3-8 ahead).

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
// none of it.  A temporal load that finds the MALL full of dirty lines (the
// previous step's output, a cache flush) pays for their write-back: the
// temporal tiles' K loops run ~25 us longer than the non-temporal ones, and
// the gather gains ~45 us.  Measured at the DeepSeek-V3 shape (C4 step,
// builds alternated in one session, each step after a 1 GiB rewrite): 0 /
// 114 / 228 / 280 MiB temporal 1.719 / 1.700 / 1.686 / 1.706 ms.
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
  auto kern = route_fused_kernel<BM, E, KTC, V, KK, SC>;
  // blocks of 256 pairs = 2^pt_log2 tokens (k a power of two), else one
  // histogram per tile
  int pt_log2 = 31;
  if (blockcnt) {
    pt_log2 = 0;
    while ((k << pt_log2) < kPairsPerBlock) ++pt_log2;
  }
  const int nblk = dispatch_blocks((long long)T * k);
  hipLaunchKernelGGL(kern, dim3((unsigned)((T + BM - 1) / BM)), dim3(rf::Cfg<BM, E, KTC>::NT), 0, s, x, wf,
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
