// Stage 1: the router GEMM, logits[T,N] = x[T,H] . w[N,H]^T, bf16 in, fp32 out.
//
// Replaces the reference's cublasGemmEx call (K:4327-4339) with gfx950 MFMA
// kernels.  Both operands are K-contiguous (x row-major [T,H], w row-major
// [N,H]), which is exactly the operand layout of v_mfma_f32_16x16x32_bf16:
// a lane feeds 8 consecutive k of one row of A and the same 8 k of one
// column of B, so a fragment is a single 16-byte LDS read.
//
// Tiles are brought into LDS by the gfx950
// global_load_lds_dwordx4 DMA (no register staging), into an NS-stage ring
// with an XOR-swizzled 16-byte-chunk layout (conflict-free fragment reads),
// one s_barrier per K step.  At N >= 256 a 1024-thread block (16 waves of
// 64 x 32 accumulators) owns 256 rows x 128 experts with a 3-stage ring (two
// stages in flight, 144 KB of LDS): at T = 32768, E = 256 the 128 row tiles x
// 2 expert tiles fill 256 CUs without splitting K, and the two blocks of a
// row tile (neighbouring hardware ids, the same XCD) read their x rows once
// from HBM and once from L2.  The earlier 256 x 256 tile with a 2-stage ring
// needed split-K = 2 to fill the chip and waited on each K step's DMA (route
// stage 202 against 189 us in the C4 step).  When the row tiles alone leave
// the chip idle (small T), the K range is still split: the fp32 partial sums
// land side by side as [T, ksplit * N] and the scoring kernel adds them in a
// fixed order (deterministic, no atomics).
// x is loaded with ordinary (temporal) loads although the GEMM reads it once:
// the part of x still held in the 256 MB memory-side cache (MALL) when the
// permute reads x again is not fetched from HBM a second time.  Measured on
// the C4 step: the GEMM is ~30 us slower than with non-temporal x loads, the
// gather and the combine after it ~15 and ~55 us faster (1745 vs 1791 us per
// step, outputs bit-identical).
//
// Smaller N use smaller row tiles (and split-K when even those leave the
// chip idle): there the router weight is small and the GEMM is an x stream.
#include "moe_common.h"

namespace moe {

// fp32 w[E,H] -> wpk[2E,H] bf16, rows [0,E) = bf16(w), rows [E,2E) = bf16(w - bf16(w)).
// One bf16 GEMM against wpk yields hi and lo partial logits whose sum is the
// fp32-accurate logit (the reference's wsplit_kernel, K:1786-1824, which packs
// the same two halves as columns of a [H,2E] matrix).
__global__ __launch_bounds__(256) void wsplit_kernel(const float* __restrict__ w,
                                                     unsigned short* __restrict__ wpk,
                                                     long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x) {
    const float v = w[i];
    const unsigned int hi = f2bf(v);
    const float lo = v - __uint_as_float(hi << 16);
    wpk[i] = (unsigned short)hi;
    wpk[n + i] = (unsigned short)f2bf(lo);
  }
}

hipError_t launch_wsplit(const float* w, __bf16* wpk, int E, int H, hipStream_t s) {
  const long long n = (long long)E * H;
  const int grid = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(wsplit_kernel, dim3(grid), dim3(256), 0, s, w, (unsigned short*)wpk, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// LDS-DMA pipelined kernel.
//   BM x BN block tile, BK = 64 K per stage (128-byte LDS rows, 8 chunks of 16 B),
//   NS stages, WM x WN waves.  A wave instruction moves 1 KB (8 rows).  Logical
//   chunk c of tile row r lives at physical chunk c ^ ((r >> 1) & 7): the 16
//   rows of one fragment read land on 16 distinct bank groups.
// ---------------------------------------------------------------------------
template <int BM, int BN, int NS, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void router_gemm_dma_kernel(
    const __bf16* __restrict__ x, const __bf16* __restrict__ w, int T, int H, int N,
    int kchunk, float* __restrict__ out, int ldo) {
  constexpr int BK = 64, CH = 8, ROWB = 128, RPI = 8;
  constexpr int STAGE_B = (BM + BN) * ROWB;
  constexpr int A_INST = BM / RPI, B_INST = BN / RPI, NW = WM * WN;
  constexpr int PER_WAVE = (A_INST + B_INST) / NW;
  constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 16, FN = WTN / 16;
  static_assert((A_INST + B_INST) % NW == 0, "every wave issues the same number of loads");
  static_assert(FM >= 1 && FN >= 1, "wave tile below one MFMA tile");
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE_B];

  // wave index as a scalar: the x / weight role of each DMA below is a uniform branch
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const long long m0 = (long long)blockIdx.x * BM;
  const int n0 = blockIdx.y * BN;
  const int kb = blockIdx.z * kchunk;
  const int KT = kchunk / BK;
  auto swz = [](int r) { return (r >> 1) & (CH - 1); };

  // Per-lane source of each of this wave's DMA instructions (row clamped
  // into range: rows past T / N are loaded but never stored).
  const __bf16* src[PER_WAVE];
#pragma unroll
  for (int q = 0; q < PER_WAVE; ++q) {
    const int gi = wave * PER_WAVE + q;
    const int p = lane % CH;
    if (gi < A_INST) {
      const int r = gi * RPI + lane / CH;
      long long row = m0 + r;
      if (row >= T) row = T - 1;
      src[q] = x + row * H + kb + (p ^ swz(r)) * 8;
    } else {
      const int r = (gi - A_INST) * RPI + lane / CH;
      int row = n0 + r;
      if (row >= N) row = N - 1;
      src[q] = w + (long long)row * H + kb + (p ^ swz(r)) * 8;
    }
  }
  auto issue = [&](int kt, int st) {
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
      auto* dst = (__attribute__((address_space(3))) void*)(lds + st * STAGE_B +
                                                            (wave * PER_WAVE + q) * 1024);
      // x and the weight alike: temporal (x is read again by the permute)
      __builtin_amdgcn_global_load_lds((const void*)(src[q] + kt * BK), dst, 16, 0, 0);
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int st = 0; st < NS - 1; ++st)
    if (st < KT) issue(st, st);
  const int fr = lane & 15, fc = lane >> 4;
  for (int kt = 0; kt < KT; ++kt) {
    // This wave's loads of stage kt are done once at most (NS-2) later
    // stages are outstanding; the barrier then publishes every wave's
    // loads and retires the reads of the buffer reloaded next.
    if (kt + NS - 2 < KT)
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 2) * PER_WAVE) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    if (kt + NS - 1 < KT) issue(kt + NS - 1, (kt + NS - 1) % NS);
    const char* sb = lds + (kt % NS) * STAGE_B;
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      bf16x8 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * WTM + i * 16 + fr, c = kk * 4 + fc;
        a[i] = *reinterpret_cast<const bf16x8*>(sb + r * ROWB + ((c ^ swz(r)) * 16));
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int r = wn * WTN + j * 16 + fr, c = kk * 4 + fc;
        b[j] = *reinterpret_cast<const bf16x8*>(sb + BM * ROWB + r * ROWB + ((c ^ swz(r)) * 16));
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // partial z of the split-K writes columns [z*N, (z+1)*N) of a row of ldo floats
  float* o = out + (long long)blockIdx.z * N;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + wn * WTN + j * 16 + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const long long row = m0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r;
        if (row < T && col < N) o[row * ldo + col] = acc[i][j][r];
      }
    }
}

template <int BM, int BN, int NS, int WM, int WN>
static hipError_t launch_dma(const __bf16* x, const __bf16* w, int T, int H, int N, int ksplit,
                             float* out, hipStream_t s) {
  const dim3 grid((unsigned)((T + BM - 1) / BM), (unsigned)((N + BN - 1) / BN), (unsigned)ksplit);
  hipLaunchKernelGGL((router_gemm_dma_kernel<BM, BN, NS, WM, WN>), grid, dim3(64 * WM * WN), 0,
                     s, x, w, T, H, N, H / ksplit, out, N * ksplit);
  return hipGetLastError();
}

// Tile configuration per N, and the K partition count that fills the chip.
//   N >= 256: 256 x 128 tile, 16 waves, 3 stages (W re-read once per 256 rows)
//   N = 128, 64, 32: 64-row tiles, 4 waves (W is small and stays in L2)
//   N = 16 / 8: 32 x 16 tile, 2 waves (a pure x stream)
// ksplit doubles while blocks * ksplit is below the target and H still
// splits into whole 64-wide K steps; the partial sums are [T, ksplit*N].
struct GemmTile { int bm, bn, target; };
static GemmTile gemm_tile(int N) {
  if (N >= 256) return {256, 128, 256};
  if (N >= 32) return {64, N, 256};
  return {32, 16, 1024};
}

int router_gemm_ksplit(int T, int H, int N) {
  const GemmTile g = gemm_tile(N);
  const long long blocks = (long long)((T + g.bm - 1) / g.bm) * ((N + g.bn - 1) / g.bn);
  int ks = 1;
  while (blocks * ks < g.target && ks < 8 && H % (64 * ks * 2) == 0) ks *= 2;
  return ks;
}

// N in {8, 16, 32, 64, 128} or a multiple of 256; H % 64 == 0 (checked by
// the caller); H % (64 * ksplit) == 0.
hipError_t launch_router_gemm(const __bf16* x, const __bf16* w, int T, int H, int N, int ksplit,
                              float* out, hipStream_t s) {
  if (N >= 256) return launch_dma<256, 128, 3, 4, 4>(x, w, T, H, N, ksplit, out, s);
  if (N == 128) return launch_dma<64, 128, 3, 1, 4>(x, w, T, H, N, ksplit, out, s);
  if (N == 64) return launch_dma<64, 64, 3, 2, 2>(x, w, T, H, N, ksplit, out, s);
  if (N == 32) return launch_dma<64, 32, 3, 4, 1>(x, w, T, H, N, ksplit, out, s);
  return launch_dma<32, 16, 4, 2, 1>(x, w, T, H, N, ksplit, out, s);
}

}  // namespace moe
