// Stage 1: the router GEMM, logits[T,N] = x[T,H] . w[N,H]^T, bf16 in, fp32 out.
//
// Replaces the reference's cublasGemmEx call (K:4327-4339) with gfx950 MFMA
// kernels.  Both operands are K-contiguous (x row-major [T,H], w row-major
// [N,H]), which is exactly the operand layout of v_mfma_f32_16x16x32_bf16:
// a lane feeds 8 consecutive k of one row of A and the same 8 k of one
// column of B, so a fragment is a single 16-byte LDS read.
//
// Main kernel (N >= 64): tiles are brought into LDS by the gfx950
// global_load_lds_dwordx4 DMA (no register staging), into an NS-stage ring
// with an XOR-swizzled 16-byte-chunk layout (conflict-free fragment reads),
// one s_barrier per K step.  At N = 256 a 512-thread block owns 256 rows x
// all 256 experts: the router weight (3.7 MB) is then re-read from L2 once
// per 256 rows instead of once per 128, which halved the kernel's time on
// MI355X.  To still fill 256 CUs at T = 32768 the K range is split in two
// (split-K); the two fp32 partial sums land side by side as [T, 2N] and the
// scoring kernel adds them in a fixed order (deterministic, no atomics).
// 16 waves (4 per SIMD, 64x64 accumulator tiles) hide the DMA latency better
// than 8 waves with 128x64 tiles (measured 122 vs 141 us at T = 32768).
// x is loaded with the non-temporal bit: it streams through once.
//
// Small N (8..32) keeps a plain register-staged kernel: there the GEMM is a
// pure x stream.
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

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void router_gemm_kernel(const __bf16* __restrict__ x,
                                                          const __bf16* __restrict__ w,
                                                          int T, int H, int N,
                                                          float* __restrict__ out) {
  constexpr int BK = 64;
  constexpr int LDK = BK + 8;  // padded LDS row, elements
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int A_VEC = BM * (BK / 8), B_VEC = BN * (BK / 8);  // 16-byte vectors per tile
  constexpr int A_PER = (A_VEC + 255) / 256, B_PER = (B_VEC + 255) / 256;
  static_assert(WM * WN == 4, "4 waves");
  static_assert(FM >= 1 && FN >= 1, "wave tile below one MFMA tile");

  __shared__ __attribute__((aligned(16))) __bf16 sA[BM * LDK];
  __shared__ __attribute__((aligned(16))) __bf16 sB[BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const long long m0 = (long long)blockIdx.x * BM;
  const int n0 = blockIdx.y * BN;

  u32x4 ra[A_PER], rb[B_PER];
  auto gload = [&](int kt) {
    const long long kofs = (long long)kt * BK;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int idx = tid + i * 256;
      const int r = idx >> 3, c = idx & 7;
      const long long row = m0 + r;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (idx < A_VEC && row < T)
        v = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(x + row * H + kofs + c * 8));
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int idx = tid + i * 256;
      const int r = idx >> 3, c = idx & 7;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (idx < B_VEC && n0 + r < N)
        v = *reinterpret_cast<const u32x4*>(w + (long long)(n0 + r) * H + kofs + c * 8);
      rb[i] = v;
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int idx = tid + i * 256;
      if (idx < A_VEC)
        *reinterpret_cast<u32x4*>(sA + (idx >> 3) * LDK + (idx & 7) * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int idx = tid + i * 256;
      if (idx < B_VEC)
        *reinterpret_cast<u32x4*>(sB + (idx >> 3) * LDK + (idx & 7) * 8) = rb[i];
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int KT = H / BK;
  const int frow = lane & 15, fk = (lane >> 4) * 8;
  gload(0);
  for (int kt = 0; kt < KT; ++kt) {
    sstore();
    __syncthreads();
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      bf16x8 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(sA + (wm * WTM + i * 16 + frow) * LDK + kk + fk);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(sB + (wn * WTN + j * 16 + frow) * LDK + kk + fk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // 16x16 accumulator layout: lane holds column (lane & 15), rows 4*(lane >> 4) + r.
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + wn * WTN + j * 16 + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const long long row = m0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r;
        if (row < T && col < N) out[row * N + col] = acc[i][j][r];
      }
    }
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

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
      if (wave * PER_WAVE + q < A_INST)  // x: streamed once, non-temporal
        __builtin_amdgcn_global_load_lds((const void*)(src[q] + kt * BK), dst, 16, 0, 2);
      else
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

template <int BM, int BN, int WM, int WN>
static hipError_t launch_cfg(const __bf16* x, const __bf16* w, int T, int H, int N, float* out,
                             hipStream_t s) {
  const dim3 grid((unsigned)((T + BM - 1) / BM), (unsigned)((N + BN - 1) / BN));
  hipLaunchKernelGGL((router_gemm_kernel<BM, BN, WM, WN>), grid, dim3(256), 0, s, x, w, T, H, N,
                     out);
  return hipGetLastError();
}

template <int BM, int BN, int NS, int WM, int WN>
static hipError_t launch_dma(const __bf16* x, const __bf16* w, int T, int H, int N, int ksplit,
                             float* out, hipStream_t s) {
  const dim3 grid((unsigned)((T + BM - 1) / BM), (unsigned)(N / BN), (unsigned)ksplit);
  hipLaunchKernelGGL((router_gemm_dma_kernel<BM, BN, NS, WM, WN>), grid, dim3(64 * WM * WN), 0,
                     s, x, w, T, H, N, H / ksplit, out, N * ksplit);
  return hipGetLastError();
}

// Number of K partitions the GEMM uses for (T, H, N): 2 when the 256-row
// blocks alone would leave CUs idle, else 1.  The partial sums are [T, ksplit*N].
int router_gemm_ksplit(int T, int H, int N) {
  if (N < 256 || N % 256 != 0) return 1;
  const long long blocks = (long long)((T + 255) / 256) * (N / 256);
  return (blocks < 256 && H % 128 == 0) ? 2 : 1;
}

// N in {8, 16, 32, 64, 128} or a multiple of 256; H % 64 == 0 (checked by
// the caller).  ksplit > 1 only for N % 256 == 0 and H % (64 * ksplit) == 0.
hipError_t launch_router_gemm(const __bf16* x, const __bf16* w, int T, int H, int N, int ksplit,
                              float* out, hipStream_t s) {
  if (N >= 256) return launch_dma<256, 256, 2, 4, 4>(x, w, T, H, N, ksplit, out, s);
  if (N == 128) return launch_dma<256, 128, 2, 4, 2>(x, w, T, H, N, 1, out, s);
  if (N == 64) return launch_dma<128, 64, 3, 2, 2>(x, w, T, H, N, 1, out, s);
  if (N == 32) return launch_cfg<64, 32, 4, 1>(x, w, T, H, N, out, s);
  return launch_cfg<64, 16, 4, 1>(x, w, T, H, N, out, s);
}

}  // namespace moe
