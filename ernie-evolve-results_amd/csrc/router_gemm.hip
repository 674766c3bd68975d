// Stage 1: the router GEMM, logits[T,N] = x[T,H] . w[N,H]^T, bf16 in, fp32 out.
//
// Replaces the reference's cublasGemmEx call (K:4327-4339) with a gfx950 MFMA
// kernel.  Both operands are K-contiguous (x row-major [T,H], w row-major
// [N,H]), which is exactly the operand layout of v_mfma_f32_16x16x32_bf16:
// a lane feeds 8 consecutive k of one row of A and the same 8 k of one
// column of B, so a fragment is a single 16-byte LDS read.
//
// Tiling: a 256-thread workgroup (4 waves) owns BM rows x BN columns and
// walks K in steps of 64.  The x and w tiles are staged through LDS (rows
// padded by 16 bytes), the next tile is prefetched into registers while the
// current one feeds the MFMAs.  For the DeepSeek-V3 shape (N = 256) a block
// is 128 x 256, so x is read from HBM exactly once and w (3.7 MB) is re-read
// from L2 by each of the T/128 blocks.
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

template <int BM, int BN, int WM, int WN>
static hipError_t launch_cfg(const __bf16* x, const __bf16* w, int T, int H, int N, float* out,
                             hipStream_t s) {
  const dim3 grid((unsigned)((T + BM - 1) / BM), (unsigned)((N + BN - 1) / BN));
  hipLaunchKernelGGL((router_gemm_kernel<BM, BN, WM, WN>), grid, dim3(256), 0, s, x, w, T, H, N,
                     out);
  return hipGetLastError();
}

// N in {8, 16, 32, 64, 128} or a multiple of 256; H % 64 == 0 (checked by the caller).
hipError_t launch_router_gemm(const __bf16* x, const __bf16* w, int T, int H, int N, float* out,
                              hipStream_t s) {
  if (N >= 256) return launch_cfg<128, 256, 1, 4>(x, w, T, H, N, out, s);
  if (N == 128) return launch_cfg<64, 128, 2, 2>(x, w, T, H, N, out, s);
  if (N == 64) return launch_cfg<64, 64, 2, 2>(x, w, T, H, N, out, s);
  if (N == 32) return launch_cfg<64, 32, 4, 1>(x, w, T, H, N, out, s);
  return launch_cfg<64, 16, 4, 1>(x, w, T, H, N, out, s);
}

}  // namespace moe
