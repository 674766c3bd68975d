// Per-row symmetric int8 quantisation for the int8 expert path.
//
// The reference's int8 experts quantise three kinds of rows inside run():
// the tokens (xquant_kernel, one scale per token), the SwiGLU output h after a
// Walsh-Hadamard rotation of its contraction axis (hquant_kernel, one scale
// per row), and the expert weights (wquant_kernel; the down projection
// rotated the same way) -- kernel.cu:61-66, kernel.cu:125-129,
// moe_wq.h:150-188.  This kernel serves all three:
//
//   v      = row r of x (bf16 -> fp32, exact), optionally rotated in blocks of
//            128 along the row by the UNNORMALISED Walsh-Hadamard transform
//            (butterfly stages s = 1, 2, ..., 64: v[k] = a + b, v[k^s] = a - b
//            for k with bit s clear, a = v[k], b = v[k^s]);
//   amax   = max |v|;
//   q[r,k] = clamp(rint(v[k] * (127 / amax)), -127, 127)   (0 if amax == 0);
//   s[r]   = (amax / 127) * scale_mul.
//
// A rotated operand pair contracts to 128 x the unrotated product (H H^T =
// 128 I), so the caller folds 1/128 into one side's scale_mul.  The rotation
// spreads the heavy tail of h = silu(g) * u over 128 elements before it is
// rounded to 127 levels.  With group_counts, row r is skipped when
// group_counts[r / group_rows] == 0 (the weights of experts that received no
// rows are never read).
//
// Layout: one 256-thread block per row; thread t holds 16 consecutive
// elements of each 4096-wide chunk (two 16-byte loads), so eight neighbouring
// lanes hold one 128-element rotation block: four butterfly stages run inside
// a lane, three across lanes.  The row stays in registers between the amax
// and the rounding: HBM sees one read and one write.
#include "moe_common.h"

namespace moe {

constexpr int kQuantThreads = 256;
constexpr int kQuantChunk = kQuantThreads * 16;  // elements per chunk

template <int NC, bool HAD>
__global__ __launch_bounds__(kQuantThreads) void quant_rows_i8_kernel(
    const __bf16* __restrict__ x, int K, float scale_mul, int group_rows,
    const int* __restrict__ group_counts, signed char* __restrict__ q, float* __restrict__ s) {
  const long long r = blockIdx.x;
  if (group_counts && group_counts[r / group_rows] == 0) return;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const __bf16* xr = x + r * K;
  float v[NC][16];
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e0 = c * kQuantChunk + t * 16;
    const bool ok = e0 < K;  // K % 16 == 0 (K % 128 == 0 with the rotation)
    u32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
    if (ok) {
      lo = ld_nt(reinterpret_cast<const u32x4*>(xr + e0));
      hi = ld_nt(reinterpret_cast<const u32x4*>(xr + e0 + 8));
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      v[c][2 * h] = bf16lo(lo[h]);
      v[c][2 * h + 1] = bf16hi(lo[h]);
      v[c][8 + 2 * h] = bf16lo(hi[h]);
      v[c][8 + 2 * h + 1] = bf16hi(hi[h]);
    }
    if constexpr (HAD) {
#pragma unroll
      for (int st = 1; st < 16; st <<= 1)
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if ((k & st) == 0) {
            const float a = v[c][k], b = v[c][k ^ st];
            v[c][k] = a + b;
            v[c][k ^ st] = a - b;
          }
      // element index bits 4..6 are lane bits 0..2
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) {
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const float o = __shfl_xor(v[c][k], m, 64);
          v[c][k] = upper ? o - v[c][k] : v[c][k] + o;
        }
      }
    }
    if (ok)
#pragma unroll
      for (int k = 0; k < 16; ++k) amax = fmaxf(amax, fabsf(v[c][k]));
  }
  // block max
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  __shared__ float part[kQuantThreads / 64];
  if (lane == 0) part[wave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  if (t == 0) s[r] = (amax / 127.0f) * scale_mul;
  signed char* qr = q + r * K;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e0 = c * kQuantChunk + t * 16;
    if (e0 >= K) continue;
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      unsigned int pk = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float qv = fminf(fmaxf(rintf(v[c][4 * w + b] * inv), -127.0f), 127.0f);
        pk |= ((unsigned int)(int)qv & 0xffu) << (8 * b);
      }
      out[w] = pk;
    }
    *reinterpret_cast<u32x4*>(qr + e0) = out;
  }
}

template <int NC>
static void launch_nc(const __bf16* x, long long R, int K, bool had, float scale_mul,
                      int group_rows, const int* counts, signed char* q, float* s,
                      hipStream_t st) {
  const dim3 grid((unsigned)R), blk(kQuantThreads);
  if (had)
    hipLaunchKernelGGL((quant_rows_i8_kernel<NC, true>), grid, blk, 0, st, x, K, scale_mul,
                       group_rows, counts, q, s);
  else
    hipLaunchKernelGGL((quant_rows_i8_kernel<NC, false>), grid, blk, 0, st, x, K, scale_mul,
                       group_rows, counts, q, s);
}

int quant_rows_max_k() { return 4 * kQuantChunk; }

hipError_t launch_quant_rows_i8(const __bf16* x, long long R, int K, bool had, float scale_mul,
                                int group_rows, const int* counts, signed char* q, float* s,
                                hipStream_t st) {
  if (R == 0) return hipSuccess;
  if (K <= kQuantChunk)
    launch_nc<1>(x, R, K, had, scale_mul, group_rows, counts, q, s, st);
  else if (K <= 2 * kQuantChunk)
    launch_nc<2>(x, R, K, had, scale_mul, group_rows, counts, q, s, st);
  else
    launch_nc<4>(x, R, K, had, scale_mul, group_rows, counts, q, s, st);
  return hipGetLastError();
}

}  // namespace moe
