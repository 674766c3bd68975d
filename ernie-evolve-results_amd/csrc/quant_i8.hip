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
//            n = 16 or 128 along the row by the UNNORMALISED Walsh-Hadamard
//            transform (butterfly stages s = 1, 2, ..., n/2: v[k] = a + b,
//            v[k^s] = a - b for k with bit s clear, a = v[k], b = v[k^s]);
//   amax   = max |v|;
//   q[r,k] = clamp(rint(v[k] * (127 / amax)), -127, 127)   (0 if amax == 0);
//   s[r]   = (amax / 127) * scale_mul.
//
// A rotated operand pair contracts to n x the unrotated product (H H^T =
// n I), so the caller folds 1/n into one side's scale_mul.  The rotation
// spreads the heavy tail of h = silu(g) * u over n elements before it is
// rounded to 127 levels (the reference uses n = 16, moe_wq.h:170-188).  With group_counts, row r is skipped when
// group_counts[r / group_rows] == 0 (the weights of experts that received no
// rows are never read).
//
// Layout: 256-thread blocks (at most 8 per CU), which walk the rows of the
// non-empty groups only (listed per block in LDS), RB consecutive rows per pass
// (RB = 4 / 2 / 1 for K up to 4096 / 8192 / 16384) and issuing all their
// loads before the first reduction; for one row, thread t holds 16 consecutive
// elements of each 4096-wide chunk (two 16-byte loads).  A 16-point block is
// one lane's; a 128-point block spans eight neighbouring lanes: four
// butterfly stages run inside a lane, three across lanes (DPP moves).  The row stays in registers between the amax
// and the rounding: HBM sees one read and one write.
#include "moe_common.h"

namespace moe {

constexpr int kQuantThreads = 256;
constexpr int kQuantChunk = kQuantThreads * 16;  // elements per chunk
constexpr int kQuantBlocks = 256 * 8;            // 8 resident blocks per CU
constexpr int kQuantMaxGroups = 4096;            // groups gated by group_counts

// v of lane (lane ^ m), m in {1, 2, 4}, through DPP moves (no LDS traffic):
// quad permutations for 1 and 2, a row shift by 4 either way for 4.
template <int>
__device__ __forceinline__ float xor_lane(float v, int m) {
  const int iv = __float_as_int(v);
  const int lane = threadIdx.x & 63;
  if (m == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false));
  if (m == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false));
  const int up = __builtin_amdgcn_update_dpp(0, iv, 0x104, 0xF, 0xF, false);  // lane + 4
  const int dn = __builtin_amdgcn_update_dpp(0, iv, 0x114, 0xF, 0xF, false);  // lane - 4
  return __int_as_float((lane & 4) ? dn : up);
}

template <int NC, int RB, int HAD>
__global__ __launch_bounds__(kQuantThreads) void quant_rows_i8_kernel(
    const __bf16* __restrict__ x, int R, int K, float scale_mul, int group_rows,
    const int* __restrict__ group_counts, signed char* __restrict__ q, float* __restrict__ s) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  __shared__ float part[RB][kQuantThreads / 64];
  // With group_counts, the rows to quantise are those of the non-empty groups:
  // wave 0 lists them in LDS (ascending), and the blocks walk only those rows
  // (virtual row v -> group grp[v / group_rows], row v % group_rows in it).
  __shared__ int grp[kQuantMaxGroups];
  __shared__ int n_grp;
  int Rv = R;
  if (group_counts) {
    if (wave == 0) {
      int n = 0;
      const int G = R / group_rows;
      for (int base = 0; base < G; base += 64) {
        const bool live = base + lane < G && group_counts[base + lane] != 0;
        const unsigned long long m = __ballot(live);
        if (live) grp[n + __popcll(m & ((1ull << lane) - 1ull))] = base + lane;
        n += __popcll(m);
      }
      if (lane == 0) n_grp = n;
    }
    __syncthreads();
    Rv = n_grp * group_rows;
  }
  for (int rb = blockIdx.x * RB; rb < Rv; rb += gridDim.x * RB) {
    // RB consecutive (virtual) rows per pass: all their loads are issued together
    bool act[RB];
    int rows[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int v = rb + i;
      act[i] = v < Rv;
      rows[i] = group_counts ? grp[min(v, Rv - 1) / group_rows] * group_rows + v % group_rows : v;
    }
    float v[RB][NC][16];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int e0 = c * kQuantChunk + t * 16;
        u32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
        if (act[i] && e0 < K) {  // K % 16 == 0 (K % 128 == 0 with the 128-point rotation)
          const __bf16* p = x + (long long)rows[i] * K + e0;
          lo = ld_nt(reinterpret_cast<const u32x4*>(p));
          hi = ld_nt(reinterpret_cast<const u32x4*>(p + 8));
        }
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          v[i][c][2 * h] = bf16lo(lo[h]);
          v[i][c][2 * h + 1] = bf16hi(lo[h]);
          v[i][c][8 + 2 * h] = bf16lo(hi[h]);
          v[i][c][8 + 2 * h + 1] = bf16hi(hi[h]);
        }
      }
    float amax[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      amax[i] = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if constexpr (HAD >= 16) {
#pragma unroll
          for (int st = 1; st < 16; st <<= 1)
#pragma unroll
            for (int k = 0; k < 16; ++k)
              if ((k & st) == 0) {
                const float a = v[i][c][k], b = v[i][c][k ^ st];
                v[i][c][k] = a + b;
                v[i][c][k ^ st] = a - b;
              }
        }
        if constexpr (HAD == 128) {
          // element index bits 4..6 are lane bits 0..2
#pragma unroll
          for (int m = 1; m < 8; m <<= 1) {
            const bool upper = (lane & m) != 0;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
              const float o = xor_lane<1>(v[i][c][k], m);
              v[i][c][k] = upper ? o - v[i][c][k] : v[i][c][k] + o;
            }
          }
        }
        // lanes past K hold zeros (and rotated zeros): they do not move the max
#pragma unroll
        for (int k = 0; k < 16; ++k) amax[i] = fmaxf(amax[i], fabsf(v[i][c][k]));
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) amax[i] = fmaxf(amax[i], __shfl_xor(amax[i], o, 64));
      if (lane == 0) part[i][wave] = amax[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      if (!act[i]) continue;
      const int r = rows[i];
      const float am = fmaxf(fmaxf(part[i][0], part[i][1]), fmaxf(part[i][2], part[i][3]));
      const float inv = am > 0.0f ? 127.0f / am : 0.0f;
      if (t == 0) s[r] = (am / 127.0f) * scale_mul;
      signed char* qr = q + (long long)r * K;
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
            const float qv = fminf(fmaxf(rintf(v[i][c][4 * w + b] * inv), -127.0f), 127.0f);
            pk |= ((unsigned int)(int)qv & 0xffu) << (8 * b);
          }
          out[w] = pk;
        }
        *reinterpret_cast<u32x4*>(qr + e0) = out;
      }
    }
    __syncthreads();  // part[] is rewritten by the next pass
  }
}

template <int NC, int RB>
static void launch_nc(const __bf16* x, long long R, int K, int had, float scale_mul,
                      int group_rows, const int* counts, signed char* q, float* s,
                      hipStream_t st) {
  const long long passes = (R + RB - 1) / RB;
  const dim3 grid((unsigned)(passes < kQuantBlocks ? passes : kQuantBlocks)), blk(kQuantThreads);
  if (had == 128)
    hipLaunchKernelGGL((quant_rows_i8_kernel<NC, RB, 128>), grid, blk, 0, st, x, (int)R, K,
                       scale_mul, group_rows, counts, q, s);
  else if (had == 16)
    hipLaunchKernelGGL((quant_rows_i8_kernel<NC, RB, 16>), grid, blk, 0, st, x, (int)R, K,
                       scale_mul, group_rows, counts, q, s);
  else
    hipLaunchKernelGGL((quant_rows_i8_kernel<NC, RB, 0>), grid, blk, 0, st, x, (int)R, K,
                       scale_mul, group_rows, counts, q, s);
}

int quant_rows_max_k() { return 4 * kQuantChunk; }
int quant_rows_max_groups() { return kQuantMaxGroups; }

hipError_t launch_quant_rows_i8(const __bf16* x, long long R, int K, int had, float scale_mul,
                                int group_rows, const int* counts, signed char* q, float* s,
                                hipStream_t st) {
  if (R == 0) return hipSuccess;
  if (K <= kQuantChunk)
    launch_nc<1, 4>(x, R, K, had, scale_mul, group_rows, counts, q, s, st);
  else if (K <= 2 * kQuantChunk)
    launch_nc<2, 2>(x, R, K, had, scale_mul, group_rows, counts, q, s, st);
  else
    launch_nc<4, 1>(x, R, K, had, scale_mul, group_rows, counts, q, s, st);
  return hipGetLastError();
}

}  // namespace moe
