// Expert grouped GEMM over the expert-contiguous rows the permute produces.
//
// Replaces the reference's CUTLASS grouped GEMMs (moe_gemm.h:66-95,
// moe_gemm.cu:616-650): group g owns rows [offs[g-1], offs[g]) of a
// (offs = inclusive group ends, offs[-1] = 0 -- exactly `offsets + 1` of
// moe_permute) and
//   plain : out[r, :] = a[r, :] . w[g]^T                     (grouped_mm)
//   swiglu: h[r, :]   = silu(a[r, :] . wg[g]^T) * (a[r, :] . wu[g]^T)
//           (grouped_mm_pair followed by silu*mul, fused into the epilogue)
// with a [M, K] bf16, w [G, N, K] bf16 (both K-contiguous), fp32 accumulate.
//
// Plan (the reference's plan_kernel builds per-group pointers for CUTLASS on
// the device; here it is one scan): tile_start[g] = sum over g' < g of
// ceil(m_g' / BM), on the device, so nothing waits for the host.  Up to 256
// groups every block scans the group ends itself (no plan launch); beyond,
// gg_plan_kernel writes tile_start into the workspace first.  The grid is
// sized by the bound sum ceil(m_g / BM) <= ceil(M / BM) + G; blocks past the
// last tile return at once.
//
// Tiles: 256 rows x 256 weight rows (128 x 512 for groups of at most 128
// rows on average), 128-byte K steps (64 bf16 or 128 int8 elements), staged
// in LDS by the gfx950 global_load_lds DMA into a 2-stage ring with an
// XOR-swizzled 16-byte chunk layout, v_mfma_f32_16x16x32_bf16 or
// v_mfma_i32_16x16x64_i8 accumulators (bf16 / int8 A: 8 waves of 64 x 128
// with a software-pipelined K loop; fp8 A: 16 waves of 64 x 64, plain loop).
// Block ids are remapped so that each XCD runs a contiguous range of logical
// tiles, and inside a group the tiles go in 4 x 8 (row x column) super-tiles:
// the blocks running together on one XCD share A and weight slices in L2.
//
// swiglu interleaves the two weights at 16-row granularity inside the B
// tile (rows 16f..16f+15 come from wg for even f, from wu for odd f), so the
// gate and up accumulators of the same output columns sit in one wave and
// the epilogue forms h without an exchange.  A tile then covers half its
// weight rows in output columns.
//
// Identity shortcut (the reference's ident_a / ident_m): a group whose row
// count equals ident_m takes its A rows from ident_a (row i of the group =
// row i of ident_a) instead of a.
#include "moe_common.h"

namespace moe {

constexpr int kGgBN = 256;  // narrowest tile: weight rows per tile (tile shape: template parameters)

// One workgroup of 1024 threads: inclusive scan of per-group tile counts.
__global__ __launch_bounds__(1024) void gg_plan_kernel(const int* __restrict__ offs, int G, int M,
                                                       int bm, int* __restrict__ tile_start) {
  __shared__ int part[16];
  __shared__ int carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int base = 0; base < G; base += 1024) {
    const int g = base + threadIdx.x;
    int tiles = 0;
    if (g < G) {
      const int lo = g > 0 ? min(max(offs[g - 1], 0), M) : 0;
      const int hi = min(max(offs[g], 0), M);
      tiles = hi > lo ? (hi - lo + bm - 1) / bm : 0;
    }
    // wave inclusive scan
    int v = tiles;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(v, o, 64);
      if (lane >= o) v += u;
    }
    if (lane == 63) part[wave] = v;
    __syncthreads();
    if (threadIdx.x < 16) {
      int p = part[threadIdx.x];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const int u = __shfl_up(p, o, 16);
        if ((threadIdx.x & 15) >= o) p += u;
      }
      part[threadIdx.x] = p;  // inclusive over waves
    }
    __syncthreads();
    const int incl = carry + (wave > 0 ? part[wave - 1] : 0) + v;
    if (g < G) tile_start[g + 1] = incl;
    if (g == 0) tile_start[0] = 0;
    __syncthreads();
    if (threadIdx.x == 1023) carry = incl;
    __syncthreads();
  }
  if (G == 0 && threadIdx.x == 0) tile_start[0] = 0;
}

// Up to kScanG groups a block finds its group itself: one wave-wide scan of
// the row-tile counts per 64 groups (a load or two from L2, shuffles and a
// ballot), instead of a separate plan launch and a binary search over its
// output (a chain of dependent loads at the start of every tile).
constexpr int kScanG = 256;

// Row tiles of group gi (ends clamped into [0, M], as the tile itself does);
// 0 past G.
__device__ __forceinline__ int group_tiles(const int* __restrict__ offs, int gi, int G, int M,
                                           int bm) {
  if (gi >= G) return 0;
  const int lo = gi > 0 ? min(max(offs[gi - 1], 0), M) : 0;
  const int hi = min(max(offs[gi], 0), M);
  return hi > lo ? (hi - lo + bm - 1) / bm : 0;
}

// Inclusive wave scan.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(v, o, 64);
    if (lane >= o) v += n;
  }
  return v;
}

// silu(g) * u in fp32
__device__ __forceinline__ float swiglu(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// 16 e4m3fn bytes -> 16 bf16(q * s): exact fp8 -> fp32 conversion, one fp32
// multiply, and the gfx950 fp32 -> bf16 conversion (round to nearest even).
__device__ __forceinline__ void dequant16(u32x4 raw, float s, bf16x8& lo8, bf16x8& hi8) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)raw[h], false);
    const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)raw[h], true);
    bf16x8& d = h < 2 ? lo8 : hi8;
    const int o = (h & 1) * 4;
    d[o + 0] = (__bf16)(a[0] * s);
    d[o + 1] = (__bf16)(a[1] * s);
    d[o + 2] = (__bf16)(b[0] * s);
    d[o + 3] = (__bf16)(b[1] * s);
  }
}

// Accumulator type and one MFMA of the K loop: bf16 16x16x32 (fp32 acc) or
// int8 16x16x64 (int32 acc, exact).  Both read 16 bytes per lane per operand.
typedef int i32x4 __attribute__((ext_vector_type(4)));
template <bool I8> struct AccOf { typedef f32x4 type; };
template <> struct AccOf<true> { typedef i32x4 type; };
template <bool I8>
__device__ __forceinline__ typename AccOf<I8>::type mfma_step(bf16x8 a, bf16x8 b,
                                                              typename AccOf<I8>::type c) {
  if constexpr (I8)
    return __builtin_amdgcn_mfma_i32_16x16x64_i8((i32x4)a, (i32x4)b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 32-bit LDS address of a __shared__ location, for inline-asm LDS reads.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)((__attribute__((address_space(3))) const char*)p);
}

// The A operand's row map (bf16 and int8 A) and the row / column scales of the
// int8 operands (unused by the bf16 and fp8 paths).
struct GgExtra {
  const float* a;      // int8: per row of a
  const int* a_idx;    // NULL, or [M]: operand row r is row a_idx[r] of a (data and scale)
  const float* ident;  // [ident_m] per row of ident_a
  const float* w0;     // [G, N] per weight row of w0
  const float* w1;     // [G, N] per weight row of w1 (SwiGLU up)
};

template <bool SWIGLU, bool AFP8, int BK, int NS, int WM, int WN, bool PIPE, int BM, bool I8,
          int BNT>
__global__ __launch_bounds__(64 * WM * WN) void grouped_gemm_kernel(
    const void* __restrict__ a_, const float* __restrict__ a_scales, const void* __restrict__ ident_,
    int ident_m, const void* __restrict__ w0_, const void* __restrict__ w1_,
    const int* __restrict__ offs, const int* __restrict__ tile_start, int G, int M, int N, int K,
    int n_tiles, unsigned short* __restrict__ out, GgExtra i8s) {
  // LDS rows: B (weights) BK*WEL bytes; A BK*2 bytes (bf16) or BK bytes (fp8,
  // int8).  bf16 steps are 64 wide, int8 steps 128 wide: 128-byte rows either
  // way.  A DMA wave instruction moves 1 KB = 1024 / row-bytes rows.
  constexpr int BN = BNT;  // weight rows per tile
  constexpr int WEL = I8 ? 1 : 2;  // bytes per weight element
  constexpr int ROWB = BK * WEL, CH = ROWB / 16, RPI = 1024 / ROWB;
  constexpr int AROWB = (AFP8 || I8) ? BK : BK * 2, ACH = AROWB / 16, ARPI = 1024 / AROWB;
  // MFMA depth: v_mfma_f32_16x16x32_bf16 or v_mfma_i32_16x16x64_i8; both
  // take 16 bytes per lane with the same lane -> (row, K chunk) layout.
  constexpr int KSUB = I8 ? 64 : 32;
  const char* const w0 = (const char*)w0_;
  const char* const w1 = (const char*)w1_;
  constexpr int A_BYTES = BM * AROWB, STAGE_B = A_BYTES + BN * ROWB;
  // fp8 A: the DMA stages hold the e4m3fn bytes; each K step they are
  // dequantised once, cooperatively, into one bf16 tile (BM x BK) that the
  // fragment reads use.
  constexpr int DQ_BYTES = AFP8 ? BM * BK * 2 : 0;
  constexpr int NW = WM * WN, NT = 64 * NW;
  constexpr int A_INST = BM / ARPI, B_INST = BN / RPI, PER_WAVE = (A_INST + B_INST) / NW;
  constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 16, FN = WTN / 16;
  static_assert(I8 ? BK == 128 : (BK == 32 || BK == 64), "K step of one or two MFMA depths");
  static_assert(!(I8 && AFP8), "int8 and fp8 A are separate paths");
  static_assert((A_INST + B_INST) % NW == 0, "every wave issues the same number of loads");
  static_assert(!AFP8 || BK == 64, "fp8 A: one 128-wide scale block spans two K steps");
  static_assert(!AFP8 || (BM * ACH) % NT == 0, "fp8 A: whole 16-byte chunks per thread per K step");
  static_assert(!SWIGLU || FN % 2 == 0, "swiglu: gate/up fragment pairs inside one wave");
  static_assert(!PIPE || (!AFP8 && ROWB == 128 && NS == 2 &&
                          ((BM == 256 && BN == 256 && WM == 4 && WN == 2) ||
                           (BM == 128 && BN == 512 && WM == 2 && WN == 4))),
                "pipelined loop: bf16 / int8 A, 2 stages of 128-byte rows, 8 waves of 64 x 128: "
                "256 x 256 or 128 x 512 tiles");
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE_B + DQ_BYTES];
  char* const dq = lds + NS * STAGE_B;
  const char* a = (const char*)a_;
  const char* ident_a = (const char*)ident_;
  constexpr int AEL = (AFP8 || I8) ? 1 : 2;  // bytes per A element

  // XCD-aware order: hardware block b runs on XCD b % 8.  The grid is sized
  // by a bound on the tile count; the real count nreal is known here, and the
  // logical tiles [x*r, (x+1)*r), r = ceil(nreal / 8), all run on XCD x, so
  // every XCD gets an eighth of the real tiles.  (Spreading the bound instead
  // leaves the bound's surplus on the last XCD and up to a round more on the
  // others: the T = 2048 shared down projection, 256 tiles, took 305 us.)
  // Logical tiles are numbered group by group: group g owns
  // [gstart * n_tiles, (gstart + mtg) * n_tiles), gstart = tile_start[g].
  const unsigned b = blockIdx.x;
  const int lane0 = threadIdx.x & 63;
  // total row tiles: from the plan (G > kScanG) or a scan of the group ends
  int total_rt = 0, incl0 = 0, tiles0 = 0;  // incl0 / tiles0: groups 0..63, lane = group
  if (G <= kScanG) {
    for (int base = 0; base < G; base += 64) {
      const int t = group_tiles(offs, base + lane0, G, M, BM);
      const int incl = wave_incl_scan(t);
      if (base == 0) {
        incl0 = incl;
        tiles0 = t;
      }
      total_rt += __shfl(incl, 63, 64);
    }
  } else {
    total_rt = tile_start[G];
  }
  total_rt = __builtin_amdgcn_readfirstlane(total_rt);  // wave-uniform: keep it in an SGPR
  const unsigned nreal = (unsigned)total_rt * (unsigned)n_tiles;
  const unsigned r = (nreal + 7u) >> 3;
  if ((b >> 3) >= r) return;
  const unsigned l = (b & 7u) * r + (b >> 3);
  if (l >= nreal) return;
  const int lt = (int)(l / (unsigned)n_tiles);
  // group g of row tile lt: gstart <= lt < gstart + mtg (the first group whose
  // inclusive tile count exceeds lt; groups without tiles never qualify)
  int g = 0, gstart = 0, mtg = 0;
  if (G <= 64) {
    const unsigned long long m = __ballot(lane0 < G && incl0 > lt);
    g = __ffsll((long long)m) - 1;
    mtg = __shfl(tiles0, g, 64);
    gstart = __shfl(incl0, g, 64) - mtg;
  } else if (G <= kScanG) {
    int carry = 0;
    for (int base = 0; base < G; base += 64) {
      const int t = group_tiles(offs, base + lane0, G, M, BM);
      const int incl = wave_incl_scan(t) + carry;
      const unsigned long long m = __ballot(base + lane0 < G && incl > lt);
      if (m) {
        const int L = __ffsll((long long)m) - 1;
        g = base + L;
        mtg = __shfl(t, L, 64);
        gstart = __shfl(incl, L, 64) - mtg;
        break;
      }
      carry = __shfl(incl, 63, 64);
    }
  } else {
    // the last g with tile_start[g] <= lt
    int lo = 0, hi = G - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tile_start[mid] <= lt) lo = mid; else hi = mid - 1;
    }
    g = lo;
    gstart = tile_start[g];
    mtg = tile_start[g + 1] - gstart;
  }
  // wave-uniform results of shuffles: SGPRs, not VGPRs the K loop needs
  g = __builtin_amdgcn_readfirstlane(g);
  gstart = __builtin_amdgcn_readfirstlane(gstart);
  mtg = __builtin_amdgcn_readfirstlane(mtg);
  // Inside a group, column blocks of kSuperN n-tiles, row tiles across each
  // block, n fastest: 32 consecutive tiles (one XCD's co-running blocks) are
  // 4 row tiles x 8 weight tiles, so each A slice and each weight slice of a
  // K step is fetched from HBM once and then reused from that XCD's L2.
  constexpr int kSuperN = 8;
  const int li = (int)l - gstart * n_tiles;
  const int nblk = li / (mtg * kSuperN);
  const int rem = li - nblk * mtg * kSuperN;
  const int ncols = min(kSuperN, n_tiles - nblk * kSuperN);
  const int mt_local = rem / ncols;
  const int nt = nblk * kSuperN + rem % ncols;
  const int gs = g > 0 ? min(max(offs[g - 1], 0), M) : 0;
  const int ge = min(max(offs[g], 0), M);
  const int r0 = gs + mt_local * BM;               // first row of the tile
  const int rlast = ge - 1;                        // last row of the group
  const bool ident = ident_m > 0 && ge - gs == ident_m;

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  // A wave whose rows all lie past the group (the last, partial row tile of a
  // group) still issues its share of the DMA and joins every barrier, but
  // skips its fragment reads and MFMAs: its results are never stored.
  const bool live = r0 + wm * WTM <= rlast;
  // logical 16-byte chunk c of an LDS row r sits at c ^ swz(r): the 16 rows
  // of one fragment read fall on distinct bank groups
  auto swz = [](int r, int ch) { return ch == 8 ? (r >> 1) & 7 : (r >> 2) & 3; };
  const long long wbase = (long long)g * N * K * WEL;  // bytes

  // DMA sources (bytes) and the byte advance per K step of each instruction
  const char* src[PER_WAVE];
  int kstep[PER_WAVE];
#pragma unroll
  for (int q = 0; q < PER_WAVE; ++q) {
    const int gi = wave * PER_WAVE + q;
    if (gi < A_INST) {
      const int r = gi * ARPI + lane / ACH, p = lane % ACH;
      const int row = min(r0 + r, rlast);  // rows past the group are loaded, never stored
      const int arow_i = (!ident && i8s.a_idx) ? i8s.a_idx[row] : row;
      const char* arow = ident ? ident_a + (long long)(row - gs) * K * AEL
                               : a + (long long)arow_i * K * AEL;
      src[q] = arow + (p ^ swz(r, ACH)) * 16;
      kstep[q] = BK * AEL;
    } else {
      const int r = (gi - A_INST) * RPI + lane / CH, p = lane % CH;
      int wrow;
      const char* wsrc = w0;
      if (SWIGLU) {
        const int f = r >> 4;
        wrow = nt * (BN / 2) + (f >> 1) * 16 + (r & 15);
        if (f & 1) wsrc = w1;
      } else {
        wrow = nt * BN + r;
      }
      wrow = min(wrow, N - 1);
      src[q] = wsrc + wbase + (long long)wrow * K * WEL + (p ^ swz(r, CH)) * 16;
      kstep[q] = BK * WEL;
    }
  }
  auto issue = [&](int kt, int st) {
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
      auto* dst = (__attribute__((address_space(3))) void*)(lds + st * STAGE_B +
                                                            (wave * PER_WAVE + q) * 1024);
      __builtin_amdgcn_global_load_lds((const void*)(src[q] + (long long)kt * kstep[q]), dst, 16,
                                       0, 0);
    }
  };

  // fp8: every K step thread t dequantises the 16-byte chunks t, t + NT, ...
  // (chunk q: tile row q / ACH, 16-byte column q % ACH); it keeps each of
  // its rows' scales for the current 128-wide K block and the next block's,
  // loaded one block ahead.
  const int fr = lane & 15, fc = lane >> 4;
  const int nsb = K / 128;
  constexpr int DQ_PER = AFP8 ? BM * ACH / NT : 1;
  float sc[DQ_PER], scn[DQ_PER];
  int dq_row[DQ_PER];
#pragma unroll
  for (int u = 0; u < DQ_PER; ++u) {
    dq_row[u] = min(r0 + (int)(threadIdx.x + u * NT) / ACH, rlast) * nsb;
    sc[u] = AFP8 ? a_scales[dq_row[u]] : 0.0f;
    scn[u] = AFP8 && nsb > 1 ? a_scales[dq_row[u] + 1] : 0.0f;
  }

  using AccV = typename AccOf<I8>::type;
  AccV acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = AccV{0, 0, 0, 0};

  const int KT = K / BK;
  if constexpr (PIPE) {
    // Software-pipelined K loop, two 128-byte-row stages, each K step in two
    // halves (kk = 0, 1) with their own fragment registers F0 / F1.  The
    // MFMAs of a half are interleaved with the LDS reads of the next half's
    // fragments (one read after every second MFMA) and, in the kk = 1 half,
    // with the DMA of the stage after next (one instruction after every
    // fourth MFMA), so neither the LDS queue nor the DMA issue holds the
    // matrix pipe.  Step s:
    //   wait F0 (stage s, kk 0); MFMA(F0) + reads F1 (stage s, kk 1);
    //   wait F1 and stage s+1's DMA (this wave); barrier (every wave: stage
    //   s+1 landed, the reads of stage s done);
    //   MFMA(F1) + reads F0 (stage s+1, kk 0) + DMA of stage s+2 into stage
    //   s's buffer.
    // Each accumulator sees K steps ascending, kk 0 then 1: bit-identical to
    // the plain loop.
    const unsigned l0 = lds_addr(lds);
    unsigned abase[2][2], bbase[2][2];  // [stage][kk]: fragment 0; fragment i / j at +i*2048 / +j*2048
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const unsigned c = (unsigned)(((kk * 4 + fc) ^ swz(fr, CH)) * 16);
        abase[st][kk] = l0 + st * STAGE_B + (wm * WTM + fr) * AROWB + c;
        bbase[st][kk] = l0 + st * STAGE_B + A_BYTES + (wn * WTN + fr) * ROWB + c;
      }
    bf16x8 a0[FM], b0[FN], a1[FM], b1[FN];
    // One 16-byte LDS fragment read issued as an instruction the compiler does
    // not track: the loop places its own lgkmcnt waits, so the reads stay in
    // flight across the MFMAs they are interleaved with.
    auto read_one = [&](bf16x8& dst, unsigned addr) {
      asm volatile("ds_read_b128 %0, %1" : "=v"(dst) : "v"(addr));
    };
    auto dma_one = [&](int q, int kt, int st) {
      auto* dst = (__attribute__((address_space(3))) void*)(lds + st * STAGE_B +
                                                            (wave * PER_WAVE + q) * 1024);
      __builtin_amdgcn_global_load_lds((const void*)(src[q] + (long long)kt * kstep[q]), dst, 16,
                                       0, 0);
    };
    constexpr int kReads = FM + FN;
    // DMA instruction q follows MFMA q * kDs + kDs / 2
    constexpr int kDs = FM * FN >= 4 * PER_WAVE ? 4 : 2;
    static_assert(2 * kReads <= FM * FN && kDs * PER_WAVE <= FM * FN,
                  "the reads and the DMA fit between the MFMAs of a half step");
    // MFMAs on (av, bv); reads into (ra, rb) from (rab, rbb) when rd; DMA of
    // stage dkt into buffer dst when dkt >= 0
    auto half = [&](bf16x8 (&av)[FM], bf16x8 (&bv)[FN], bf16x8 (&ra)[FM], bf16x8 (&rb)[FN],
                    unsigned rab, unsigned rbb, bool rd, int dkt, int dst) {
#pragma unroll
      for (int t = 0; t < FM * FN; ++t) {
        acc[t / FN][t % FN] = mfma_step<I8>(av[t / FN], bv[t % FN], acc[t / FN][t % FN]);
        if ((t & 1) && (t >> 1) < kReads && rd) {
          const int r = t >> 1;
          if (r < FM) read_one(ra[r], rab + r * 2048);
          else read_one(rb[r - FM], rbb + (r - FM) * 2048);
        }
        if (t % kDs == kDs / 2 && t / kDs < PER_WAVE && dkt >= 0) dma_one(t / kDs, dkt, dst);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    issue(0, 0);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    if (KT > 1) issue(1, 1);
    if (!live) {
      // DMA and barriers only, in the same order as the live loop below
      for (int k2 = 0; k2 < KT; ++k2) {
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (k2 + 2 < KT) issue(k2 + 2, k2 & 1);
      }
    } else {
#pragma unroll
      for (int r = 0; r < FM; ++r) read_one(a0[r], abase[0][0] + r * 2048);
#pragma unroll
      for (int r = 0; r < FN; ++r) read_one(b0[r], bbase[0][0] + r * 2048);
      for (int kt = 0; kt < KT; kt += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int k2 = kt + u;  // stage k2 lives in buffer u
          if (k2 < KT) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // F0 of stage k2
            __builtin_amdgcn_sched_barrier(0);
            half(a0, b0, a1, b1, abase[u][1], bbase[u][1], true, -1, 0);
            // F1 landed (this wave's reads of stage k2 are done) and stage
            // k2+1's DMA landed; the barrier makes both true for every wave
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            half(a1, b1, a0, b0, abase[u ^ 1][0], bbase[u ^ 1][0], k2 + 1 < KT,
                 k2 + 2 < KT ? k2 + 2 : -1, u);
          }
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  } else {
  #pragma unroll
    for (int st = 0; st < NS - 1; ++st)
      if (st < KT) issue(st, st);
    for (int kt = 0; kt < KT; ++kt) {
      // this wave's stage kt landed once at most the NS-2 later stages are
      // outstanding; the barrier then publishes every wave's DMA and retires
      // all reads of the buffer reloaded next
      if (kt + NS - 2 < KT)
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 2) * PER_WAVE) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      if (kt + NS - 1 < KT) issue(kt + NS - 1, (kt + NS - 1) % NS);
      const char* sb = lds + (kt % NS) * STAGE_B;
      if (AFP8) {
        const bool nb = kt > 0 && (kt & 1) == 0;  // a new 128-wide scale block starts
  #pragma unroll
        for (int u = 0; u < DQ_PER; ++u) {
          if (nb) {
            sc[u] = scn[u];
            scn[u] = (kt >> 1) + 1 < nsb ? a_scales[dq_row[u] + (kt >> 1) + 1] : 0.0f;
          }
          const int q = threadIdx.x + u * NT, r = q / ACH, c = q % ACH;
          const u32x4 raw = *reinterpret_cast<const u32x4*>(sb + r * AROWB + ((c ^ swz(r, ACH)) * 16));
          bf16x8 lo8, hi8;
          dequant16(raw, sc[u], lo8, hi8);
          *reinterpret_cast<bf16x8*>(dq + r * ROWB + (((2 * c) ^ swz(r, CH)) * 16)) = lo8;
          *reinterpret_cast<bf16x8*>(dq + r * ROWB + (((2 * c + 1) ^ swz(r, CH)) * 16)) = hi8;
        }
        // the bf16 tile is complete for every wave (its previous contents were
        // retired by the barrier at the top of this step)
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
      }
      if (!live) continue;
  #pragma unroll
      for (int kk = 0; kk < BK / KSUB; ++kk) {
        bf16x8 bv[FN];
  #pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int r = wn * WTN + j * 16 + fr, c = kk * 4 + fc;
          bv[j] = *reinterpret_cast<const bf16x8*>(sb + A_BYTES + r * ROWB + ((c ^ swz(r, CH)) * 16));
        }
        bf16x8 av[FM];
  #pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int r = wm * WTM + i * 16 + fr, c = kk * 4 + fc;
          av[i] = AFP8 ? *reinterpret_cast<const bf16x8*>(dq + r * ROWB + ((c ^ swz(r, CH)) * 16))
                       : *reinterpret_cast<const bf16x8*>(sb + r * AROWB + ((c ^ swz(r, ACH)) * 16));
        }
  #pragma unroll
        for (int i = 0; i < FM; ++i)
  #pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = mfma_step<I8>(av[i], bv[j], acc[i][j]);
      }
    }
  }

  // Epilogue: lane holds rows (lane>>4)*4 + r, column lane & 15 of each 16x16 tile.
  // int8: value = float(acc) * (row scale * column scale), in that order.  All
  // scales are loaded before the first store (a load issued after a store
  // would wait for it: both count in vmcnt).
  constexpr int OUTC = SWIGLU ? BN / 2 : BN;  // output columns of a tile
  float cs0[FN], cs1[FN], rsc[FM][4];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    cs0[j] = cs1[j] = 1.0f;
    if constexpr (I8) {
      const int col = SWIGLU ? nt * (BN / 2) + (wn * FN + (j & ~1)) / 2 * 16 + (lane & 15)
                             : nt * BN + wn * WTN + j * 16 + (lane & 15);
      if (col < N) {
        cs0[j] = i8s.w0[(long long)g * N + col];
        if (SWIGLU) cs1[j] = i8s.w1[(long long)g * N + col];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      rsc[i][r] = 1.0f;
      if constexpr (I8) {
        const int row = min(r0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r, rlast);
        rsc[i][r] = ident ? i8s.ident[row - gs] : i8s.a[i8s.a_idx ? i8s.a_idx[row] : row];
      }
    }
  // output value of accumulator (i, j, r); SwiGLU pairs j (gate) with j + 1 (up)
  auto value = [&](int i, int j, int r) -> float {
    if (SWIGLU) {
      float gv, uv;
      if constexpr (I8) {
        gv = (float)acc[i][j][r] * (rsc[i][r] * cs0[j]);
        uv = (float)acc[i][j + 1][r] * (rsc[i][r] * cs1[j]);
      } else {
        gv = acc[i][j][r];
        uv = acc[i][j + 1][r];
      }
      return swiglu(gv, uv);
    }
    if constexpr (I8) return (float)acc[i][j][r] * (rsc[i][r] * cs0[j]);
    else return acc[i][j][r];
  };
  constexpr int JSTEP = SWIGLU ? 2 : 1;
  const int ldo = N;
  if ((N & 7) == 0) {
    // Stage the bf16 tile in LDS (the operand buffers are idle once every wave is
    // past its last fragment read), then write whole 16-byte chunks of output
    // rows.  LDS row = OUTC bf16; 16-byte chunk c of tile row rl sits at
    // c ^ (2 * ((rl >> 2) & 3)), so the four row groups one ds_write covers
    // land in distinct banks.
    static_assert(BM * OUTC * 2 <= (int)sizeof(lds), "output tile fits in the LDS");
    constexpr int RCH = OUTC / 8;
    unsigned short* ct = reinterpret_cast<unsigned short*>(lds);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rl = wm * WTM + i * 16 + (lane >> 4) * 4 + r;
        const int sw = 2 * ((rl >> 2) & 3);
#pragma unroll
        for (int j = 0; j < FN; j += JSTEP) {
          const int cl = (SWIGLU ? (wn * FN + j) / 2 * 16 : wn * WTN + j * 16) + (lane & 15);
          ct[rl * OUTC + (((cl >> 3) ^ sw) << 3) + (cl & 7)] = (unsigned short)f2bf(value(i, j, r));
        }
      }
    __syncthreads();
    const int c0 = nt * OUTC;
    for (int q = threadIdx.x; q < BM * RCH; q += NT) {
      const int rl = q / RCH, c = q % RCH;
      const int row = r0 + rl, col = c0 + c * 8;
      if (row > rlast || col >= N) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(ct + rl * OUTC +
                                                      ((c ^ (2 * ((rl >> 2) & 3))) << 3));
      *reinterpret_cast<u32x4*>(out + (long long)row * ldo + col) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = r0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r;
      if (row > rlast) continue;
      unsigned short* orow = out + (long long)row * ldo;
#pragma unroll
      for (int j = 0; j < FN; j += JSTEP) {
        const int col = SWIGLU ? nt * (BN / 2) + (wn * FN + j) / 2 * 16 + (lane & 15)
                               : nt * BN + wn * WTN + j * 16 + (lane & 15);
        if (col < N) orow[col] = (unsigned short)f2bf(value(i, j, r));
      }
    }
}

int grouped_gemm_n_tiles(int N, bool swiglu) {
  const int per = swiglu ? kGgBN / 2 : kGgBN;
  return (N + per - 1) / per;
}
template <int BNT>
static int n_tiles_of(int N, bool swiglu) {
  const int per = swiglu ? BNT / 2 : BNT;
  return (N + per - 1) / per;
}

template <bool AFP8, int WM, int WN, bool PIPE, int BM, int NS, bool I8 = false, int BNT = 256>
static hipError_t launch_gg(const void* a, const float* a_scales, const void* ident_a, int ident_m,
                            const void* w0, const void* w1, const int32_t* offs, int G, int M, int N,
                            int K, bool swiglu, void* out, int32_t* tile_start, hipStream_t s,
                            GgExtra i8s = GgExtra{}) {
  constexpr int BK = I8 ? 128 : 64;  // K-step elements
  if (G > kScanG) {  // the kernel scans up to kScanG group ends itself
    hipLaunchKernelGGL(gg_plan_kernel, dim3(1), dim3(1024), 0, s, offs, G, M, BM, tile_start);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (M == 0 || N == 0 || G == 0) return hipSuccess;
  const int n_tiles = n_tiles_of<BNT>(N, swiglu);
  const long long m_bound = ((long long)M + BM - 1) / BM + G;
  long long blocks = m_bound * n_tiles;
  blocks = (blocks + 7) / 8 * 8;
  const dim3 grid((unsigned)blocks), blk(64 * WM * WN);
  if (swiglu)
    hipLaunchKernelGGL((grouped_gemm_kernel<true, AFP8, BK, NS, WM, WN, PIPE, BM, I8, BNT>), grid, blk,
                       0, s, a, a_scales, ident_a, ident_m, w0, w1, offs, tile_start, G, M, N, K,
                       n_tiles, (unsigned short*)out, i8s);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<false, AFP8, BK, NS, WM, WN, PIPE, BM, I8, BNT>), grid, blk,
                       0, s, a, a_scales, ident_a, ident_m, w0, w0, offs, tile_start, G, M, N, K,
                       n_tiles, (unsigned short*)out, i8s);
  return hipGetLastError();
}

// tile_start: [G+1] ints of workspace.  offs: inclusive group ends (device).
// a_scales == NULL: a is bf16.  Else a is e4m3fn bytes with one fp32 scale per
// row and 128-wide K block ([M, K/128]).  a_rows (bf16 A only; may be NULL):
// operand row r is row a_rows[r] of a.
hipError_t launch_grouped_gemm(const void* a, const float* a_scales, const int32_t* a_rows,
                               const void* ident_a, int ident_m, const void* w0, const void* w1,
                               const int32_t* offs, int G, int M, int N, int K, bool swiglu,
                               void* out, int32_t* tile_start, hipStream_t s) {
  const GgExtra ex{nullptr, a_rows, nullptr, nullptr, nullptr};
  // fp8 A (its dequantisation pass needs a barrier inside each K step): 256-row
  // tiles, 16 waves of 64 x 64, the plain loop.
  if (a_scales)
    return launch_gg<true, 4, 4, false, 256, 2>(a, a_scales, ident_a, ident_m, w0, w1, offs, G, M,
                                                N, K, swiglu, out, tile_start, s);
  // bf16 A with at most 128 rows per group on average (e.g. T = 512 routed
  // top-8 over 64 experts): 128 x 512 tiles, which pad a small group's last
  // row tile less than 256 x 256; against 128 x 256 they move 40 instead of 48
  // bytes per K step per 1024 MFMA cycles.  The pipelined loop with 8 waves of
  // 64 x 128, as below.  run() measured (ms, 128 x 512 / 256 x 256): spread
  // routing T = 512 (64 rows per expert) int8 4.93 / 5.04, bf16 2.50 / 2.67;
  // T = 1571 (196 rows) int8 5.69 / 5.46, bf16 3.80 / 3.29; the harness's
  // routing (8 groups of T rows) T = 1571 int8 2.33 / 2.15, T = 2048 bf16
  // 3.68 / 3.20.
  if ((long long)M <= 128ll * G)
    return launch_gg<false, 2, 4, true, 128, 2, false, 512>(a, nullptr, ident_a, ident_m, w0, w1,
                                                            offs, G, M, N, K, swiglu, out,
                                                            tile_start, s, ex);
  // bf16 A, larger groups: 256 x 256 tiles, 8 waves of 64 x 128 accumulators,
  // the software-pipelined K loop.
  return launch_gg<false, 4, 2, true, 256, 2>(a, nullptr, ident_a, ident_m, w0, w1, offs, G, M, N,
                                              K, swiglu, out, tile_start, s, ex);
}

// int8 A and weights, int32 accumulation, 128-wide K steps: the same tile
// choice as bf16 (the LDS rows are 128 bytes in both).
hipError_t launch_grouped_gemm_i8(const void* a, const float* a_rs, const int32_t* a_rs_idx,
                                  const void* ident_a, const float* ident_rs, int ident_m,
                                  const void* w0, const float* w0s, const void* w1,
                                  const float* w1s, const int32_t* offs, int G, int M, int N, int K,
                                  bool swiglu, void* out, int32_t* tile_start, hipStream_t s) {
  const GgExtra sc{a_rs, a_rs_idx, ident_rs, w0s, swiglu ? w1s : w0s};
  if ((long long)M <= 128ll * G)
    return launch_gg<false, 2, 4, true, 128, 2, true, 512>(a, nullptr, ident_a, ident_m, w0, w1,
                                                           offs, G, M, N, K, swiglu, out,
                                                           tile_start, s, sc);
  return launch_gg<false, 4, 2, true, 256, 2, true>(a, nullptr, ident_a, ident_m, w0, w1, offs, G,
                                                    M, N, K, swiglu, out, tile_start, s, sc);
}

}  // namespace moe
