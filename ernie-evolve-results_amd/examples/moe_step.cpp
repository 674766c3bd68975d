// A C++ host program that drives libmoe_route.so through its C ABI alone (no
// torch): one DeepSeek-V3-style step -- route, stable permute + gather,
// combine -- on raw hipMalloc buffers, then checks the step's invariants:
//   * counts sum to T*k, offsets are the exclusive scan of counts;
//   * pair_row is a bijection onto the rows and row_token[pair_row[p]] = p / k;
//   * each expert segment holds ascending tokens;
//   * gathered rows equal x[row_token];
//   * with identity experts (y = xg) the combine returns x * sum_j w_j.
// This is what a C++ caller of the reference's run() (kernel.cu:4067-4077)
// would write; moe_route.run() makes the same calls from Python.
//
// Build (done by moe_route.build): g++ -O2 -std=c++17 moe_step.cpp
//   -I include -I /opt/rocm/include -D__HIP_PLATFORM_AMD__ -L <lib dir> -lmoe_route
//   -L /opt/rocm/lib -lamdhip64
// Run: moe_step [T]   (prints "moe_step OK ..." and exits 0 on success)
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "moe_route.h"

#define HIP_OK(x)                                                                   \
  do {                                                                              \
    hipError_t e_ = (x);                                                            \
    if (e_ != hipSuccess) {                                                         \
      std::fprintf(stderr, "HIP error %d at %s:%d\n", (int)e_, __FILE__, __LINE__); \
      return 2;                                                                     \
    }                                                                               \
  } while (0)
#define CHECK_MOE(x)                                                                          \
  do {                                                                                     \
    int rc_ = (x);                                                                         \
    if (rc_ != MOE_OK) {                                                                   \
      std::fprintf(stderr, "libmoe_route error %d: %s\n", rc_, moe_last_error_string()); \
      return 3;                                                                            \
    }                                                                                      \
  } while (0)

static uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
static float from_bf16(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

int main(int argc, char** argv) {
  const int T = argc > 1 ? std::atoi(argv[1]) : 2048;
  const int H = 1024, E = 256, k = 8;
  if (T < 1) return 1;
  const long long ns = (long long)T * k;

  std::mt19937 gen(17);
  std::normal_distribution<float> nd(0.f, 1.f);
  std::vector<uint16_t> hx((size_t)T * H), hw((size_t)E * H);
  std::vector<float> hb(E);
  for (auto& v : hx) v = to_bf16(nd(gen));
  for (auto& v : hw) v = to_bf16(0.02f * nd(gen));
  for (auto& v : hb) v = 0.1f * nd(gen);

  void *x, *w, *xg, *out, *ws_r, *ws_p;
  float *bias, *logits, *topk_w;
  int32_t *ids, *row_token, *pair_row, *offsets, *counts;
  const size_t nws_r = moe_route_workspace_bytes(T, H, E, MOE_DTYPE_BF16);
  const size_t nws_p = moe_permute_workspace_bytes(T, E, k);
  HIP_OK(hipMalloc(&x, hx.size() * 2));
  HIP_OK(hipMalloc(&w, hw.size() * 2));
  HIP_OK(hipMalloc(&bias, E * 4));
  HIP_OK(hipMalloc(&logits, (size_t)T * E * 4));
  HIP_OK(hipMalloc(&ids, ns * 4));
  HIP_OK(hipMalloc(&topk_w, ns * 4));
  HIP_OK(hipMalloc(&row_token, ns * 4));
  HIP_OK(hipMalloc(&pair_row, ns * 4));
  HIP_OK(hipMalloc(&offsets, (E + 1) * 4));
  HIP_OK(hipMalloc(&counts, E * 4));
  HIP_OK(hipMalloc(&xg, ns * H * 2));
  HIP_OK(hipMalloc(&out, (size_t)T * H * 2));
  HIP_OK(hipMalloc(&ws_r, nws_r > 0 ? nws_r : 256));
  HIP_OK(hipMalloc(&ws_p, nws_p));
  HIP_OK(hipMemcpy(x, hx.data(), hx.size() * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(w, hw.data(), hw.size() * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(bias, hb.data(), E * 4, hipMemcpyHostToDevice));
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));

  // DeepSeek-V3 routing: sigmoid + bias for selection, 8 groups keep 4, x2.5
  const moe_route_cfg cfg{MOE_SCORING_SIGMOID_GROUP, 1, 8, 4, 2.5f, 0.0f};
  CHECK_MOE(moe_route(x, w, MOE_DTYPE_BF16, bias, T, H, E, k, &cfg, logits, ids, topk_w, nullptr,
                   ws_r, nws_r, s));
  CHECK_MOE(moe_permute(x, MOE_DTYPE_BF16, ids, T, H, E, k, MOE_DTYPE_BF16, xg, nullptr, row_token,
                     pair_row, offsets, counts, ws_p, nws_p, s));
  // identity experts: the expert outputs are the gathered rows themselves
  CHECK_MOE(moe_combine(xg, MOE_DTYPE_BF16, pair_row, topk_w, nullptr, T, H, k, out, s));
  HIP_OK(hipStreamSynchronize(s));

  std::vector<int32_t> cid(ns), crt(ns), cpr(ns), coff(E + 1), ccnt(E);
  std::vector<float> cw(ns);
  std::vector<uint16_t> cxg((size_t)ns * H), cout((size_t)T * H);
  HIP_OK(hipMemcpy(cid.data(), ids, ns * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(cw.data(), topk_w, ns * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(crt.data(), row_token, ns * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(cpr.data(), pair_row, ns * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(coff.data(), offsets, (E + 1) * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(ccnt.data(), counts, E * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(cxg.data(), xg, cxg.size() * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(cout.data(), out, cout.size() * 2, hipMemcpyDeviceToHost));

  int bad = 0;
  auto expect = [&](bool ok, const char* what) {
    if (!ok && bad++ < 10) std::fprintf(stderr, "FAILED: %s\n", what);
  };
  long long total = 0;
  for (int e = 0; e < E; ++e) {
    expect(coff[e] == total, "offsets are the exclusive scan of counts");
    total += ccnt[e];
  }
  expect(total == ns && coff[E] == ns, "counts sum to T*k");
  std::vector<char> hit(ns, 0);
  for (long long p = 0; p < ns; ++p) {
    const int r = cpr[p];
    expect(r >= 0 && r < ns, "pair_row in range");
    if (r < 0 || r >= ns) continue;
    expect(!hit[r], "pair_row is a bijection");
    hit[r] = 1;
    expect(crt[r] == (int)(p / k), "row_token[pair_row[p]] = p / k");
    expect(r >= coff[cid[p]] && r < coff[cid[p] + 1], "row inside its expert segment");
  }
  for (int e = 0; e < E; ++e)
    for (int r = coff[e] + 1; r < coff[e + 1]; ++r)
      expect(crt[r] > crt[r - 1], "expert segments hold ascending tokens");
  for (long long r = 0; r < ns; ++r)
    expect(std::memcmp(&cxg[(size_t)r * H], &hx[(size_t)crt[r] * H], (size_t)H * 2) == 0,
           "gathered row equals x[row_token]");
  for (int t = 0; t < T; ++t) {
    float sw = 0.f;
    for (int j = 0; j < k; ++j) sw += cw[(size_t)t * k + j];
    expect(std::fabs(sw - 2.5f) < 1e-4f, "weights sum to route_scale 2.5");
    for (int h = 0; h < H; h += 37) {
      const float xv = from_bf16(hx[(size_t)t * H + h]);
      const float got = from_bf16(cout[(size_t)t * H + h]);
      const float want = xv * sw;
      expect(std::fabs(got - want) <= std::fabs(want) * 0.008f + 1e-6f,
             "identity experts: combine returns x * sum(w)");
    }
  }
  if (bad) {
    std::fprintf(stderr, "moe_step FAILED (%d checks)\n", bad);
    return 1;
  }
  std::printf("moe_step OK: T=%d H=%d E=%d k=%d through the C ABI (route, permute, combine)\n", T,
              H, E, k);
  return 0;
}
