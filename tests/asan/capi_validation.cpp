// Host-only driver for the C-ABI argument validation, built with
// AddressSanitizer on the host pass (tests/test_capi_asan.py).  Every call
// below must be rejected before anything is launched, so no GPU is needed.
#include <cstdio>
#include <cstring>

#include "moe_route.h"

static int failures = 0;
#define EXPECT(call, code)                                                             \
  do {                                                                                 \
    int rc_ = (call);                                                                  \
    if (rc_ != (code)) {                                                               \
      std::printf("FAIL %s: got %d want %d (%s)\n", #call, rc_, code,                  \
                  moe_last_error_string());                                            \
      ++failures;                                                                      \
    } else if (std::strlen(moe_last_error_string()) == 0 && (code) != 0) {             \
      std::printf("FAIL %s: empty error string\n", #call);                            \
      ++failures;                                                                      \
    }                                                                                  \
  } while (0)

int main() {
  void* fake = reinterpret_cast<void*>(0x10000);
  moe_route_cfg cfg{MOE_SCORING_SIGMOID_GROUP, 1, 8, 4, 2.5f, 0.0f};
  int32_t* ip = static_cast<int32_t*>(fake);
  float* fp = static_cast<float*>(fake);
  EXPECT(moe_route(fake, fake, 0, fp, 16, 100, 256, 8, &cfg, fp, ip, fp, nullptr, nullptr, 0, nullptr), MOE_ERR_UNSUPPORTED);
  EXPECT(moe_route(fake, fake, 0, fp, 16, 128, 12, 8, &cfg, fp, ip, fp, nullptr, nullptr, 0, nullptr), MOE_ERR_UNSUPPORTED);
  EXPECT(moe_route(fake, fake, 1, fp, 16, 128, 256, 8, &cfg, fp, ip, fp, nullptr, nullptr, 0, nullptr), MOE_ERR_WORKSPACE);
  EXPECT(moe_route(nullptr, fake, 0, fp, 16, 128, 256, 8, &cfg, fp, ip, fp, nullptr, nullptr, 0, nullptr), MOE_ERR_NULL_POINTER);
  EXPECT(moe_route(fake, fake, 0, fp, 16, 128, 256, 8, nullptr, fp, ip, fp, nullptr, nullptr, 0, nullptr), MOE_ERR_NULL_POINTER);
  cfg.n_group = 6;
  EXPECT(moe_topk(fp, nullptr, 4, 256, 8, &cfg, ip, fp, nullptr, nullptr), MOE_ERR_INVALID_ARG);
  cfg.n_group = 128;
  EXPECT(moe_topk(fp, nullptr, 4, 256, 8, &cfg, ip, fp, nullptr, nullptr), MOE_ERR_UNSUPPORTED);
  EXPECT(moe_permute(fake, 0, ip, 8, 256, 16, 9, 0, fake, nullptr, ip, ip, nullptr, nullptr, fake, 1 << 20, nullptr), MOE_ERR_INVALID_ARG);
  EXPECT(moe_permute(fake, 0, ip, 8, 192, 16, 2, 2, fake, fp, ip, ip, nullptr, nullptr, fake, 1 << 20, nullptr), MOE_ERR_UNSUPPORTED);
  EXPECT(moe_permute(fake, 0, ip, 8, 256, 16, 2, 0, fake, nullptr, ip, ip, nullptr, nullptr, fake, 8, nullptr), MOE_ERR_WORKSPACE);
  EXPECT(moe_combine(fake, 0, ip, fp, nullptr, 4, 4, 2, fake, nullptr), MOE_ERR_ALIGNMENT);
  EXPECT(moe_combine(nullptr, 0, nullptr, nullptr, nullptr, 0, 64, 2, nullptr, nullptr), MOE_OK);
  EXPECT(moe_offsets(ip, 2000, ip, nullptr), MOE_ERR_INVALID_ARG);
  EXPECT(moe_router_gemm(fake, fake, 4, 96, 8, fp, nullptr), MOE_ERR_UNSUPPORTED);
  EXPECT(moe_grouped_gemm(fake, fake, ip, 0, 64, 128, 256, nullptr, 0, fake, fake, 4096, nullptr), MOE_ERR_INVALID_ARG);
  EXPECT(moe_grouped_gemm(fake, fake, ip, 4, 64, 128, 100, nullptr, 0, fake, fake, 4096, nullptr), MOE_ERR_UNSUPPORTED);
  EXPECT(moe_grouped_gemm(fake, fake, ip, 4, 64, 128, 256, nullptr, 3, fake, fake, 4096, nullptr), MOE_ERR_NULL_POINTER);
  EXPECT(moe_grouped_gemm(fake, fake, ip, 4, 64, 128, 256, nullptr, 0, fake, fake, 8, nullptr), MOE_ERR_WORKSPACE);
  EXPECT(moe_grouped_swiglu(fake, fake, nullptr, ip, 4, 64, 128, 256, nullptr, 0, fake, fake, 4096, nullptr), MOE_ERR_NULL_POINTER);
  EXPECT(moe_grouped_gemm_rows(fake, nullptr, fake, ip, 4, 64, 128, 256, fake, fake, 4096, nullptr), MOE_ERR_NULL_POINTER);
  EXPECT(moe_grouped_swiglu_rows(fake, ip, fake, fake, ip, 4, 64, 128, 200, fake, fake, 4096, nullptr), MOE_ERR_UNSUPPORTED);
  const int8_t* q8 = (const int8_t*)fake;
  EXPECT(moe_grouped_gemm_i8(q8, fp, nullptr, q8, fp, ip, 4, 64, 128, 192, nullptr, nullptr, 0, fake, fake, 4096, nullptr), MOE_ERR_UNSUPPORTED);
  EXPECT(moe_grouped_swiglu_i8(q8, nullptr, nullptr, q8, fp, q8, fp, ip, 4, 64, 128, 256, nullptr, nullptr, 0, fake, fake, 4096, nullptr), MOE_ERR_NULL_POINTER);
  EXPECT(moe_quant_rows_i8(fake, 4, 256, 64, 1.0f, 0, nullptr, (int8_t*)fake, fp, nullptr), MOE_ERR_INVALID_ARG);
  EXPECT(moe_quant_rows_i8(fake, 6, 256, 16, 1.0f, 4, ip, (int8_t*)fake, fp, nullptr), MOE_ERR_INVALID_ARG);
  EXPECT(moe_quant_rows_i8(nullptr, 0, 256, 0, 1.0f, 0, nullptr, nullptr, nullptr, nullptr), MOE_OK);
  if (moe_grouped_gemm_workspace_bytes(64) != 512) ++failures;
  // C4 bf16: the fused GEMM + scoring kernel's fragment-major weight copy [256, 7168] bf16
  if (moe_route_workspace_bytes(32768, 7168, 256, MOE_DTYPE_BF16) != (size_t)256 * 7168 * 2) ++failures;
  // fp32 weights: [2E,H] bf16 hi/lo split + [T,2E] fp32 hi/lo partial logits
  if (moe_route_workspace_bytes(32768, 7168, 256, MOE_DTYPE_FP32) != (size_t)2 * 256 * 7168 * 2 + (size_t)32768 * 512 * 4) ++failures;
  if (moe_permute_workspace_bytes(32768, 256, 8) != (size_t)256 * 1024 * 4 + 1024) ++failures;
  // C2 (E = 8, bf16): the small-E GEMM + scoring kernel needs no route workspace; through
  // moe_route_permute it adds its 32-token histograms, 8 experts x 256 columns of int32
  if (moe_route_workspace_bytes(8192, 4096, 8, MOE_DTYPE_BF16) != 0) ++failures;
  if (moe_route_workspace_bytes(8192, 4096, 8, MOE_DTYPE_FP32) != 0) ++failures;
  if (moe_route_permute_workspace_bytes(8192, 4096, 8, 2, MOE_DTYPE_BF16) !=
      moe_permute_fp8_workspace_bytes(8192, 4096, 8, 2) + (size_t)8 * 256 * 4)
    ++failures;
  // route + permute in one call: the workspace and both stages' checks come first
  {
    moe_route_cfg rc{MOE_SCORING_SOFTMAX, 1, 1, 1, 1.0f, 0.0f};
    const size_t rp = moe_route_permute_workspace_bytes(16, 128, 8, 2, MOE_DTYPE_BF16);
    // route's workspace (rounded up to 256), the permute's, the fp8 scale stage
    // (16 tokens x 1 block of 128 fp32, rounded up to 256)
    if (rp != ((moe_route_workspace_bytes(16, 128, 8, MOE_DTYPE_BF16) + 255) / 256) * 256 +
                  moe_permute_workspace_bytes(16, 8, 2) + 256)
      ++failures;
    if (moe_permute_fp8_workspace_bytes(16, 128, 8, 2) != moe_permute_workspace_bytes(16, 8, 2) + 256)
      ++failures;
    EXPECT(moe_route_permute(fake, fake, 0, nullptr, 16, 128, 8, 2, &rc, fp, ip, fp, 0, fake, nullptr, ip, ip, ip, ip, nullptr, rp, nullptr), MOE_ERR_WORKSPACE);
    EXPECT(moe_route_permute(fake, fake, 0, nullptr, 16, 128, 8, 2, &rc, fp, ip, fp, 1, fake, nullptr, ip, ip, ip, ip, fake, rp, nullptr), MOE_ERR_UNSUPPORTED);
    EXPECT(moe_route_permute(fake, fake, 0, nullptr, 16, 128, 8, 2, &rc, fp, ip, fp, 0, fake, nullptr, nullptr, ip, ip, ip, fake, rp, nullptr), MOE_ERR_NULL_POINTER);
  }
  if (moe_version() != MOE_ROUTE_VERSION) ++failures;
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "OK", failures);
  return failures ? 1 : 0;
}
