// Host-side AddressSanitizer run of the C-ABI's argument validation.
//
// Linked against a host-only build of the library (device code left out,
// host code instrumented), it calls every entry point with arguments each
// check must reject, so ASan watches the validation paths for out-of-bounds
// or use-after-free accesses.  No call reaches a kernel launch: pointers are
// never dereferenced and every call fails validation.  Exit status 0 when
// every call returns the expected status code.
#include <cstdint>
#include <cstdio>
#include <initializer_list>

#include "mx_kernels.h"

static int failures = 0;
#define EXPECT(call, code)                                                                      \
  do {                                                                                          \
    const long long got_ = (long long)(call);                                                   \
    if (got_ != (long long)(code)) {                                                            \
      std::fprintf(stderr, "%s:%d: %s returned %lld, expected %lld\n", __FILE__, __LINE__, #call, \
                   got_, (long long)(code));                                                    \
      ++failures;                                                                               \
    }                                                                                           \
  } while (0)

int main() {
  void* P = reinterpret_cast<void*>(0x10000);  // 16-byte aligned, never dereferenced
  void* U = reinterpret_cast<void*>(0x10008);  // misaligned
  float* F = static_cast<float*>(P);
  void* s_in = reinterpret_cast<void*>(0x100000);
  void* s_out = reinterpret_cast<void*>(0x100000 + 256);

  for (int c = 1; c >= -9; --c)
    if (mx_strerror(c) == nullptr) ++failures;
  if (mx_version() == nullptr) ++failures;

  // bf16 GEMM and its batched form
  EXPECT(mx_gemm_bf16(nullptr, P, P, 64, 64, 64, 64, 64, 64, nullptr), MX_ERR_NULL);
  EXPECT(mx_gemm_bf16(P, P, P, 0, 64, 64, 64, 64, 64, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_gemm_bf16(P, P, P, 64, 64, 60, 60, 64, 64, nullptr), MX_ERR_ALIGN);
  EXPECT(mx_gemm_bf16(U, P, P, 64, 64, 64, 64, 64, 64, nullptr), MX_ERR_ALIGN);
  EXPECT(mx_gemm_bf16(P, P, P, 64, 64, 64, 20971520, 64, 64, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_gemm_bf16_batched(nullptr, P, P, 2, 64, 64, 64, 64, 64, 64, 4096, 4096, 4096, nullptr), MX_ERR_NULL);
  EXPECT(mx_gemm_bf16_batched(P, P, P, 70000, 64, 64, 64, 64, 64, 64, 0, 0, 0, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_gemm_bf16_batched(P, P, P, 2, 64, 64, 64, 64, 64, 64, 4, 0, 0, nullptr), MX_ERR_ALIGN);
  EXPECT(mx_gemm_bf16_batched(P, P, P, 2, 64, 64, 64, 64, 20971520, 64, 0, 0, 0, nullptr), MX_ERR_SHAPE);

  // fp8 block-scaled GEMM and the activation quantiser
  EXPECT(mx_gemm_fp8_bs(P, F, P, F, nullptr, 64, 64, 128, nullptr), MX_ERR_NULL);
  EXPECT(mx_gemm_fp8_bs(P, F, P, F, P, 64, 64, 100, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_gemm_fp8_bs(P, F, P, F, P, 64, 40, 128, nullptr), MX_ERR_ALIGN);
  EXPECT(mx_gemm_fp8_bs(P, F, P, F, P, (1 << 30) + 1, 16, 128, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_quant_fp8_act(nullptr, P, F, 4, 128, 128, 0, nullptr), MX_ERR_NULL);
  EXPECT(mx_quant_fp8_act(P, P, F, 4, 96, 96, 0, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_quant_fp8_act(P, P, F, 4, 128, 132, 0, nullptr), MX_ERR_ALIGN);
  EXPECT(mx_quant_fp8_act(P, P, F, 4, 128, 128, 2, nullptr), MX_ERR_DTYPE);

  // attention forward (GQA, MLA prefill)
  EXPECT(mx_gqa_fwd(nullptr, P, P, P, 1, 4, 2, 16, 64, 0.125f, 1, 0, nullptr), MX_ERR_NULL);
  EXPECT(mx_gqa_fwd(P, P, P, P, 1, 4, 3, 16, 64, 0.125f, 1, 0, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_gqa_fwd(P, P, P, P, 1, 4, 2, 16, 64, 0.125f, 1, 7, nullptr), MX_ERR_DTYPE);
  EXPECT(mx_gqa_fwd_tile(P, P, P, P, 1, 32, 8, 256, 128, 0.088f, 1, 0, 64, 32, 32, nullptr), MX_ERR_UNSUPPORTED);
  EXPECT(mx_gqa_fwd_tile(P, P, P, P, 1, 32, 8, 256, 128, 0.088f, 1, 0, 16, 64, 32, nullptr), MX_ERR_UNSUPPORTED);
  EXPECT(mx_gqa_fwd_tile_check(32, 8, 128, 128, 64, 64), MX_OK);
  EXPECT(mx_gqa_fwd_tile_check(32, 7, 128, 128, 64, 64), MX_ERR_SHAPE);
  EXPECT(mx_gqa_fwd_tile_info(32, 8, 128, 0, 1, 64, 64, 32, nullptr, nullptr), MX_ERR_NULL);
  EXPECT(mx_mla_prefill_fwd(P, P, P, P, 1, 4, 16, 160, 128, 0.07f, 0, 0, nullptr), MX_ERR_UNSUPPORTED);
  EXPECT(mx_mla_prefill_fwd(P, P, P, P, 1, 4, 16, 192, 128, 0.0f, 0, 0, nullptr), MX_ERR_SHAPE);

  // MLA decode, its allocation-free form and the absorbed step
  const size_t ws = mx_mla_decode_workspace(32, 128, 4096, 512);
  if (ws == 0 || mx_mla_decode_workspace(1, 16, 64, 512) != 0) ++failures;
  if (mx_mla_decode_splits(32, 128, 4096) < 1) ++failures;
  EXPECT(mx_mla_decode(P, P, P, 32, 128, 4096, 512, 64, 0.07f, nullptr, 0, nullptr), MX_ERR_WORKSPACE);
  EXPECT(mx_mla_decode(P, P, P, 1, 16, 64, 256, 64, 0.07f, nullptr, 0, nullptr), MX_ERR_UNSUPPORTED);
  EXPECT(mx_mla_decode(nullptr, P, P, 1, 16, 64, 512, 64, 0.07f, nullptr, 0, nullptr), MX_ERR_NULL);
  EXPECT(mx_mla_decode_noalloc(nullptr, P, P, 1, 16, 64, 512, 64, 0.07f, nullptr), MX_ERR_NULL);
  EXPECT(mx_mla_decode_noalloc(P, P, P, 1, 16, 64, 256, 64, 0.07f, nullptr), MX_ERR_UNSUPPORTED);
  const size_t wsa = mx_mla_decode_absorbed_workspace(32, 128, 4096);
  EXPECT(mx_mla_decode_absorbed(nullptr, P, P, P, P, P, 32, 128, 4096, 128, 128, 0.07f, P, wsa, nullptr), MX_ERR_NULL);
  EXPECT(mx_mla_decode_absorbed(P, P, P, P, P, P, 32, 128, 4096, 128, 128, 0.07f, P, wsa - 1, nullptr),
         MX_ERR_WORKSPACE);
  EXPECT(mx_mla_decode_absorbed(P, P, P, P, U, P, 32, 128, 4096, 128, 128, 0.07f, P, wsa, nullptr), MX_ERR_ALIGN);
  EXPECT(mx_mla_decode_absorbed(P, P, U, P, P, P, 32, 128, 4096, 128, 128, 0.07f, P, wsa, nullptr), MX_ERR_ALIGN);

  // linear-attention decode (GDN, KDA)
  EXPECT(mx_gdn_decode(nullptr, P, P, F, F, F, F, P, 2, 2, 4, 64, 64, 0, nullptr), MX_ERR_NULL);
  EXPECT(mx_gdn_decode(P, P, P, F, F, F, F, P, 2, 3, 4, 64, 64, 0, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_gdn_decode(P, P, P, F, F, static_cast<float*>(s_in), static_cast<float*>(s_out), P, 2, 2, 4, 64, 64, 0,
                       nullptr),
         MX_ERR_ALIAS);
  EXPECT(mx_kda_decode(nullptr, P, P, P, P, F, F, P, 2, 4, 64, 64, 0, nullptr), MX_ERR_NULL);
  EXPECT(mx_kda_decode(P, P, P, P, P, F, F, P, 2, 4, 96, 64, 0, nullptr), MX_ERR_SHAPE);
  EXPECT(mx_kda_decode(P, P, P, P, P, static_cast<float*>(s_in), static_cast<float*>(s_out), P, 2, 4, 64, 64, 0,
                       nullptr),
         MX_ERR_ALIAS);
  for (int d : {64, 128, 256, 512})
    if (mx_gdn_decode_block_v(64, 32, d, d) <= 0) ++failures;

  std::printf("capi_validation: %d failure(s)\n", failures);
  return failures == 0 ? 0 : 1;
}
