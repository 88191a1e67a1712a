// Host-only driver of the C ABI's argument checks, for a build of the ABI
// layer with AddressSanitizer and UndefinedBehaviorSanitizer on the host side
// (tests/test_abi_sanitizers.py). Every call here is rejected, or found to
// have nothing to do, before the library touches the GPU: the same cases the
// ctypes tests of the ABI run, plus sizes at the ends of the int range, whose
// size checks and workspace sizes must neither overflow nor accept them.
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../include/cuda_llm_abi.h"

namespace {

int failures = 0;

void expect(bool ok, const char* what) {
  if (!ok) {
    std::printf("FAIL: %s (last error: %s)\n", what, ca_last_error());
    ++failures;
  }
}

bool error_mentions(const char* s) { return std::strstr(ca_last_error(), s) != nullptr; }

}  // namespace

int main() {
  void* const P = reinterpret_cast<void*>(16);  // aligned, never dereferenced
  const int32_t* const PI = reinterpret_cast<const int32_t*>(16);
  const uint8_t* const PB = reinterpret_cast<const uint8_t*>(16);
  float* const PF = reinterpret_cast<float*>(16);
  void* const odd = reinterpret_cast<void*>(18);

  expect(ca_version() && std::strlen(ca_version()) > 0, "version string");

  // prefill
  expect(ca_flash_attention_fwd(CA_BF16, P, P, P, P, 1, 4, 4, 64, 96, 0.1f, 0, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("head_dim"),
         "prefill head_dim");
  expect(ca_flash_attention_fwd((ca_dtype)7, P, P, P, P, 1, 4, 4, 64, 64, 0.1f, 0, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("dtype"),
         "prefill dtype");
  expect(ca_flash_attention_fwd(CA_BF16, P, P, P, P, 1, 6, 4, 64, 64, 0.1f, 0, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("multiple"),
         "prefill heads");
  expect(ca_flash_attention_fwd(CA_BF16, odd, P, P, P, 1, 4, 4, 64, 64, 0.1f, 0, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("aligned"),
         "prefill alignment");
  expect(ca_flash_attention_fwd(CA_BF16, nullptr, P, P, P, 1, 4, 4, 64, 64, 0.1f, 0, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("null"),
         "prefill null");
  expect(ca_flash_attention_fwd(CA_BF16, P, P, P, P, -1, 4, 4, 64, 64, 0.1f, 0, nullptr) ==
             CA_INVALID_ARGUMENT,
         "prefill negative");
  expect(ca_flash_attention_fwd(CA_BF16, P, P, P, P, 0, 4, 4, 64, 64, 0.1f, 0, nullptr) == CA_OK,
         "prefill empty");
  // 2^30 x 2^30 x 2^20 x 128 elements: a signed 64-bit product would wrap
  expect(ca_flash_attention_fwd(CA_BF16, P, P, P, P, 1 << 30, 1 << 30, 1 << 30, 1 << 20, 128, 0.1f,
                                1, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("too large"),
         "prefill element count overflow");
  expect(ca_flash_attention_fwd(CA_F32, P, P, P, P, 1, 1, 1, INT_MAX, 128, 0.1f, 1, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("seq_len"),
         "prefill slice size");
  expect(ca_flash_attention_fwd_lse(CA_BF16, P, P, P, P, nullptr, 1, 4, 4, 64, 64, 0.1f, 0,
                                    nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("lse"),
         "prefill lse null");

  // backward
  const size_t bws = ca_flash_attention_bwd_workspace_bytes(1, 4, 64);
  expect(bws == 1 * 4 * 64 * 8, "backward workspace size");
  (void)ca_flash_attention_bwd_workspace_bytes(INT_MAX, INT_MAX, INT_MAX);
  expect(ca_flash_attention_bwd((ca_dtype)7, P, P, P, P, P, PF, P, P, P, 1, 4, 2, 64, 64, 0.1f, 1,
                                P, bws, nullptr) == CA_INVALID_ARGUMENT,
         "backward dtype");
  expect(ca_flash_attention_bwd(CA_BF16, P, P, P, P, P, PF, P, P, P, 1, 4, 2, 64, 64, 0.1f, 1, P,
                                16, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("workspace"),
         "backward workspace");
  expect(ca_flash_attention_bwd(CA_BF16, P, P, P, P, P, nullptr, P, P, P, 1, 4, 2, 64, 64, 0.1f, 1,
                                P, bws, nullptr) == CA_INVALID_ARGUMENT,
         "backward lse null");
  expect(ca_flash_attention_bwd(CA_BF16, P, P, P, P, P, PF, P, P, P, 1 << 30, 1 << 30, 1 << 30,
                                1 << 20, 128, 0.1f, 1, P, SIZE_MAX, nullptr) == CA_INVALID_ARGUMENT,
         "backward element count overflow");

  // RoPE prefill
  const size_t rws = ca_rope_workspace_bytes(CA_BF16, 2, 8, 2, 100, 64);
  expect(rws == 2 * 2 * 100 * 64 * 2, "rope workspace size");
  (void)ca_rope_workspace_bytes(CA_F32, INT_MAX, INT_MAX, INT_MAX, INT_MAX, 128);
  expect(ca_fused_rope_flash_attention(CA_BF16, P, P, P, PF, PF, P, 2, 8, 2, 100, 64, 0.1f, 1, P,
                                       rws - 1, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("workspace"),
         "rope workspace");
  expect(ca_fused_rope_flash_attention(CA_BF16, P, P, P, nullptr, PF, P, 2, 8, 2, 100, 64, 0.1f, 1,
                                       P, rws, nullptr) == CA_INVALID_ARGUMENT,
         "rope table null");

  // contiguous and paged decode
  expect(ca_decode_workspace_bytes(0, 8, 128, 100) == 0, "decode workspace empty");
  (void)ca_decode_workspace_bytes(INT_MAX, INT_MAX, 128, INT_MAX);
  expect(ca_paged_attention(CA_BF16, P, P, P, PI, PI, P, 2, 8, 2, 128, 4, 8, 10, 0.1f, nullptr, 0,
                            nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("page_size"),
         "paged page size");
  expect(ca_paged_attention(CA_BF16, P, P, P, PI, PI, P, 2, 8, 2, 128, 200, 16, 10, 0.1f, nullptr,
                            0, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("workspace"),
         "paged workspace");
  expect(ca_paged_attention(CA_BF16, P, P, P, PI, PI, P, 2, 8, 2, 128, INT_MAX, 16, 10, 0.1f, P,
                            SIZE_MAX, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("too wide"),
         "paged table width overflow");
  expect(ca_fp8_paged_attention((ca_dtype)7, P, PB, PB, nullptr, nullptr, 1, PI, PI, P, 2, 8, 2,
                                128, 4, 16, 10, 0.1f, nullptr, 0, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("dtype"),
         "fp8 paged dtype");
  expect(ca_fp8_paged_attention(CA_F32, P, PB, PB, nullptr, nullptr, 1, PI, PI, P, 2, 8, 2, 128, 4,
                                16, 10, 0.1f, nullptr, 0, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("scale"),
         "fp8 paged scales");

  // KV-cache append
  expect(ca_paged_kv_append(CA_BF16, 5, P, P, P, P, nullptr, nullptr, 0, PI, PI, nullptr, 2, 2,
                            128, 4, 8, 100, nullptr) == CA_INVALID_ARGUMENT,
         "append cache kind");
  expect(ca_paged_kv_append(CA_BF16, 1, P, P, P, P, nullptr, nullptr, 0, PI, PI, nullptr, 2, 2,
                            128, 4, 8, 100, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("k_scale"),
         "append fp8 scales");
  expect(ca_paged_kv_append(CA_BF16, 0, P, P, P, P, nullptr, nullptr, 0, PI, PI, nullptr, 2, 2,
                            128, 0, 8, 100, nullptr) == CA_OK,
         "append nothing");
  expect(ca_paged_kv_append(CA_BF16, 0, P, P, P, P, nullptr, nullptr, 0, PI, PI, nullptr, INT_MAX,
                            INT_MAX, 128, INT_MAX, 8, 100, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("too large"),
         "append element count overflow");

  // MXFP8
  const size_t mws = ca_mx_workspace_bytes(CA_SCALE_E8M0, 1, 2, 64, 128);
  expect(mws == 1 * 2 * 64 * 128 * 2, "mx workspace size");
  expect(ca_mx_workspace_bytes((ca_scale_kind)7, 1, 2, 64, 128) == 0, "mx workspace kind");
  (void)ca_mx_workspace_bytes(CA_SCALE_F32, INT_MAX, INT_MAX, INT_MAX, 128);
  expect(ca_fused_microscaled_attention(CA_BF16, PB, P, PB, P, PB, P, CA_SCALE_E8M0, P, 1, 2, 64,
                                        64, 0.1f, 1, P, mws, nullptr) == CA_INVALID_ARGUMENT,
         "mx head_dim");
  expect(ca_fused_microscaled_attention(CA_BF16, PB, P, PB, P, PB, P, (ca_scale_kind)5, P, 1, 2,
                                        64, 128, 0.1f, 1, P, mws, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("scale kind"),
         "mx scale kind");
  expect(ca_fused_microscaled_attention(CA_BF16, PB, P, PB, P, PB, P, CA_SCALE_E8M0, P, 1, 2, 64,
                                        128, 0.1f, 1, P, mws - 1, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("workspace"),
         "mx workspace");

  // measurement helper and the block-table check
  expect(ca_stream_read(P, 1000, P, nullptr) == CA_INVALID_ARGUMENT, "stream read size");
  expect(ca_stream_read(P, 0, nullptr, nullptr) == CA_OK, "stream read empty");
  expect(ca_check_block_tables(PI, PI, -1, 4, 10, 16, nullptr) == CA_INVALID_ARGUMENT,
         "block tables negative");
  expect(ca_check_block_tables(nullptr, nullptr, 2, 4, 10, 16, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("null"),
         "block tables null");
  // a table of 10^6 x 10^6 entries: rejected (null) or failing at the stream
  // wait (no GPU here) with a status, never an allocation of its size
  expect(ca_check_block_tables(nullptr, nullptr, 1000000, 1000000, 10, 16, nullptr) ==
             CA_INVALID_ARGUMENT,
         "block tables huge, null");
  expect(ca_check_block_tables(PI, PI, 1000000, 1000000, 10, 16, nullptr) != CA_OK,
         "block tables huge, no device");
  // the float MX scale check
  expect(ca_check_mx_scales(PF, PF, PF, -1, 2, 8, 128, nullptr) == CA_INVALID_ARGUMENT,
         "mx scales negative");
  expect(ca_check_mx_scales(PF, PF, PF, 1, 2, 8, 100, nullptr) == CA_INVALID_ARGUMENT,
         "mx scales head_dim");
  expect(ca_check_mx_scales(nullptr, PF, PF, 1, 2, 8, 128, nullptr) == CA_INVALID_ARGUMENT &&
             error_mentions("null"),
         "mx scales null");
  expect(ca_check_mx_scales(reinterpret_cast<const float*>(odd), PF, PF, 1, 2, 8, 128, nullptr) ==
                 CA_INVALID_ARGUMENT && error_mentions("aligned"),
         "mx scales aligned");
  expect(ca_check_mx_scales(nullptr, nullptr, nullptr, 1, 2, 0, 128, nullptr) == CA_OK,
         "mx scales empty");

  std::printf(failures ? "abi checks: %d failed\n" : "abi checks: all passed\n", failures);
  return failures ? 1 : 0;
}
