// Host-side checks of the C ABI (include/aoakv.h) for an AddressSanitizer
// build: tests/test_capi_asan.py compiles the library's sources with
// -fsanitize=address on the host pass (the device code, built as usual,
// never runs here), links this driver and runs it on the CPU.  Every call either fails validation before
// any HIP call or, with well-formed shapes, walks the host path to the
// launch (workspace layout, selection sizing, argument packing), which then
// fails for want of a device or of device code: AOAKV_ERR_HIP is accepted
// there.  Device pointers are fake addresses the host never dereferences.
// Exit status 0 when every expectation held; a sanitizer report aborts.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "../include/aoakv.h"

namespace {

int g_failures = 0;

void expect(bool ok, const char* what, int line) {
  if (!ok) {
    std::fprintf(stderr, "FAILED line %d: %s (last error: %s)\n", line, what, aoakv_last_error());
    ++g_failures;
  }
}
#define EXPECT(cond) expect((cond), #cond, __LINE__)

// a status from a call whose arguments are valid: the host path ran to the
// launch, which may fail without a GPU
bool launched_or_hip(int rc) { return rc == AOAKV_OK || rc == AOAKV_ERR_HIP; }

template <typename T = void>
T* fake(uintptr_t a) {
  return reinterpret_cast<T*>(a << 12);
}

void sizes() {
  // the layout grows with every dimension and always holds the control words
  size_t prev = 0;
  for (uint32_t sel : {1u, 8u, 128u, 129u, 1024u, 8192u}) {
    const size_t n = aoakv_decode_workspace_size(1, 32, 32, 128, sel);
    EXPECT(n >= AOAKV_WORKSPACE_CTL_BYTES && n >= prev && n % 256u == 0u);
    prev = n;
  }
  EXPECT(aoakv_decode_workspace_size(16, 32, 8, 128, 128) >
         aoakv_decode_workspace_size(1, 32, 8, 128, 128));
  const size_t d = aoakv_decode_workspace_size(2, 32, 8, 128, 128);
  const size_t l = aoakv_layer_workspace_size(2, 32, 8, 128, 128, 2048);
  EXPECT(l >= d + 2u * 8u * 2048u * 4u);
  // the largest shapes the entry points accept do not overflow size_t
  EXPECT(aoakv_layer_workspace_size(65535, 64, 8, 256, 8192, 16384) > (size_t)1 << 32);
}

void validation() {
  const int32_t* nul = nullptr;
  // null pointers, bad shapes and flags are refused before any HIP call,
  // each with a message
  int rc = aoakv_estimate_attn_score(nullptr, fake<float>(1), 64, fake(2), nul, nul, nul, nul, nul,
                                     nullptr, 1, 64, 32, 32, 128, 16, 1, 1, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID && std::strlen(aoakv_last_error()) > 0);
  rc = aoakv_estimate_attn_score(fake(1), fake<float>(2), 64, fake(3), fake<int32_t>(4),
                                 fake<int32_t>(5), fake<int32_t>(6), fake<int32_t>(7),
                                 fake<int32_t>(8), fake(9), 1, 64, 32, 32, 96, 16, 1, 1, nullptr);
  EXPECT(rc == AOAKV_ERR_UNSUPPORTED || rc == AOAKV_ERR_INVALID);
  rc = aoakv_topk_filtering(fake<float>(1), 64, fake<int32_t>(2), fake<int32_t>(3),
                            fake<int32_t>(4), 1024, nul, fake<int32_t>(5), 64, 1, 32, 16, 1u << 20,
                            nullptr, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID);
  rc = aoakv_topk_filtering(fake<float>(1), 0, fake<int32_t>(2), fake<int32_t>(3),
                            fake<int32_t>(4), 1024, nul, fake<int32_t>(5), 64, 1, 32, 16, 2,
                            nullptr, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID);
  // a workspace too small for the call
  rc = aoakv_decode_sparse_attn(fake(1), fake(2), fake(3), fake<int32_t>(4), fake<int32_t>(5),
                                fake<int32_t>(6), fake<int32_t>(7), 128, 2048, nul, fake(8), 16,
                                1, 2048, 32, 32, 128, 16, 1, 0, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID && std::strstr(aoakv_last_error(), "workspace") != nullptr);
  // group sizes the kernels do not take, head counts that do not divide
  rc = aoakv_decode_sparse_attn(fake(1), fake(2), fake(3), fake<int32_t>(4), fake<int32_t>(5),
                                fake<int32_t>(6), nul, 0, 2048, nul, fake(8), 1u << 30, 1, 2048,
                                24, 8, 128, 16, 1, 0, nullptr);
  EXPECT(rc != AOAKV_OK);
  rc = aoakv_decode_sparse_attn(fake(1), fake(2), fake(3), fake<int32_t>(4), fake<int32_t>(5),
                                fake<int32_t>(6), nul, 0, 2048, nul, fake(8), 1u << 30, 1, 2048,
                                30, 8, 128, 16, 1, 0, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID);
  // the no-allocation entry point: single launch and oversized calls
  rc = aoakv_sparse_decode_layer_noalloc(fake(1), fake(2), fake(3), fake<int32_t>(4),
                                         fake<int32_t>(5), fake<int32_t>(6), fake(7),
                                         fake<int32_t>(8), fake<int32_t>(9), fake(10),
                                         fake<float>(11), 16384, fake<int32_t>(12), 8192, 131072,
                                         nul, 1, 16384, 32, 8, 128, 16, 1,
                                         AOAKV_FLAG_VALUE_AWARE, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID && std::strstr(aoakv_last_error(), "scratch") != nullptr);
  uint32_t bits = 7u;
  rc = aoakv_noalloc_error(nullptr, 0, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID && bits == 7u);
  // prefill / append / rope shape checks
  rc = aoakv_prefill_with_paged_kv_cache(fake(1), fake(2), fake(3), fake<int32_t>(4), 10, 17,
                                         100, 1, 32, 32, 128, 16, 1, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID);  // last page length > page size
  rc = aoakv_append_kv_cache_prefill(fake(1), fake(2), 0, fake(3), fake<int32_t>(4), 1, 1,
                                     fake(5), fake<int32_t>(6), fake(7), fake(8), 32, 128, 16, 1,
                                     nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID || launched_or_hip(rc));  // zero tokens: refused or a no-op
  rc = aoakv_apply_rope_in_place(fake(1), fake(2), 4, 0, 32, 32, 100, 1.0f, 1e4f, nullptr);
  EXPECT(rc != AOAKV_OK);
  // messages stay within the library's buffer
  rc = aoakv_workspace_init(nullptr, 0, nullptr);
  EXPECT(rc == AOAKV_ERR_INVALID && std::strlen(aoakv_last_error()) < 512);
}

void host_paths() {
  // well-formed calls: every host step to the launch (ERR_HIP without a GPU)
  const int32_t* nul = nullptr;
  const uint32_t B = 3, Hq = 32, Hkv = 8, P = 2048;
  for (uint32_t layout : {0u, 1u}) {
    for (uint32_t flags : {AOAKV_FLAG_VALUE_AWARE | AOAKV_FLAG_FIXED,
                           AOAKV_FLAG_VALUE_AWARE | AOAKV_FLAG_FIXED | AOAKV_FLAG_SINGLE_LAUNCH,
                           AOAKV_FLAG_QUEST_KERNEL | AOAKV_FLAG_SINGLE_LAUNCH,
                           AOAKV_FLAG_VALUE_AWARE | AOAKV_FLAG_GROUPED_DECODE}) {
      const size_t ws = aoakv_layer_workspace_size(B, Hq, Hkv, 128, 128, P);
      int rc = aoakv_sparse_decode_layer(fake(1), fake(2), fake(3), fake<int32_t>(4),
                                         fake<int32_t>(5), fake<int32_t>(6), fake(7),
                                         fake<int32_t>(8), fake<int32_t>(9), fake(10),
                                         fake<float>(11), P, fake<int32_t>(12), 128, 2048, nul,
                                         fake(13), ws, B, P, Hq, Hkv, 128, 16, layout, flags,
                                         nullptr);
      EXPECT(launched_or_hip(rc));
      rc = aoakv_decode_sparse_attn(fake(1), fake(2), fake(3), fake<int32_t>(4),
                                    fake<int32_t>(5), fake<int32_t>(6), fake<int32_t>(7), 128,
                                    2048, fake<int32_t>(8), fake(9), ws, B, P, Hq, Hkv, 128, 16,
                                    layout, flags & (AOAKV_FLAG_QUEST_KERNEL |
                                                     AOAKV_FLAG_GROUPED_DECODE), nullptr);
      EXPECT(launched_or_hip(rc));
    }
    // more workgroups than one launch's 32-bit work-item count holds
    // (4,096 x 16 x 256 decode items): the two launches run instead
    {
      const uint32_t Bb = 4096, Hb = 16, Pb = 2048, Kb = 2047;
      const size_t wsb = aoakv_layer_workspace_size(Bb, Hb, Hb, 128, Kb, Pb);
      EXPECT(wsb / 4u > ((size_t)1 << 32));
      int rc = aoakv_sparse_decode_layer(
          fake(1), fake(2), fake(3), fake<int32_t>(4), fake<int32_t>(5), fake<int32_t>(6),
          fake(7), fake<int32_t>(8), fake<int32_t>(9), fake(10), fake<float>(11), Pb,
          fake<int32_t>(12), Kb, Kb * 16u, nul, fake(13), wsb, Bb, Pb, Hb, Hb, 128, 16, layout,
          AOAKV_FLAG_VALUE_AWARE | AOAKV_FLAG_FIXED | AOAKV_FLAG_SINGLE_LAUNCH, nullptr);
      EXPECT(launched_or_hip(rc));
    }
    // the generic shapes: any number of pages (12,500 chunks of 8 here)
    int rc = aoakv_decode_sparse_attn(fake(1), fake(2), fake(3), fake<int32_t>(4),
                                      fake<int32_t>(5), fake<int32_t>(6), nul, 0, 0, nul,
                                      fake(7), aoakv_decode_workspace_size(1, 8, 2, 64, 100000),
                                      1, 100000, 8, 2, 64, 1, layout, 0, nullptr);
    EXPECT(launched_or_hip(rc));
    rc = aoakv_decode_sparse_attn(fake(1), fake(2), fake(3), fake<int32_t>(4), fake<int32_t>(5),
                                  fake<int32_t>(6), nul, 0, 0, nul, fake(7),
                                  AOAKV_WORKSPACE_CTL_BYTES, 1, 100000, 8, 2, 64, 1, layout, 0,
                                  nullptr);
    EXPECT(rc == AOAKV_ERR_INVALID);  // the partials do not fit
    rc = aoakv_estimate_topk(fake(1), fake(2), fake<int32_t>(3), fake<int32_t>(4),
                             fake<int32_t>(5), fake<int32_t>(6), fake<int32_t>(7), fake(8),
                             fake<float>(9), P, fake<int32_t>(10), 128, 2048, nul, fake(11),
                             aoakv_decode_workspace_size(B, Hq, Hkv, 128, 128), B, P, Hq, Hkv,
                             128, 16, layout, AOAKV_FLAG_VALUE_AWARE | AOAKV_FLAG_FIXED, nullptr);
    EXPECT(launched_or_hip(rc));
    rc = aoakv_topk_filtering(fake<float>(1), P, fake<int32_t>(2), fake<int32_t>(3),
                              fake<int32_t>(4), 2048, nul, fake<int32_t>(5), 128, B, Hkv, 16,
                              AOAKV_FLAG_FIXED, fake<uint32_t>(6), nullptr);
    EXPECT(launched_or_hip(rc));
    rc = aoakv_prefill_with_paged_kv_cache(fake(1), fake(2), fake(3), fake<int32_t>(4), 512, 16,
                                           8192, 1, 32, 8, 128, 16, layout, nullptr);
    EXPECT(launched_or_hip(rc));
  }
}

}  // namespace

int main() {
  EXPECT(std::strlen(aoakv_version()) > 0);
  sizes();
  validation();
  host_paths();
  std::printf("capi_asan_driver: %d failures\n", g_failures);
  return g_failures == 0 ? 0 : 1;
}
