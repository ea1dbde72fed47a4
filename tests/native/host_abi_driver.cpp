// Host-side driver of libpal_hip.so's C ABI and page-pool allocator, built
// with -fsanitize=address,undefined by tests/test_native_sanitizers.py and
// run on the CPU.  The kernel launchers live in the .hip sources; here they
// are replaced by stand-ins that report "no device", so every host path
// (argument validation, workspace layout, the allocator and its compaction
// plans, the error strings) runs under the sanitizers without a GPU.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <set>
#include <vector>

#include "pal_hip.h"
#include "pal_hip_internal.h"

namespace pal {
hipError_t launch_fill_kv_pages(const FillParams&, hipStream_t) { return hipErrorNoDevice; }
hipError_t decode_resident_workers(int, int, int, bool, bool, bool, int* workers) {
  *workers = 1024;
  return hipSuccess;
}
int64_t decode_virtual_workers(int64_t resident, int64_t max_blocks, int partition_size) {
  if (partition_size > 0) return resident + (max_blocks + partition_size / 16 - 1) / (partition_size / 16);
  return resident + 1;
}
hipError_t launch_decode(const DecodeParams&, int, int, int, hipStream_t) { return hipErrorNoDevice; }
bool fused_shares_cu(int head_dim) { return head_dim <= 128; }
hipError_t launch_fused(const DecodeParams&, const PrefillParams&, int, int, int, hipStream_t) {
  return hipErrorNoDevice;
}
int prefill_tokens_per_tile(int group) { return 128 / (group < 16 ? group : 16); }
hipError_t launch_prefill(const PrefillParams&, int, int, int, hipStream_t) { return hipErrorNoDevice; }
hipError_t launch_copy_pages(const PageCopyParams&, hipStream_t) { return hipErrorNoDevice; }
hipError_t launch_remap_pages(uint32_t*, int64_t, const uint32_t*, int64_t, hipStream_t) { return hipErrorNoDevice; }
hipError_t scratch_buffer(void** ptr) {
  *ptr = nullptr;
  return hipErrorNoDevice;
}
hipError_t decode_debug_flags(uint32_t* out, bool) { *out = 0; return hipSuccess; }
hipError_t prefill_debug_flags(uint32_t* out, bool) { *out = 0; return hipSuccess; }
hipError_t fill_debug_flags(uint32_t* out, bool) { *out = 0; return hipSuccess; }
}  // namespace pal

static int g_fail = 0;
#define EXPECT(cond)                                                            \
  do {                                                                          \
    if (!(cond)) {                                                              \
      std::fprintf(stderr, "FAILED %s:%d: %s (last error: %s)\n", __FILE__, __LINE__, #cond, pal_last_error()); \
      ++g_fail;                                                                 \
    }                                                                           \
  } while (0)

int main() {
  // layout helpers
  int64_t ks[5], vs[4];
  EXPECT(pal_get_k_cache_shape(10, 4, 128, 16, PAL_DTYPE_BFLOAT16, ks) == PAL_OK && ks[2] == 16 && ks[4] == 8);
  EXPECT(pal_get_k_cache_shape(10, 4, 128, 16, PAL_DTYPE_FP8_E4M3, ks) == PAL_OK && ks[2] == 8 && ks[4] == 16);
  EXPECT(pal_get_v_cache_shape(10, 4, 128, 16, PAL_DTYPE_FLOAT16, vs) == PAL_OK && vs[3] == 16);
  EXPECT(pal_get_k_cache_stripe_size(9) == PAL_ERR_INVALID_ARGUMENT && std::strstr(pal_last_error(), "dtype"));
  EXPECT(pal_get_optimal_page_size() == 16);

  // fill: validation, then the launch stand-in
  std::vector<uint16_t> buf(1 << 16);
  void* b = buf.data();
  EXPECT(pal_fill_kv_pages(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, 4, 2, 12, 16, 8, 1, 1,
                           nullptr) == PAL_ERR_INVALID_ARGUMENT);
  EXPECT(pal_fill_kv_pages(b, b, b, b, (const uint32_t*)b, (const int32_t*)b, (const uint32_t*)b, 1, 4, 2, 64, 16, 8,
                           1, 1, nullptr) == PAL_ERR_HIP);
  EXPECT(pal_rope_fill_kv_pages(b, b, PAL_DTYPE_FLOAT32, b, b, PAL_DTYPE_BFLOAT16, nullptr, nullptr,
                                (const uint32_t*)b, (const int32_t*)b, (const uint32_t*)b, 4, 2, 64, 16, 8, 1, 1,
                                (const float*)b, 32, 24, PAL_ROPE_NEOX, nullptr, nullptr, 0, 1, nullptr) ==
         PAL_ERR_INVALID_ARGUMENT);  // neox rotary_dim must be a multiple of 16
  EXPECT(pal_fill_kv_pages_fp8(b, b, PAL_DTYPE_BFLOAT16, b, b, nullptr, nullptr, (const uint32_t*)b,
                               (const int32_t*)b, (const uint32_t*)b, 4, 2, 64, 16, 8, 1, 1, nullptr) ==
         PAL_ERR_INVALID_ARGUMENT);  // fp8 needs scales

  // decode: validation order, workspace sizing and the launch stand-in
  EXPECT(pal_paged_attention_decode(b, b, b, (const uint32_t*)b, (const int32_t*)b, b, 1, 4, 4, 6, 4, 128, 16, 8, 4,
                                    0, nullptr, 0, nullptr) == PAL_ERR_RUNTIME);  // Hq % Hkv
  EXPECT(pal_paged_attention_decode(b, b, b, (const uint32_t*)b, (const int32_t*)b, b, 1, 4, 4, 8, 4, 128, 16, 8, 4,
                                    100, nullptr, 0, nullptr) == PAL_ERR_INVALID_ARGUMENT);  // partition
  const size_t ws = pal_paged_attention_decode_workspace_size(PAL_DTYPE_BFLOAT16, 64, 32, 8, 128, 16, 256, 512);
  EXPECT(ws > 0);
  std::vector<uint8_t> wsb(ws + 256);
  void* wsp = reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(wsb.data()) + 255) & ~uintptr_t(255));
  EXPECT(pal_paged_attention_decode(b, b, b, (const uint32_t*)b, (const int32_t*)b, b, 1, 64, 64, 32, 8, 128, 16, 4096,
                                    256, 512, wsp, ws, nullptr) == PAL_ERR_HIP);
  EXPECT(pal_paged_attention_decode(b, b, b, (const uint32_t*)b, (const int32_t*)b, b, 1, 64, 64, 32, 8, 128, 16, 4096,
                                    256, 512, wsp, ws - 1, nullptr) == PAL_ERR_INVALID_ARGUMENT);
  EXPECT(pal_paged_attention_decode_noalloc(b, b, b, (const uint32_t*)b, (const int32_t*)b, b, 1, 4096, 4096, 32, 8,
                                            128, 16, 1 << 20, 8192, 128, nullptr) == PAL_ERR_INVALID_ARGUMENT);
  EXPECT(pal_paged_attention_decode_fp8(b, b, b, nullptr, nullptr, (const uint32_t*)b, (const int32_t*)b, b, 1, 4, 4,
                                        8, 4, 128, 16, 8, 4, 0, wsp, ws, nullptr) == PAL_ERR_INVALID_ARGUMENT);
  // prefill and fused validation
  EXPECT(pal_paged_attention_prefill(b, b, b, b, b, (const uint32_t*)b, (const int32_t*)b, b, 1, 8, 2, 8, 2, 48, 16,
                                     8, 4, nullptr) == PAL_ERR_RUNTIME);  // head_dim % 32
  EXPECT(pal_paged_attention_prefill(b, b, b, b, b, (const uint32_t*)b, (const int32_t*)b, b, 1, 8, 2, 8, 2, 64, 16, 8,
                                     4, nullptr) == PAL_ERR_HIP);
  EXPECT(pal_paged_attention_workspace_size(PAL_DTYPE_FLOAT16, 0, 8, 2, 64, 16) == 0);

  // page pool: random histories; invariants of every compaction
  std::mt19937 rng(7);
  for (int trial = 0; trial < 50; ++trial) {
    const int64_t n = 1 + rng() % 500;
    void* pool = nullptr;
    EXPECT(pal_page_pool_create(n, &pool) == PAL_OK);
    std::set<uint32_t> live;
    for (int step = 0; step < 60; ++step) {
      if (!live.empty() && rng() % 2) {
        std::vector<uint32_t> drop;
        for (uint32_t id : live)
          if (rng() % 3 == 0) drop.push_back(id);
        EXPECT(pal_page_pool_free(pool, drop.data(), static_cast<int64_t>(drop.size())) == PAL_OK);
        for (uint32_t id : drop) live.erase(id);
      } else {
        const int64_t k = rng() % (pal_page_pool_num_free(pool) + 1);
        std::vector<uint32_t> ids(k + 1);
        EXPECT(pal_page_pool_alloc(pool, k, ids.data()) == PAL_OK);
        for (int64_t i = 0; i < k; ++i) EXPECT(live.insert(ids[i]).second);
      }
    }
    const uint32_t bogus[2] = {static_cast<uint32_t>(n), 0};
    EXPECT(pal_page_pool_free(pool, bogus, 1) == PAL_ERR_INVALID_ARGUMENT);
    EXPECT(pal_page_pool_alloc(pool, n + 1, nullptr) == PAL_ERR_INVALID_ARGUMENT ||
           pal_page_pool_alloc(pool, n + 1, std::vector<uint32_t>(n + 1).data()) == PAL_ERR_RUNTIME);
    int64_t m = -1;
    EXPECT(pal_page_pool_compaction_plan(pool, nullptr, nullptr, 0, &m) == PAL_OK && m >= 0);
    std::vector<uint32_t> src(m + 1), dst(m + 1);
    EXPECT(pal_page_pool_compaction_plan(pool, src.data(), dst.data(), m, &m) == PAL_OK);
    const int64_t L = static_cast<int64_t>(live.size());
    for (int64_t i = 0; i < m; ++i) {
      EXPECT(src[i] >= L && dst[i] < L && live.count(src[i]) && !live.count(dst[i]));
      live.erase(src[i]);
      live.insert(dst[i]);
    }
    EXPECT(static_cast<int64_t>(live.size()) == L && (L == 0 || *live.rbegin() == L - 1));
    EXPECT(pal_page_pool_num_free(pool) == n - L);
    EXPECT(pal_page_pool_destroy(pool) == PAL_OK);
  }
  uint32_t flags = 1;
  EXPECT(pal_debug_flags(1, &flags) == PAL_ERR_RUNTIME && flags == 0);
  if (g_fail) {
    std::fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  std::printf("host ABI driver: all checks passed\n");
  return 0;
}
