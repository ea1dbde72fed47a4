// Page moves for the page-pool compaction (pal_page_pool_compaction_plan in
// page_pool.cpp): copy whole pages of the K / V pools (and the fp8 scale
// rows) from source to destination ids, and rewrite page tables through a
// remap table.  HBM-bound byte movement: a page of one pool is one contiguous
// block of Hkv * HD * TPP elements, copied 16 bytes per lane.
#include "pal_device.h"
#include "pal_log.h"

namespace pal {

namespace {

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 4;  // 16-byte vectors per thread per pass, loads issued together

// Workgroup (x, y): move x (grid-strided), y = 0 K pool, 1 V pool, 2 the
// scale rows of both.  Moves whose ids are out of range are skipped.
__global__ __launch_bounds__(kCopyThreads) void copy_pages_kernel(const PageCopyParams p) {
  const int which = blockIdx.y;
  for (int64_t m = blockIdx.x; m < p.num_moves; m += gridDim.x) {
    const uint32_t src = p.src[m];
    const uint32_t dst = p.dst[m];
    if (src >= p.num_pages || dst >= p.num_pages || src == dst) continue;
    if (which == 2) {
      if (p.k_scales && threadIdx.x < static_cast<unsigned>(p.num_kv_heads)) {
        p.k_scales[static_cast<int64_t>(dst) * p.num_kv_heads + threadIdx.x] =
            p.k_scales[static_cast<int64_t>(src) * p.num_kv_heads + threadIdx.x];
        p.v_scales[static_cast<int64_t>(dst) * p.num_kv_heads + threadIdx.x] =
            p.v_scales[static_cast<int64_t>(src) * p.num_kv_heads + threadIdx.x];
      }
      continue;
    }
    uint8_t* pool = static_cast<uint8_t*>(which == 0 ? p.k_pool : p.v_pool);
    const u32x4* s = reinterpret_cast<const u32x4*>(pool + static_cast<int64_t>(src) * p.page_bytes);
    u32x4* d = reinterpret_cast<u32x4*>(pool + static_cast<int64_t>(dst) * p.page_bytes);
    const int64_t nvec = p.page_bytes / 16;
    for (int64_t base = 0; base < nvec; base += kCopyThreads * kCopyUnroll) {
      u32x4 v[kCopyUnroll];
#pragma unroll
      for (int u = 0; u < kCopyUnroll; ++u) {
        const int64_t i = base + u * kCopyThreads + threadIdx.x;
        if (i < nvec) v[u] = s[i];
      }
#pragma unroll
      for (int u = 0; u < kCopyUnroll; ++u) {
        const int64_t i = base + u * kCopyThreads + threadIdx.x;
        if (i < nvec) d[i] = v[u];
      }
    }
  }
}

__global__ __launch_bounds__(kCopyThreads) void remap_pages_kernel(uint32_t* table, int64_t n, const uint32_t* remap,
                                                                   int64_t remap_len) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kCopyThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kCopyThreads) {
    const uint32_t id = table[i];
    if (id < remap_len) table[i] = remap[id];
  }
}

}  // namespace

hipError_t launch_copy_pages(const PageCopyParams& p, hipStream_t stream) {
  if (p.num_moves <= 0) return hipSuccess;
  const int64_t gx = p.num_moves < 65535 ? p.num_moves : 65535;
  PAL_LOG("copy_pages moves=%lld page_bytes=%lld scales=%d", static_cast<long long>(p.num_moves),
          static_cast<long long>(p.page_bytes), p.k_scales ? 1 : 0);
  hipLaunchKernelGGL(copy_pages_kernel, dim3(static_cast<unsigned>(gx), p.k_scales ? 3 : 2), dim3(kCopyThreads), 0,
                     stream, p);
  return hipGetLastError();
}

hipError_t launch_remap_pages(uint32_t* table, int64_t n, const uint32_t* remap, int64_t remap_len,
                              hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + kCopyThreads - 1) / kCopyThreads;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(remap_pages_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kCopyThreads), 0, stream, table, n,
                     remap, remap_len);
  return hipGetLastError();
}

}  // namespace pal
