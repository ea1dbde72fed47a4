// fill_kv_pages for gfx950: bit-exact scatter of new K/V rows into the pools.
//
// Reference behaviour: kernels/paged_attention/fill_kv_pages.h.metal:65-116 --
//   seq = q2seq[t], pos = write_pos[t], page = page_table[seq, pos / TPP],
//   slot = pos % TPP,
//   K[page, h, d / 8, slot, d % 8] = new_k[t, h, d]
//   V[page, h, d, slot]            = new_v[t, h, d]
//
// Design (MI355X): the scatter is HBM-bound byte movement, so the mapping is
// chosen for write coalescing and for parallelism at small token counts.
// Workgroup (x, y) of 256 threads owns 16 consecutive tokens and 16 of their
// 16-byte vectors (8 dims of one head each): thread (t = tid % 16,
// v = 16 y + tid / 16) moves vector v of token 16 x + t, so even a 64-token
// decode fill spreads over 32 workgroups.  When consecutive tokens
// land in consecutive slots of a page (prefill chunks), the 16 lanes that
// share v write 16 x 16 B = 256 contiguous bytes of K and, for each of the 8
// dims, 16 x 2 B = 32 contiguous bytes of V.  Reads are whole 16-byte vectors.
// Tokens whose destination falls outside the page table or the pool are
// skipped (the reference does not check and would write out of bounds).
#include "pal_device.h"

namespace pal {

namespace {

constexpr int kFillTokens = 16;
constexpr int kFillThreads = 256;

__global__ __launch_bounds__(kFillThreads) void fill_kv_pages_kernel(const FillParams p) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kFillTokens + (threadIdx.x % kFillTokens);
  const int hd = p.head_dim;
  const int stripes = hd / 8;
  const int v = blockIdx.y * (kFillThreads / kFillTokens) + threadIdx.x / kFillTokens;
  if (t >= p.num_tokens || v >= p.num_kv_heads * stripes) return;  // no barriers in this kernel
  const uint32_t seq = p.q2seq[t];
  const int32_t pos = p.write_pos[t];
  const int tpp = p.tokens_per_page;
  if (seq >= p.num_seqs || pos < 0 || pos / tpp >= p.page_table_width) return;
  const uint32_t page = p.page_table[static_cast<int64_t>(seq) * p.page_table_width + pos / tpp];
  if (page >= p.num_pages) return;
  const int slot = pos % tpp;

  const int h = v / stripes;
  const int c = v - h * stripes;
  const int64_t row = t * p.num_kv_heads * hd;
  const u32x4 kd = reinterpret_cast<const u32x4*>(p.new_k + row)[v];
  const u32x4 vd = reinterpret_cast<const u32x4*>(p.new_v + row)[v];
  const int64_t head_block = static_cast<int64_t>(hd) * tpp;
  const int64_t hb = (static_cast<int64_t>(page) * p.num_kv_heads + h) * head_block;
  *reinterpret_cast<u32x4*>(p.k_pool + hb + (static_cast<int64_t>(c) * tpp + slot) * 8) = kd;
  uint16_t* vdst = p.v_pool + hb + static_cast<int64_t>(c) * 8 * tpp + slot;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    vdst[(2 * e) * tpp] = static_cast<uint16_t>(vd[e] & 0xFFFFu);
    vdst[(2 * e + 1) * tpp] = static_cast<uint16_t>(vd[e] >> 16);
  }
}

}  // namespace

hipError_t launch_fill_kv_pages(const FillParams& p, hipStream_t stream) {
  if (p.num_tokens <= 0) return hipSuccess;
  const int64_t blocks = (p.num_tokens + kFillTokens - 1) / kFillTokens;
  const int nvec = p.num_kv_heads * (p.head_dim / 8);
  const int vec_blocks = (nvec + kFillThreads / kFillTokens - 1) / (kFillThreads / kFillTokens);
  hipLaunchKernelGGL(fill_kv_pages_kernel, dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(vec_blocks)),
                     dim3(kFillThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace pal
