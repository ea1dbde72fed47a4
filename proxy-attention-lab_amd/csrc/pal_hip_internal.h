// Internal declarations shared by the kernel translation units and the C ABI
// layer (pal_abi.cpp).  Nothing here is part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pal {

constexpr int kF16 = 0;   // == PAL_DTYPE_FLOAT16
constexpr int kBF16 = 1;  // == PAL_DTYPE_BFLOAT16

// fill_kv_pages: scatter of new K/V rows into the paged pools.
struct FillParams {
  const uint16_t* new_k;       // [N, Hkv, HD]
  const uint16_t* new_v;       // [N, Hkv, HD]
  uint16_t* k_pool;            // [P, Hkv, HD/8, TPP, 8]
  uint16_t* v_pool;            // [P, Hkv, HD, TPP]
  const uint32_t* page_table;  // [S, W]
  const int32_t* write_pos;    // [N]
  const uint32_t* q2seq;       // [N]
  int64_t num_tokens;
  int64_t num_pages;
  int64_t num_seqs;
  int64_t page_table_width;
  int num_kv_heads;
  int head_dim;
  int tokens_per_page;
};

hipError_t launch_fill_kv_pages(const FillParams& p, hipStream_t stream);

// Split-K decode.  One workgroup handles (partition, kv head, head chunk of
// up to 16 query heads, sequence); the merge pass combines partitions.
struct DecodeParams {
  const uint16_t* q;           // [>=S, Hq, HD]
  const uint16_t* k_pool;      // [P, Hkv, HD/8, TPP, 8]
  const uint16_t* v_pool;      // [P, Hkv, HD, TPP]
  const uint32_t* page_table;  // [S, W]
  const int32_t* seq_lens;     // [S]
  uint16_t* out;               // [S, Hq, HD]
  float* part_o;               // [S, Hq, max_parts, HD]
  float* part_ml;              // [S, Hq, max_parts, 2]  (max * log2e * scale, exp-sum)
  int64_t num_seqs;
  int64_t num_pages;
  int64_t page_table_width;
  int num_q_heads;
  int num_kv_heads;
  int group;        // Hq / Hkv
  int head_chunks;  // ceil(group / 16)
  int max_parts;    // partitions per sequence the workspace holds
  float scale_log2; // log2(e) / sqrt(HD)
};

// Tokens per partition = 4 waves * blocks_per_wave * 16.
hipError_t launch_decode(const DecodeParams& p, int dtype, int head_dim, int tokens_per_page,
                         int blocks_per_wave, hipStream_t stream);

}  // namespace pal
