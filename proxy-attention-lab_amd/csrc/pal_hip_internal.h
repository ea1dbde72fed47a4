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

// Decode ("stream-K"): a plan kernel splits the flat list of 16-token blocks
// of all (sequence, kv head, head chunk) segments evenly over num_workers
// wavefront workers; a merge kernel combines segments shared by workers.
struct DecodeParams {
  const uint16_t* q;           // [>=S, Hq, HD]
  const uint16_t* k_pool;      // [P, Hkv, HD/8, TPP, 8]
  const uint16_t* v_pool;      // [P, Hkv, HD, TPP]
  const uint32_t* page_table;  // [S, W]
  const int32_t* seq_lens;     // [S]
  uint16_t* out;               // [S, Hq, HD]
  // workspace
  int64_t* hdr;                // {total blocks T, workers in use}
  int64_t* cum;                // [S + 1] first global block of each sequence
  int64_t* plan;               // [num_workers][2] {sequence, block offset} of each worker's first block
  float* part_ml;              // [num_workers][2][hg_max][2] (max * log2e * scale, exp-sum)
  float* part_o;               // [num_workers][2][hg_max][HD]  unnormalised O
  int64_t num_seqs;
  int64_t num_pages;
  int64_t page_table_width;
  int num_q_heads;
  int num_kv_heads;
  int group;              // Hq / Hkv
  int head_chunks;        // ceil(group / 16)
  int hg_max;             // min(group, 16): query heads per segment
  int num_workers;        // workers launched
  int min_workers;        // workers the GPU keeps resident
  int tokens_per_worker;  // cap on tokens per worker (0 = none)
  float scale_log2;       // log2(e) / sqrt(HD)
};

// Workers the GPU keeps resident for this kernel configuration.
hipError_t decode_resident_workers(int dtype, int head_dim, int tokens_per_page, int* workers);
hipError_t launch_decode(const DecodeParams& p, int dtype, int head_dim, int tokens_per_page, hipStream_t stream);

}  // namespace pal
