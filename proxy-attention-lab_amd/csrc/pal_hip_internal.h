// Internal declarations shared by the kernel translation units and the C ABI
// layer (pal_abi.cpp).  Nothing here is part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pal {

constexpr int kF16 = 0;   // == PAL_DTYPE_FLOAT16
constexpr int kBF16 = 1;  // == PAL_DTYPE_BFLOAT16
constexpr int kFP8 = 2;   // == PAL_DTYPE_FP8_E4M3 (pools only)
constexpr int kF32 = 3;   // == PAL_DTYPE_FLOAT32 (fill sources only)

constexpr int kMaxFillHeadDim = 256;

// fill_kv_pages: scatter of new K/V rows into the paged pools, optionally
// with RoPE on K (and Q) and a cast from fp32 / 16-bit to the pool dtype.
struct FillParams {
  const void* new_k;           // [N, Hkv, HD] src_dtype
  const void* new_v;           // [N, Hkv, HD] src_dtype
  void* k_pool;                // [P, Hkv, HD/x, TPP, x], x = 16 / element bytes
  void* v_pool;                // [P, Hkv, HD, TPP]
  const float* k_scales;       // fp8 pools: [P, Hkv] dequantisation scales
  const float* v_scales;
  const uint32_t* page_table;  // [S, W]
  const int32_t* write_pos;    // [N]
  const uint32_t* q2seq;       // [N]
  const float* cos_sin;        // rope: [cos_sin_rows, rotary_dim] (cos | sin)
  const void* q_in;            // rope, optional: [N, Hq, HD] src_dtype
  void* q_out;                 // [N, Hq, HD] q_out_dtype (16-bit)
  int64_t num_tokens;
  int64_t num_pages;
  int64_t num_seqs;
  int64_t page_table_width;
  int64_t cos_sin_rows;
  int num_kv_heads;
  int num_q_heads;
  int head_dim;
  int tokens_per_page;
  int src_dtype;               // kF16, kBF16, kF32
  int kv_dtype;                // kF16, kBF16, kFP8
  int q_out_dtype;             // kF16, kBF16
  int rope_style;              // 0 none, 1 NeoX (rotate halves), 2 GPT-J (rotate pairs)
  int rotary_dim;
};

hipError_t launch_fill_kv_pages(const FillParams& p, hipStream_t stream);

// Decode: the flat list of 16-token blocks of all (sequence, kv head, head
// chunk) segments is cut into virtual workers (static shares of the resident
// wavefronts plus dynamically claimed chunks); a merge kernel combines the
// segments that several virtual workers shared.
struct DecodeParams {
  const uint16_t* q;           // [>=S, Hq, HD]
  const void* k_pool;          // [P, Hkv, HD/x, TPP, x]: 16-bit (x = 8) or fp8 (x = 16)
  const void* v_pool;          // [P, Hkv, HD, TPP]
  const float* k_scales;       // fp8 pools: [P, Hkv] (null: 16-bit pools of the query dtype)
  const float* v_scales;
  const uint32_t* page_table;  // [S, W]
  const int32_t* seq_lens;     // [S]
  uint16_t* out;               // [S, Hq, HD] (row mode: [R, Hq, HD])
  // row mode (both null for plain decode): item i is query row i of
  // sequence q2seq[i] with min(seq_lens[seq], q_offset[i]) keys, if row i is
  // alone in its run of same-sequence rows; other rows are skipped (the
  // prefill kernel owns them)
  const uint32_t* q2seq;
  const int32_t* q_offset;
  int64_t num_pt_rows;           // page-table rows (sequences) in row mode
  // workspace
  int64_t* hdr;                // hdr[0] = total blocks T
  uint32_t* claim;             // dynamic-chunk counter: 0 on entry, re-armed to 0 by the merge kernel
  int64_t* split_list;         // [list_cap][4] per virtual worker: {first block (< 0: none), blocks,
                               // output row, segment} of the split segment its range ends in
                               // (every live slot is written by each call before the merge reads it)
  int64_t list_cap;
  int64_t* cum;                // [S + 1] first global block of each sequence
  float* part_ml;              // [virtual workers][2][hg_max][2] (max * log2e * scale, exp-sum)
  uint16_t* part_o;            // [virtual workers][2][hg_max][HD]  O / exp-sum, 16-bit dtype
  int64_t num_seqs;       // items (row mode: query rows)
  int64_t num_pages;
  int64_t page_table_width;
  int num_q_heads;
  int num_kv_heads;
  int group;              // Hq / Hkv
  int head_chunks;        // ceil(group / 16)
  int hg_max;             // min(group, 16): query heads per segment
  int num_workers;        // resident wavefront workers launched
  int tokens_per_worker;  // 0: static shares + dynamic chunks; > 0: fixed chunks of this many tokens
  float scale_log2;       // log2(e) / sqrt(HD)
};

// Workers the GPU keeps resident for this kernel configuration (shared_cu:
// the fused kernel's decode workers, one workgroup per CU beside the prefill
// tiles, head dims up to 128; chunks: the fixed-chunk mode,
// partition_size > 0; kv8: fp8 pools).
hipError_t decode_resident_workers(int dtype, int head_dim, int tokens_per_page, bool shared_cu, bool chunks,
                                   bool kv8, int* workers);
// Virtual workers (merge-list and partial slots) a call can produce: the
// resident workers' equal shares, or, with a partition size, one per fixed
// chunk of max_blocks (the 16-token blocks the page tables can hold).
int64_t decode_virtual_workers(int64_t resident, int64_t max_blocks, int partition_size);
hipError_t launch_decode(const DecodeParams& p, int dtype, int head_dim, int tokens_per_page, hipStream_t stream);

// Causal attention over query tiles (prefill rows).  Uniform-prompt mode
// (prompt_len > 0): the reference prefill, keys past each sequence's history
// read from dense prompt K/V.  Window mode (prompt_len == 0): the fused op's
// rows in windows of `tokens per tile`; runs of one sequence are tiles, all
// keys from pages, and lone rows are left to the decode kernels.
struct PrefillParams {
  const uint16_t* q;           // [R, Hq, HD]
  uint16_t* out;               // [R, Hq, HD]
  const uint16_t* k_pool;      // [P, Hkv, HD/8, TPP, 8] (fp8 pools: [P, Hkv, HD/16, TPP, 16] bytes)
  const uint16_t* v_pool;      // [P, Hkv, HD, TPP]
  const float* k_scales;       // fp8 pools: [P, Hkv] (null: 16-bit pools of the query dtype)
  const float* v_scales;
  const uint16_t* k_dense;     // prompt mode: [S * prompt_len, Hkv, HD]
  const uint16_t* v_dense;
  const uint32_t* page_table;  // [S, W]
  const int32_t* seq_lens;     // window mode: keys per sequence; prompt mode: history per sequence
  const int32_t* q_offset;     // window mode: [R] keys visible to each row (before the seq_lens clamp)
  const uint32_t* q2seq;       // window mode: [R] sequence of each row
  int64_t num_rows;            // R
  int64_t num_seqs;            // page-table rows
  int64_t num_pages;
  int64_t page_table_width;
  int num_units;    // prompt mode: S * ceil(prompt_len / tokens per tile); window mode: ceil(R / tokens per tile)
  int prompt_len;   // > 0 selects uniform-prompt mode
  int tokens_per_page;  // page size (the kernels built for 16 and 32 also take it as a constant)
  int num_q_heads;
  int num_kv_heads;
  int group;
  int head_chunks;
  int hg_max;
  float scale_log2;      // log2(e) / sqrt(HD)
  float scale_inv_log2;  // 1 / scale_log2
};

// Query tokens per prefill tile (and window) for a GQA group size.
int prefill_tokens_per_tile(int group);
hipError_t launch_prefill(const PrefillParams& p, int dtype, int head_dim, int tokens_per_page, hipStream_t stream);

// The fused mixed batch: the decode rows (dp, row mode) and the prefill tiles
// (pp, window mode) in one kernel for head dims up to 128 (then dp's workers
// are one workgroup per CU: fused_shares_cu), one after the other above.
bool fused_shares_cu(int head_dim);
hipError_t launch_fused(const DecodeParams& dp, const PrefillParams& pp, int dtype, int head_dim, int tokens_per_page,
                        hipStream_t stream);

// Page moves of a compaction: pages src[m] -> dst[m] of both pools (whole
// pages, page_bytes each) and, for fp8 pools, their scale rows.  Sources and
// destinations must be disjoint sets.
struct PageCopyParams {
  void* k_pool;
  void* v_pool;
  float* k_scales;  // null: 16-bit pools
  float* v_scales;
  const uint32_t* src;  // [num_moves] device
  const uint32_t* dst;
  int64_t num_moves;
  int64_t num_pages;
  int64_t page_bytes;
  int num_kv_heads;
};

hipError_t launch_copy_pages(const PageCopyParams& p, hipStream_t stream);
hipError_t launch_remap_pages(uint32_t* table, int64_t n, const uint32_t* remap, int64_t remap_len,
                              hipStream_t stream);

// Debug-check flag words of the kernel translation units (all zero in a
// build without PAL_DEBUG_CHECKS); reset clears them after reading.
hipError_t decode_debug_flags(uint32_t* out, bool reset);
hipError_t prefill_debug_flags(uint32_t* out, bool reset);
hipError_t fill_debug_flags(uint32_t* out, bool reset);

// Scratch memory held by the library for pal_paged_attention_decode_noalloc:
// kScratchBytes per device, in a file-scope device array (scratch.hip).
// scratch_buffer returns its device address on the current device.
constexpr size_t kScratchBytes = static_cast<size_t>(64) << 20;
hipError_t scratch_buffer(void** ptr);

}  // namespace pal
