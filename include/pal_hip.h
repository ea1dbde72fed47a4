/*
 * pal_hip.h -- C ABI of libpal_hip.so, the gfx950 (MI355X) implementation of
 * PAL's paged-attention operator family.
 *
 * This header replaces the reference's nanobind module `pal_core`
 * (src/pal_core/bindings.cpp:41-226) and the MLX graph-op layer behind it
 * (src/pal_core/src/ops.cpp:36-241).  Each entry point below names the
 * reference function it stands in for.
 *
 * Conventions
 *  - All tensor arguments are raw device pointers to contiguous row-major
 *    buffers allocated by the caller; the library never allocates or frees.
 *  - fp16 / bf16 data is passed as `void*`, with a dtype code.
 *  - `stream` is a hipStream_t passed as `void*` (NULL = the null stream).
 *    Launches are asynchronous; the caller synchronises.
 *  - Return value: PAL_OK (0) or a negative status.  The message of the last
 *    failure on the calling thread is returned by pal_last_error().
 *    PAL_ERR_INVALID_ARGUMENT corresponds to the reference's
 *    std::invalid_argument (Python ValueError), PAL_ERR_RUNTIME to its
 *    std::runtime_error (Python RuntimeError), e.g. ops.cpp:204-211 and
 *    paged_attention_decode_primitive.cpp:152-159.
 *
 * Pool layouts (paged_attention_decode_primitive.cpp:373-397):
 *    K pool  [num_pages, num_kv_heads, head_dim / x, tokens_per_page, x]
 *    V pool  [num_pages, num_kv_heads, head_dim, tokens_per_page]
 *    with x = 16 / sizeof(element) = 8 for fp16 and bf16.
 * Page table: uint32 (int32 with the same bits is accepted) [num_seqs, width].
 */
#ifndef PAL_HIP_H_
#define PAL_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PAL_DTYPE_FLOAT16 0
#define PAL_DTYPE_BFLOAT16 1

#define PAL_OK 0
#define PAL_ERR_INVALID_ARGUMENT (-1)
#define PAL_ERR_RUNTIME (-2)
#define PAL_ERR_HIP (-3)

/* Message of the last failed call on this thread ("" if none). */
const char* pal_last_error(void);

/* Library version string (the reference module reports "2025.06.4",
 * bindings.cpp:225). */
const char* pal_version(void);

/* Replaces get_k_cache_stripe_size (bindings.cpp:44-48): 16 / sizeof(dtype).
 * Returns a negative status for an unsupported dtype. */
int pal_get_k_cache_stripe_size(int dtype);

/* Replaces get_optimal_page_size (constants.hpp:7-11, bindings.cpp:66-72). */
int pal_get_optimal_page_size(void);

/* Replace get_k_cache_shape / get_v_cache_shape
 * (paged_attention_decode_primitive.cpp:373-397, bindings.cpp:50-64). */
int pal_get_k_cache_shape(int64_t num_pages, int num_kv_heads, int head_dim, int tokens_per_page,
                          int dtype, int64_t out_shape[5]);
int pal_get_v_cache_shape(int64_t num_pages, int num_kv_heads, int head_dim, int tokens_per_page,
                          int dtype, int64_t out_shape[4]);

/*
 * Replaces fill_kv_pages (ops.py:133-171 -> bindings.cpp:182-222 ->
 * ops.cpp:188-239 -> fill_kv_pages_primitive.cpp:70-170).
 * For each new token t: seq = query_to_seq_map[t], pos = write_positions[t],
 * page = page_table[seq * page_table_width + pos / tokens_per_page],
 * slot = pos % tokens_per_page; new_keys[t] / new_values[t] ([num_kv_heads,
 * head_dim]) are copied bit-exactly into that page slot of k_pool / v_pool.
 * The pools are updated IN PLACE (the reference returns fresh copies).
 * Destinations must be distinct; tokens writing the same slot race, as in
 * the reference.
 */
int pal_fill_kv_pages(const void* new_keys, const void* new_values, void* k_pool, void* v_pool,
                      const uint32_t* page_table, const int32_t* write_positions,
                      const uint32_t* query_to_seq_map, int dtype, int64_t num_tokens,
                      int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages,
                      int64_t num_seqs, int64_t page_table_width, void* stream);

/*
 * Workspace bytes pal_paged_attention_decode needs for these shapes on the
 * current device (0 for unsupported arguments or when no device is present).
 * The workspace holds a scan of the sequence lengths, a work-claim counter
 * and the fp32 partials (max, exp-sum, unnormalised output) of KV segments
 * split between workers; its size follows from the number of wavefront
 * workers the device keeps resident.
 * partition_size: 0 (default: the KV blocks of the batch are shared out
 * evenly, three quarters statically and the rest in small chunks claimed by
 * whichever worker is free) or 128 / 256 / 512: fixed chunks of that many
 * tokens, each merged by log-sum-exp (the reference's CHUNK_SIZE is 512,
 * paged_attention_types.h:33).
 * The workspace must be zero-filled before its first use; each call leaves
 * it ready for the next one on the same stream.
 */
size_t pal_paged_attention_decode_workspace_size(int dtype, int64_t num_seqs, int num_q_heads,
                                                 int num_kv_heads, int head_dim, int tokens_per_page,
                                                 int64_t page_table_width, int partition_size);

/*
 * Replaces paged_attention_decode (ops.py:42-84 -> bindings.cpp:125-180 ->
 * ops.cpp:36-108 -> paged_attention_decode_primitive.cpp:71-266).
 * queries: [num_query_rows, num_q_heads, head_dim]; row s serves sequence s
 * (rows >= num_seqs are ignored, as in decode.h.metal:106-108).
 * out: [num_seqs, num_q_heads, head_dim] in the query dtype.
 * Sequence s attends to tokens [0, sequence_lengths[s]) of its pages with
 * scale 1/sqrt(head_dim); query head h reads KV head
 * h / (num_q_heads / num_kv_heads).  A sequence of length <= 0 yields zeros.
 * The KV blocks of all sequences are split evenly over the device's
 * resident workers; a sequence split between workers is merged with a
 * log-sum-exp pass (the reference's two-pass mode,
 * decode_primitive.cpp:100-102,163-240) from fp32 partials.  The workspace
 * (256-byte aligned, size from pal_paged_attention_decode_workspace_size,
 * zero-filled before its first use) must not be shared by calls that can
 * run concurrently.
 */
int pal_paged_attention_decode(const void* queries, const void* k_pool, const void* v_pool,
                               const uint32_t* page_table, const int32_t* sequence_lengths,
                               void* out, int dtype, int64_t num_query_rows, int64_t num_seqs,
                               int num_q_heads, int num_kv_heads, int head_dim,
                               int tokens_per_page, int64_t num_pages, int64_t page_table_width,
                               int partition_size, void* workspace, size_t workspace_bytes,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAL_HIP_H_ */
