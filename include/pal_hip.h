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
 *    buffers allocated by the caller; no entry point allocates or frees
 *    device memory.  The one static reservation: a 64 MiB `__device__`
 *    scratch array (the no-allocation decode entry's workspace) that the
 *    code object holds on every GPU where the library is loaded, whether
 *    or not that entry is called (the PAL_DEBUG_CHECKS build,
 *    libpal_hip_debug.so, holds its own copy).
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
/* fp8 e4m3 (OCP "fn": bias 7, max 448, no infinities) KV pages, each
 * (page, kv head) block with an fp32 scale: value = fp8 * scale.  Pool
 * layouts as above with x = 16 / sizeof(fp8) = 16.  The reference supports
 * f16 / bf16 only (paged_attention_kernels.metal:41-42). */
#define PAL_DTYPE_FP8_E4M3 2
/* fp32 sources of the fused RoPE + cast + scatter (the projection output). */
#define PAL_DTYPE_FLOAT32 3

#define PAL_ROPE_NONE 0
#define PAL_ROPE_NEOX 1 /* rotate halves: dims (f, f + rotary_dim / 2) */
#define PAL_ROPE_GPTJ 2 /* rotate pairs: dims (2f, 2f + 1) */

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
 * fill_kv_pages into fp8 e4m3 pools (no reference counterpart: the
 * reference's pools are f16 / bf16 only; this extends ops.py:133-171 with the
 * same index math, fill_kv_pages.h.metal:65-116, and x = 16 for the K stripe,
 * paged_attention_decode_primitive.cpp:384-397).  new_keys / new_values
 * ([N, Hkv, HD], src_dtype f16, bf16 or f32) are quantized with the
 * caller's per-(page, kv head) scales (k_scales / v_scales, fp32
 * [num_pages, Hkv]): q = x / scale, held to [-448, 448], rounded to nearest
 * even.  head_dim 64, 128 or 256 (the head dims the fp8 attention entries
 * read; others are rejected).  In place.
 */
int pal_fill_kv_pages_fp8(const void* new_keys, const void* new_values, int src_dtype, void* k_pool, void* v_pool,
                          const float* k_scales, const float* v_scales, const uint32_t* page_table,
                          const int32_t* write_positions, const uint32_t* query_to_seq_map, int64_t num_tokens,
                          int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages, int64_t num_seqs,
                          int64_t page_table_width, void* stream);

/*
 * RoPE + cast + scatter in one pass: the step that produces fill_kv_pages'
 * inputs (ops.py:133-171 -> fill_kv_pages.h.metal:56-116) fused with it.
 * No reference counterpart.  For token t at position p = write_positions[t]:
 * K (and, when queries is given, every query head of the token) is rotated
 * by the angles of row p of cos_sin_cache ([cos_sin_rows, rotary_dim] fp32:
 * cos of the rotary_dim / 2 frequencies, then their sin): NeoX style
 * (PAL_ROPE_NEOX) pairs dims (f, f + rotary_dim / 2), GPT-J style
 * (PAL_ROPE_GPTJ) pairs (2f, 2f + 1); dims at and past rotary_dim pass
 * through.  x' = x cos - y sin, y' = y cos + x sin in fp32, each product
 * rounded (no fused multiply-add).  K and V are then cast to kv_dtype
 * (f16 / bf16: round to nearest even; fp8: as pal_fill_kv_pages_fp8) and
 * scattered as fill_kv_pages does; the rotated queries are cast to
 * q_out_dtype (f16 / bf16) into queries_out ([N, Hq, HD]).  Tokens whose
 * position has no row in the table are not written to the pools; their
 * queries are cast without rotation.  head_dim <= 256; NeoX needs
 * rotary_dim % 16 == 0, GPT-J rotary_dim % 8 == 0.
 */
int pal_rope_fill_kv_pages(const void* new_keys, const void* new_values, int src_dtype, void* k_pool, void* v_pool,
                           int kv_dtype, const float* k_scales, const float* v_scales, const uint32_t* page_table,
                           const int32_t* write_positions, const uint32_t* query_to_seq_map, int64_t num_tokens,
                           int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages, int64_t num_seqs,
                           int64_t page_table_width, const float* cos_sin_cache, int64_t cos_sin_rows,
                           int rotary_dim, int rope_style, const void* queries, void* queries_out,
                           int num_q_heads, int q_out_dtype, void* stream);

/*
 * Workspace bytes pal_paged_attention_decode needs for these shapes on the
 * current device (0 for unsupported arguments or when no device is present).
 * The workspace holds a scan of the sequence lengths, a work-claim counter
 * and the partials (fp32 max and exp-sum, output / exp-sum in the query
 * dtype) of KV segments split between workers; its size follows from the
 * number of wavefront workers the device keeps resident.
 * partition_size: 0 (default: the KV blocks of the batch are cut into one
 * equal share per resident worker) or 128 / 256 / 512: fixed chunks of that
 * many tokens, each worker streaming an equal run of consecutive chunks,
 * every chunk its own partial, merged by log-sum-exp (the reference's
 * CHUNK_SIZE is 512, paged_attention_types.h:33).
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
 * decode_primitive.cpp:100-102,163-240) from the partials.  The workspace
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

/*
 * paged_attention_decode over fp8 e4m3 pools (no reference counterpart: the
 * reference's pools are f16 / bf16, paged_attention_kernels.metal:41-42; the
 * semantics are those of pal_paged_attention_decode, ops.py:42-84).  Keys
 * and values are the pools' codes times their (page, kv head) scale
 * (k_scales / v_scales, fp32 [num_pages, Hkv]); queries, output and the
 * arithmetic stay in dtype (f16 / bf16).  head_dim 64, 128 or 256.  The
 * workspace size comes from pal_paged_attention_decode_fp8_workspace_size.
 */
size_t pal_paged_attention_decode_fp8_workspace_size(int dtype, int64_t num_seqs, int num_q_heads, int num_kv_heads,
                                                     int head_dim, int tokens_per_page, int64_t page_table_width,
                                                     int partition_size);
int pal_paged_attention_decode_fp8(const void* queries, const void* k_pool, const void* v_pool,
                                   const float* k_scales, const float* v_scales, const uint32_t* page_table,
                                   const int32_t* sequence_lengths, void* out, int dtype, int64_t num_query_rows,
                                   int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                   int tokens_per_page, int64_t num_pages, int64_t page_table_width,
                                   int partition_size, void* workspace, size_t workspace_bytes, void* stream);

/*
 * No counterpart in the reference.  The same operation as
 * pal_paged_attention_decode for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): there is no workspace argument, and the call allocates nothing.
 * Its scratch (the length scan, merge list and split partials) is a
 * library-held device array of 64 MiB per GPU, kept until the process ends;
 * shapes whose workspace (pal_paged_attention_decode_workspace_size) would
 * exceed it are rejected with PAL_ERR_INVALID_ARGUMENT.  Every call on one
 * GPU shares that GPU's array: calls that can overlap on one GPU (different
 * streams, or threads) race and must be serialised by the caller.
 */
int pal_paged_attention_decode_noalloc(const void* queries, const void* k_pool, const void* v_pool,
                                       const uint32_t* page_table, const int32_t* sequence_lengths, void* out,
                                       int dtype, int64_t num_query_rows, int64_t num_seqs, int num_q_heads,
                                       int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages,
                                       int64_t page_table_width, int partition_size, void* stream);

/*
 * Replaces paged_attention_prefill (ops.py:87-130 -> bindings.cpp:74-124 ->
 * ops.cpp:110-186 -> paged_attention_prefill_primitive.cpp:63-167).
 * num_seqs = page-table rows; prompt_len P = num_query_rows / num_seqs
 * (primitive :115-116); rows s*P .. s*P+P-1 of q_prompt / k_prompt /
 * v_prompt ([rows, heads, head_dim]) are the prompt of sequence s, whose
 * cached history is tokens [0, context_lens[s]) of its pages.  Prompt token
 * i attends to the whole history plus prompt tokens 0..i, scale
 * 1/sqrt(head_dim) (prefill.h.metal:147-234).  out: [num_query_rows *
 * num_q_heads, head_dim], row (s*P + i) * num_q_heads + h; rows at and past
 * num_seqs * P are not written.  head_dim % 32 == 0 (primitive :91-93).
 * tokens_per_page: any multiple of 8 up to 1024, as the reference prefill
 * reads it at run time (paged_attention_prefill.h.metal:243-263); 16 and 32
 * have dedicated kernels, other sizes read their history keys through the
 * registers (slower).  No workspace.
 */
int pal_paged_attention_prefill(const void* q_prompt, const void* k_prompt, const void* v_prompt,
                                const void* k_cache_paged, const void* v_cache_paged, const uint32_t* page_table,
                                const int32_t* context_lens, void* out, int dtype, int64_t num_query_rows,
                                int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                int tokens_per_page, int64_t num_pages, int64_t page_table_width, void* stream);

/*
 * paged_attention_prefill over fp8 e4m3 paged history (no reference
 * counterpart; semantics of pal_paged_attention_prefill, ops.py:87-130):
 * the history's keys and values are their codes times the (page, kv head)
 * scales (k_scales / v_scales, fp32 [num_pages, Hkv]), dequantized to dtype
 * on the way into the tile; the dense prompt K/V and the queries are in
 * dtype.  head_dim 64, 128 or 256; tokens_per_page 16 or 32.
 */
int pal_paged_attention_prefill_fp8(const void* q_prompt, const void* k_prompt, const void* v_prompt,
                                    const void* k_cache_paged, const void* v_cache_paged, const float* k_scales,
                                    const float* v_scales, const uint32_t* page_table, const int32_t* context_lens,
                                    void* out, int dtype, int64_t num_query_rows, int64_t num_seqs, int num_q_heads,
                                    int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages,
                                    int64_t page_table_width, void* stream);

/*
 * Workspace bytes pal_paged_attention needs for num_query_rows rows on the
 * current device (0 for unsupported arguments or without a device).  Zero-fill
 * it before its first use; each call leaves it ready for the next one.
 */
size_t pal_paged_attention_workspace_size(int dtype, int64_t num_query_rows, int num_q_heads, int num_kv_heads,
                                          int head_dim, int tokens_per_page);

/*
 * Fused mixed batch of decode and prefill rows in one call.  The reference
 * has no such function: it only prepares query_to_seq_map and
 * query_token_offset in a benchmark
 * (benchmarks/.../batch_latency_vs_num_sequences.cpp:124-131); this is the
 * build's definition.  Row r (queries [num_query_rows, num_q_heads,
 * head_dim]) belongs to sequence s = query_to_seq_map[r] and attends to
 * tokens [0, min(sequence_lengths[s], query_token_offset[r])) of s's pages;
 * new tokens must already be in the pages (pal_fill_kv_pages).  A decode row
 * has offset >= its length; prompt token at absolute position p has offset
 * p + 1.  Rows with no visible token, or naming no sequence (s >= num_seqs),
 * yield zeros.  out: [num_query_rows, num_q_heads, head_dim].  Runs of
 * consecutive rows of one sequence go to MFMA prefill tiles, single rows to
 * split-K decode workers, in one kernel whose first workgroups are the decode
 * workers (head dims up to 128; above, the decode and prefill kernels run one
 * after the other), followed by the merge kernel; the decode workers find
 * and schedule the single rows on the device, so the call never reads row
 * metadata on the host.  The workspace (size
 * from pal_paged_attention_workspace_size, 256-byte aligned, zero-filled
 * before its first use) must not be shared by concurrent calls.
 */
int pal_paged_attention(const void* queries, const void* k_pool, const void* v_pool, const uint32_t* page_table,
                        const int32_t* sequence_lengths, const uint32_t* query_to_seq_map,
                        const int32_t* query_token_offset, void* out, int dtype, int64_t num_query_rows,
                        int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim, int tokens_per_page,
                        int64_t num_pages, int64_t page_table_width, void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * The fused mixed batch over fp8 e4m3 pools (pal_paged_attention's
 * semantics; keys and values are codes times their (page, kv head) scale,
 * k_scales / v_scales fp32 [num_pages, Hkv]).  No reference counterpart.
 * head_dim 64, 128 or 256; workspace from
 * pal_paged_attention_fp8_workspace_size.
 */
size_t pal_paged_attention_fp8_workspace_size(int dtype, int64_t num_query_rows, int num_q_heads, int num_kv_heads,
                                              int head_dim, int tokens_per_page);
int pal_paged_attention_fp8(const void* queries, const void* k_pool, const void* v_pool, const float* k_scales,
                            const float* v_scales, const uint32_t* page_table, const int32_t* sequence_lengths,
                            const uint32_t* query_to_seq_map, const int32_t* query_token_offset, void* out, int dtype,
                            int64_t num_query_rows, int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                            int tokens_per_page, int64_t num_pages, int64_t page_table_width, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Page-pool allocator and compaction.  No reference counterpart: the
 * reference takes page tables from its caller (ops.py:61-63,
 * paged_attention_decode_primitive.cpp:71-266 reads them as an input); this
 * is the allocator a serving engine keeps in front of the pools.  Host-side
 * state, internally locked.
 *
 * pal_page_pool_create: a pool of num_pages free page ids (< 2^32).
 * pal_page_pool_alloc: the n lowest free ids, ascending, into out_ids; fails
 *   with PAL_ERR_RUNTIME (and allocates nothing) when fewer are free.
 * pal_page_pool_free: returns ids; an id out of range, not allocated or
 *   listed twice fails the whole call (PAL_ERR_INVALID_ARGUMENT), nothing
 *   freed.
 * pal_page_pool_num_free: free ids (negative status for a null pool).
 * pal_page_pool_compaction_plan: moves every allocated id at or above L
 *   (the number of allocated ids) to a free id below L, both in ascending
 *   order, so the allocated ids become exactly [0, L); writes the moves to
 *   src / dst (host arrays of `capacity` entries) and their count to
 *   *n_moves, and updates the allocator.  With src = dst = NULL and
 *   capacity 0 it only reports the count.  Apply the moves with
 *   pal_copy_pages, then rewrite page tables with pal_remap_pages.
 */
int pal_page_pool_create(int64_t num_pages, void** pool);
int pal_page_pool_destroy(void* pool);
int pal_page_pool_alloc(void* pool, int64_t n, uint32_t* out_ids);
int pal_page_pool_free(void* pool, const uint32_t* ids, int64_t n);
int64_t pal_page_pool_num_free(void* pool);
int pal_page_pool_compaction_plan(void* pool, uint32_t* src, uint32_t* dst, int64_t capacity, int64_t* n_moves);

/*
 * Copies pages src[m] -> dst[m] (device arrays, num_moves entries) of both
 * pools, page_bytes bytes per page and pool (Hkv * HD * TPP * element size),
 * and for fp8 pools the scale rows (k_scales / v_scales [num_pages, Hkv],
 * both or neither).  Ids >= num_pages are skipped.  Sources and
 * destinations must be disjoint sets (a compaction plan is).  Bit-exact.
 */
int pal_copy_pages(void* k_pool, void* v_pool, float* k_scales, float* v_scales, int64_t num_pages, int num_kv_heads,
                   int64_t page_bytes, const uint32_t* src, const uint32_t* dst, int64_t num_moves, void* stream);

/*
 * In place over num_entries page ids (device): id -> remap[id] for
 * id < remap_len, other ids unchanged.
 */
int pal_remap_pages(uint32_t* page_table, int64_t num_entries, const uint32_t* remap, int64_t remap_len,
                    void* stream);

/*
 * Debug checks.  A library built with PAL_DEBUG_CHECKS (build_lib.py
 * --debug-checks: libpal_hip_debug.so) records, instead of silently
 * tolerating, inputs the caller most likely did not mean: a page id past
 * the pool where a token was to be read (PAL_DEBUG_PAGE_ID), a sequence
 * length or history past page_table_width * tokens_per_page
 * (PAL_DEBUG_LENGTH), a fill token with no valid destination
 * (PAL_DEBUG_FILL_DEST).  pal_debug_flags waits for nothing: call it after
 * synchronising; it ORs the recorded bits into *flags and, with reset,
 * clears them.  No reference counterpart (the reference's Debug build only
 * adds host-side checks, src/pal_core/CMakeLists.txt:16-31).  A release
 * build returns PAL_ERR_RUNTIME and flags 0.
 */
#define PAL_DEBUG_PAGE_ID 1u
#define PAL_DEBUG_LENGTH 2u
#define PAL_DEBUG_FILL_DEST 4u
int pal_debug_flags(int reset, uint32_t* flags);

#ifdef __cplusplus
}
#endif

#endif /* PAL_HIP_H_ */
