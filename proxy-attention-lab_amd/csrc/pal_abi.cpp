// C ABI of libpal_hip.so: argument validation, workspace sizing and launch.
//
// Replaces the reference's binding + primitive host layers
// (src/pal_core/bindings.cpp, src/pal_core/src/ops.cpp,
// src/pal_core/src/*_primitive.cpp).  The library keeps a thread-local error
// message, a cache of occupancy-derived worker counts and, per device, the
// scratch array of the no-allocation entry point; it never allocates device
// memory.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/pal_hip.h"
#include "pal_hip_internal.h"
#include "pal_log.h"

namespace {

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  pal::set_last_error(buf);
  return code;
}

int ok() {
  pal::clear_last_error();
  return PAL_OK;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return ok();
  return fail(PAL_ERR_HIP, "[%s] HIP error: %s", what, hipGetErrorString(err));
}

bool valid_dtype(int dtype) { return dtype == PAL_DTYPE_FLOAT16 || dtype == PAL_DTYPE_BFLOAT16; }
bool valid_pool_dtype(int dtype) { return valid_dtype(dtype) || dtype == PAL_DTYPE_FP8_E4M3; }
int pool_elem_bytes(int dtype) { return dtype == PAL_DTYPE_FP8_E4M3 ? 1 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool decode_head_dim_supported(int hd) {
  return hd == 32 || hd == 64 || hd == 80 || hd == 96 || hd == 128 || hd == 256;
}

bool prefill_head_dim_supported(int hd) { return hd == 32 || hd == 64 || hd == 96 || hd == 128 || hd == 256; }

float scale_log2_for(int head_dim) {
  return static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_dim)));
}

bool decode_partition_ok(int partition_size) {
  return partition_size == 0 || partition_size == 128 || partition_size == 256 || partition_size == 512;
}

size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

constexpr int kMaxPageSize = 1024;  // prefill's run-time page sizes (multiples of 8)

// Decode workspace layout (all offsets 256-aligned).  The claim counter at
// byte 64 must be zero when a call starts; every call leaves it zero.  Every
// other byte is scratch that each call writes before it reads.
struct DecodeLayout {
  size_t hdr, claim, cum, list, part_ml, part_o, total;
  int64_t list_cap;
};

DecodeLayout decode_layout(int64_t num_seqs, int head_dim, int hg_max, int64_t virtual_workers) {
  DecodeLayout l;
  size_t off = 0;
  l.hdr = off;
  l.claim = off + 64;
  off += 256;
  l.cum = off;
  off += align256(static_cast<size_t>(num_seqs + 1) * sizeof(int64_t));
  // merge list: one slot per virtual worker
  l.list_cap = virtual_workers;
  l.list = off;
  off += align256(static_cast<size_t>(l.list_cap) * 4 * sizeof(int64_t));
  l.part_ml = off;
  off += align256(static_cast<size_t>(virtual_workers) * 2 * hg_max * 2 * sizeof(float));
  l.part_o = off;
  off += align256(static_cast<size_t>(virtual_workers) * 2 * hg_max * head_dim * sizeof(uint16_t));
  l.total = off;
  return l;
}

// Resident wavefront workers, and the number of virtual workers (partial
// slots) the cut can produce: one per equal static share, or, with a
// partition size, one per chunk of the page-table capacity.
int decode_workers(int dtype, int head_dim, int tokens_per_page, int64_t num_seqs, int num_kv_heads,
                   int head_chunks, int64_t page_table_width, int partition_size, bool shared_cu, bool kv8,
                   int* resident, int64_t* virtual_workers) {
  int res = 0;
  hipError_t err =
      pal::decode_resident_workers(dtype, head_dim, tokens_per_page, shared_cu, partition_size > 0, kv8, &res);
  if (err != hipSuccess)
    return fail(PAL_ERR_HIP, "[paged_attention_decode] occupancy query failed: %s", hipGetErrorString(err));
  const int64_t max_blocks =
      num_seqs * ((page_table_width * tokens_per_page + 15) / 16) * num_kv_heads * head_chunks;
  const int64_t vw = pal::decode_virtual_workers(res, max_blocks, partition_size);
  if (vw > (1LL << 28)) return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] problem too large for one call");
  *resident = res;
  *virtual_workers = vw;
  return PAL_OK;
}

// Common decode parameter set-up (plain decode: item i = row i = sequence i).
pal::DecodeParams decode_params(const void* queries, const void* k_pool, const void* v_pool,
                                const uint32_t* page_table, const int32_t* sequence_lengths, void* out,
                                char* ws, const DecodeLayout& lay, int64_t num_items, int64_t num_pages,
                                int64_t page_table_width, int num_q_heads, int num_kv_heads, int head_dim,
                                int resident, int partition_size) {
  const int group = num_q_heads / num_kv_heads;
  pal::DecodeParams p;
  p.q = static_cast<const uint16_t*>(queries);
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.k_scales = nullptr;
  p.v_scales = nullptr;
  p.page_table = page_table;
  p.seq_lens = sequence_lengths;
  p.out = static_cast<uint16_t*>(out);
  p.q2seq = nullptr;
  p.q_offset = nullptr;
  p.num_pt_rows = num_items;
  p.hdr = reinterpret_cast<int64_t*>(ws + lay.hdr);
  p.claim = reinterpret_cast<uint32_t*>(ws + lay.claim);
  p.split_list = reinterpret_cast<int64_t*>(ws + lay.list);
  p.list_cap = lay.list_cap;
  p.cum = reinterpret_cast<int64_t*>(ws + lay.cum);
  p.part_ml = reinterpret_cast<float*>(ws + lay.part_ml);
  p.part_o = reinterpret_cast<uint16_t*>(ws + lay.part_o);
  p.num_seqs = num_items;
  p.num_pages = num_pages;
  p.page_table_width = page_table_width;
  p.num_q_heads = num_q_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = group;
  p.head_chunks = (group + 15) / 16;
  p.hg_max = group < 16 ? group : 16;
  p.num_workers = resident;
  p.tokens_per_worker = partition_size;
  p.scale_log2 = scale_log2_for(head_dim);
  return p;
}

// Checks shared by every attention entry point; returns PAL_OK or an error.
int check_attention_dims(const char* op, int dtype, int num_q_heads, int num_kv_heads, int head_dim,
                         int tokens_per_page, int64_t num_pages, int64_t page_table_width, bool any_page_size = false) {
  if (!valid_dtype(dtype)) return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] unsupported dtype code %d", op, dtype);
  if (num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || tokens_per_page <= 0 || num_pages < 0 ||
      page_table_width < 0)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] negative or zero dimension", op);
  if (num_q_heads % num_kv_heads != 0)
    return fail(PAL_ERR_RUNTIME, "num_q_heads must be divisible by num_kv_heads (%d %% %d != 0)", num_q_heads,
                num_kv_heads);
  if (any_page_size) {  // prefill over 16-bit pools: any multiple of 8 up to kMaxPageSize
    if (tokens_per_page % 8 != 0 || tokens_per_page > kMaxPageSize)
      return fail(PAL_ERR_RUNTIME, "[%s] no kernel for tokens_per_page %d (supported: multiples of 8 up to %d)", op,
                  tokens_per_page, kMaxPageSize);
  } else if (tokens_per_page != 16 && tokens_per_page != 32) {
    return fail(PAL_ERR_RUNTIME, "[%s] no kernel for tokens_per_page %d (supported: 16, 32)", op, tokens_per_page);
  }
  return PAL_OK;
}

size_t decode_workspace_size(int dtype, int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                             int tokens_per_page, int64_t page_table_width, int partition_size, bool kv8) {
  if (!valid_dtype(dtype) || num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      tokens_per_page <= 0 || page_table_width < 0 || num_q_heads % num_kv_heads != 0 ||
      !decode_partition_ok(partition_size) || !decode_head_dim_supported(head_dim) ||
      (tokens_per_page != 16 && tokens_per_page != 32))
    return 0;
  const int group = num_q_heads / num_kv_heads;
  const int chunks = (group + 15) / 16;
  int resident = 0;
  int64_t vw = 0;
  if (decode_workers(dtype, head_dim, tokens_per_page, num_seqs, num_kv_heads, chunks, page_table_width,
                     partition_size, false, kv8, &resident, &vw) != PAL_OK)
    return 0;
  return decode_layout(num_seqs, head_dim, group < 16 ? group : 16, vw).total;
}

// Arguments of the three fill entry points (pal_fill_kv_pages,
// pal_fill_kv_pages_fp8, pal_rope_fill_kv_pages), validated in one place.
struct FillArgs {
  const void* new_keys = nullptr;
  const void* new_values = nullptr;
  int src_dtype = -1;
  void* k_pool = nullptr;
  void* v_pool = nullptr;
  int kv_dtype = -1;
  const float* k_scales = nullptr;
  const float* v_scales = nullptr;
  const uint32_t* page_table = nullptr;
  const int32_t* write_positions = nullptr;
  const uint32_t* query_to_seq_map = nullptr;
  int64_t num_tokens = 0;
  int num_kv_heads = 0;
  int head_dim = 0;
  int tokens_per_page = 0;
  int64_t num_pages = 0;
  int64_t num_seqs = 0;
  int64_t page_table_width = 0;
  const float* cos_sin = nullptr;
  int64_t cos_sin_rows = 0;
  int rotary_dim = 0;
  int rope_style = 0;
  const void* queries = nullptr;
  void* queries_out = nullptr;
  int num_q_heads = 0;
  int q_out_dtype = PAL_DTYPE_BFLOAT16;
};

int fill_call(const char* op, const FillArgs& a, hipStream_t stream) {
  const bool fp8 = a.kv_dtype == PAL_DTYPE_FP8_E4M3;
  if (!valid_dtype(a.kv_dtype) && !fp8) return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] unsupported pool dtype code %d", op, a.kv_dtype);
  if (!valid_dtype(a.src_dtype) && a.src_dtype != PAL_DTYPE_FLOAT32)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] unsupported source dtype code %d", op, a.src_dtype);
  if (a.num_tokens < 0 || a.num_kv_heads <= 0 || a.head_dim <= 0 || a.tokens_per_page <= 0 || a.num_pages < 0 ||
      a.num_seqs < 0 || a.page_table_width < 0)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] negative or zero dimension", op);
  const int chunk_dims = fp8 ? 16 : 8;  // one K stripe
  if (a.head_dim % chunk_dims != 0)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] head_dim %d must be a multiple of %d", op, a.head_dim, chunk_dims);
  // fp8 pools are written only at the head dims the fp8 attention kernels
  // read (a pool no kernel can attend over would only fail later)
  if (fp8 && a.head_dim != 64 && a.head_dim != 128 && a.head_dim != 256)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] fp8 pools: no attention kernel for head_dim %d (supported: 64, 128, "
                "256)", op, a.head_dim);
  if (a.head_dim > pal::kMaxFillHeadDim)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] head_dim %d above the supported %d", op, a.head_dim,
                pal::kMaxFillHeadDim);
  if (a.rope_style < 0 || a.rope_style > 2)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] rope_style %d not in {0 none, 1 neox, 2 gptj}", op, a.rope_style);
  if (a.rope_style != 0) {
    const int mult = a.rope_style == 1 ? 16 : 8;
    if (a.rotary_dim <= 0 || a.rotary_dim > a.head_dim || a.rotary_dim % mult != 0)
      return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] rotary_dim %d must be a positive multiple of %d up to head_dim %d",
                  op, a.rotary_dim, mult, a.head_dim);
    if (a.cos_sin_rows < 0 || (a.num_tokens > 0 && (!a.cos_sin || a.cos_sin_rows == 0)))
      return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] rope needs a cos/sin table", op);
  }
  if (a.queries) {
    if (a.rope_style == 0) return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] queries given without rope", op);
    if (!a.queries_out || !valid_dtype(a.q_out_dtype) || a.num_q_heads <= 0 || a.num_q_heads % a.num_kv_heads != 0)
      return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] queries need an output, a 16-bit output dtype and num_q_heads a "
                  "multiple of num_kv_heads", op);
  }
  if (a.num_tokens == 0) return ok();
  if (!a.new_keys || !a.new_values || !a.k_pool || !a.v_pool || !a.page_table || !a.write_positions ||
      !a.query_to_seq_map || (fp8 && (!a.k_scales || !a.v_scales)))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] null pointer argument", op);
  if (!aligned16(a.new_keys) || !aligned16(a.new_values) || !aligned16(a.k_pool) || !aligned16(a.v_pool) ||
      (a.queries && (!aligned16(a.queries) || !aligned16(a.queries_out))))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] new keys/values, pools and queries must be 16-byte aligned", op);
  pal::FillParams p;
  p.new_k = a.new_keys;
  p.new_v = a.new_values;
  p.k_pool = a.k_pool;
  p.v_pool = a.v_pool;
  p.k_scales = a.k_scales;
  p.v_scales = a.v_scales;
  p.page_table = a.page_table;
  p.write_pos = a.write_positions;
  p.q2seq = a.query_to_seq_map;
  p.cos_sin = a.cos_sin;
  p.q_in = a.queries;
  p.q_out = a.queries_out;
  p.num_tokens = a.num_tokens;
  p.num_pages = a.num_pages;
  p.num_seqs = a.num_seqs;
  p.page_table_width = a.page_table_width;
  p.cos_sin_rows = a.rope_style != 0 ? a.cos_sin_rows : 0;
  p.num_kv_heads = a.num_kv_heads;
  p.num_q_heads = a.num_q_heads;
  p.head_dim = a.head_dim;
  p.tokens_per_page = a.tokens_per_page;
  p.src_dtype = a.src_dtype;
  p.kv_dtype = a.kv_dtype;
  p.q_out_dtype = a.q_out_dtype;
  p.rope_style = a.rope_style;
  p.rotary_dim = a.rope_style != 0 ? a.rotary_dim : 0;
  PAL_LOG("%s tokens=%lld Hkv=%d HD=%d TPP=%d src=%d kv=%d rope=%d/%d queries=%d pages=%lld stream=%p", op,
          static_cast<long long>(a.num_tokens), a.num_kv_heads, a.head_dim, a.tokens_per_page, a.src_dtype,
          a.kv_dtype, a.rope_style, p.rotary_dim, a.queries ? a.num_q_heads : 0, static_cast<long long>(a.num_pages),
          static_cast<void*>(stream));
  return hip_status(pal::launch_fill_kv_pages(p, stream), op);
}

// fp8 pools: both scale arrays, and a head dim of whole 64-dim rounds
int check_fp8_scales(const char* op, const float* k_scales, const float* v_scales, int head_dim) {
  if (!k_scales && !v_scales) return PAL_OK;
  if (!k_scales || !v_scales) return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] fp8 pools need both k_scales and v_scales", op);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(PAL_ERR_RUNTIME, "[%s] no fp8 kernel for head_dim %d (supported: 64, 128, 256)", op, head_dim);
  return PAL_OK;
}

int prefill_call(const void* q_prompt, const void* k_prompt, const void* v_prompt, const void* k_cache_paged,
                 const void* v_cache_paged, const float* k_scales, const float* v_scales, const uint32_t* page_table,
                 const int32_t* context_lens, void* out, int dtype, int64_t num_query_rows, int64_t num_seqs,
                 int num_q_heads, int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages,
                 int64_t page_table_width, hipStream_t stream) {
  const char* op = "paged_attention_prefill";
  // 16-bit pools: any page size that is a multiple of 8 (the reference
  // prefill reads it at run time); fp8 pools: 16 or 32
  int st = check_attention_dims(op, dtype, num_q_heads, num_kv_heads, head_dim, tokens_per_page, num_pages,
                                page_table_width, k_scales == nullptr && v_scales == nullptr);
  if (st != PAL_OK) return st;
  st = check_fp8_scales(op, k_scales, v_scales, head_dim);
  if (st != PAL_OK) return st;
  if (num_query_rows < 0 || num_seqs < 0) return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] negative dimension", op);
  if (head_dim % 32 != 0)
    return fail(PAL_ERR_RUNTIME, "[%s] head_dim %d must be divisible by 32", op, head_dim);
  if (!prefill_head_dim_supported(head_dim))
    return fail(PAL_ERR_RUNTIME, "[%s] no kernel for head_dim %d (supported: 32, 64, 96, 128, 256)", op, head_dim);
  if (num_seqs == 0) return ok();
  if (num_pages == 0) page_table_width = 0;  // no page to read: no history
  const int64_t prompt_len = num_query_rows / num_seqs;
  if (prompt_len == 0) return ok();
  if (!q_prompt || !k_prompt || !v_prompt || !context_lens || !out ||
      (num_pages > 0 && (!k_cache_paged || !v_cache_paged)) || (page_table_width > 0 && !page_table))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] null pointer argument", op);
  if (!aligned16(q_prompt) || !aligned16(k_prompt) || !aligned16(v_prompt) || !aligned16(k_cache_paged) ||
      !aligned16(v_cache_paged) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] inputs must be 16-byte aligned, out 8-byte aligned", op);
  const int group = num_q_heads / num_kv_heads;
  const int hg_max = group < 16 ? group : 16;
  const int qt = pal::prefill_tokens_per_tile(group);
  const int64_t tiles = num_seqs * ((prompt_len + qt - 1) / qt);
  if (tiles * num_kv_heads * ((group + 15) / 16) > 0x7fffffffLL || num_query_rows > 0x7fffffffLL)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] problem too large for one call", op);
  pal::PrefillParams p;
  p.q = static_cast<const uint16_t*>(q_prompt);
  p.out = static_cast<uint16_t*>(out);
  p.k_pool = static_cast<const uint16_t*>(k_cache_paged);
  p.v_pool = static_cast<const uint16_t*>(v_cache_paged);
  p.k_scales = k_scales;
  p.v_scales = v_scales;
  p.k_dense = static_cast<const uint16_t*>(k_prompt);
  p.v_dense = static_cast<const uint16_t*>(v_prompt);
  p.page_table = page_table;
  p.seq_lens = context_lens;
  p.q_offset = nullptr;
  p.q2seq = nullptr;
  p.num_rows = num_query_rows;
  p.num_seqs = num_seqs;
  p.num_pages = num_pages;
  p.page_table_width = page_table_width;
  p.num_units = static_cast<int>(tiles);
  p.prompt_len = static_cast<int>(prompt_len);
  p.tokens_per_page = tokens_per_page;
  p.num_q_heads = num_q_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = group;
  p.head_chunks = (group + 15) / 16;
  p.hg_max = hg_max;
  p.scale_log2 = scale_log2_for(head_dim);
  p.scale_inv_log2 = 1.f / p.scale_log2;
  PAL_LOG("%s rows=%lld seqs=%lld P=%d Hq=%d Hkv=%d HD=%d TPP=%d dtype=%d fp8=%d tiles=%d stream=%p", op,
          static_cast<long long>(num_query_rows), static_cast<long long>(num_seqs), p.prompt_len, num_q_heads,
          num_kv_heads, head_dim, tokens_per_page, dtype, k_scales ? 1 : 0, p.num_units, static_cast<void*>(stream));
  return hip_status(pal::launch_prefill(p, dtype, head_dim, tokens_per_page, stream), op);
}

size_t fused_workspace_size(int dtype, int64_t num_query_rows, int num_q_heads, int num_kv_heads, int head_dim,
                            int tokens_per_page, bool kv8) {
  if (!valid_dtype(dtype) || num_query_rows <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0 || !prefill_head_dim_supported(head_dim) ||
      (tokens_per_page != 16 && tokens_per_page != 32) || num_query_rows > 0x7fffffffLL)
    return 0;
  if (kv8 && head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
  const int group = num_q_heads / num_kv_heads;
  int resident = 0;
  int64_t vw = 0;
  if (decode_workers(dtype, head_dim, tokens_per_page, num_query_rows, num_kv_heads, (group + 15) / 16, 0, 0,
                     pal::fused_shares_cu(head_dim), kv8, &resident, &vw) != PAL_OK)
    return 0;
  return decode_layout(num_query_rows, head_dim, group < 16 ? group : 16, vw).total;
}

int fused_call(const void* queries, const void* k_pool, const void* v_pool, const float* k_scales,
               const float* v_scales, const uint32_t* page_table, const int32_t* sequence_lengths,
               const uint32_t* query_to_seq_map, const int32_t* query_token_offset, void* out, int dtype,
               int64_t num_query_rows, int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
               int tokens_per_page, int64_t num_pages, int64_t page_table_width, void* workspace,
               size_t workspace_bytes, hipStream_t hs) {
  const char* op = "paged_attention";
  int st = check_attention_dims(op, dtype, num_q_heads, num_kv_heads, head_dim, tokens_per_page, num_pages,
                                page_table_width);
  if (st != PAL_OK) return st;
  st = check_fp8_scales(op, k_scales, v_scales, head_dim);
  if (st != PAL_OK) return st;
  const bool kv8 = k_scales != nullptr;
  if (num_query_rows < 0 || num_seqs < 0) return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] negative dimension", op);
  if (!prefill_head_dim_supported(head_dim))
    return fail(PAL_ERR_RUNTIME, "[%s] no kernel for head_dim %d (supported: 32, 64, 96, 128, 256)", op, head_dim);
  if (num_query_rows > 0x7fffffffLL || num_seqs > 0x7fffffffLL)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] problem too large for one call", op);
  if (num_query_rows == 0) return ok();
  if (num_pages == 0) page_table_width = 0;  // no page to read: every row is empty
  if (!queries || !sequence_lengths || !query_to_seq_map || !query_token_offset || !out ||
      (num_pages > 0 && (!k_pool || !v_pool)) || (page_table_width > 0 && !page_table))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] null pointer argument", op);
  if (!aligned16(queries) || !aligned16(k_pool) || !aligned16(v_pool) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] queries and pools must be 16-byte aligned, out 8-byte aligned", op);
  const int group = num_q_heads / num_kv_heads;
  const int hg_max = group < 16 ? group : 16;
  const int chunks = (group + 15) / 16;
  int resident = 0;
  int64_t vw = 0;
  st = decode_workers(dtype, head_dim, tokens_per_page, num_query_rows, num_kv_heads, chunks, 0, 0,
                      pal::fused_shares_cu(head_dim), kv8, &resident, &vw);
  if (st != PAL_OK) return st;
  const DecodeLayout lay = decode_layout(num_query_rows, head_dim, hg_max, vw);
  if (workspace == nullptr || workspace_bytes < lay.total)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] workspace of %zu bytes needed, %zu given", op, lay.total,
                workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] workspace must be 256-byte aligned", op);
  const int qt = pal::prefill_tokens_per_tile(group);
  const int64_t windows = (num_query_rows + qt - 1) / qt;
  if (windows * num_kv_heads * chunks > 0x7fffffffLL)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] problem too large for one call", op);

  // 1. runs of rows of one sequence: MFMA tiles over windows of rows
  pal::PrefillParams pp;
  pp.q = static_cast<const uint16_t*>(queries);
  pp.out = static_cast<uint16_t*>(out);
  pp.k_pool = static_cast<const uint16_t*>(k_pool);
  pp.v_pool = static_cast<const uint16_t*>(v_pool);
  pp.k_scales = k_scales;
  pp.v_scales = v_scales;
  pp.k_dense = nullptr;
  pp.v_dense = nullptr;
  pp.page_table = page_table;
  pp.seq_lens = sequence_lengths;
  pp.q_offset = query_token_offset;
  pp.q2seq = query_to_seq_map;
  pp.num_rows = num_query_rows;
  pp.num_seqs = num_seqs;
  pp.num_pages = num_pages;
  pp.page_table_width = page_table_width;
  pp.num_units = static_cast<int>(windows);
  pp.prompt_len = 0;
  pp.tokens_per_page = tokens_per_page;
  pp.num_q_heads = num_q_heads;
  pp.num_kv_heads = num_kv_heads;
  pp.group = group;
  pp.head_chunks = chunks;
  pp.hg_max = hg_max;
  pp.scale_log2 = scale_log2_for(head_dim);
  pp.scale_inv_log2 = 1.f / pp.scale_log2;
  // 2. rows alone in their run: split-K decode
  pal::DecodeParams dp = decode_params(queries, k_pool, v_pool, page_table, sequence_lengths, out,
                                       static_cast<char*>(workspace), lay, num_query_rows, num_pages,
                                       page_table_width, num_q_heads, num_kv_heads, head_dim, resident, 0);
  dp.k_scales = k_scales;
  dp.v_scales = v_scales;
  dp.q2seq = query_to_seq_map;
  dp.q_offset = query_token_offset;
  dp.num_pt_rows = num_seqs;

  PAL_LOG("%s rows=%lld seqs=%lld Hq=%d Hkv=%d HD=%d TPP=%d dtype=%d fp8=%d windows=%lld decode_workers=%d stream=%p",
          op, static_cast<long long>(num_query_rows), static_cast<long long>(num_seqs), num_q_heads, num_kv_heads,
          head_dim, tokens_per_page, dtype, kv8 ? 1 : 0, static_cast<long long>(windows), resident,
          static_cast<void*>(hs));
  return hip_status(pal::launch_fused(dp, pp, dtype, head_dim, tokens_per_page, hs), op);
}

// pal_paged_attention_decode and its no-allocation variant: with
// use_scratch the workspace is the library's per-device scratch array (no
// caller buffer, nothing allocated), and calls needing more than it holds
// are rejected.
int decode_call(const void* queries, const void* k_pool, const void* v_pool, const float* k_scales,
                const float* v_scales, const uint32_t* page_table, const int32_t* sequence_lengths, void* out,
                int dtype, int64_t num_query_rows, int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                int tokens_per_page, int64_t num_pages, int64_t page_table_width, int partition_size,
                void* workspace, size_t workspace_bytes, bool use_scratch, hipStream_t stream) {
  const bool kv8 = k_scales != nullptr || v_scales != nullptr;
  if (kv8 && (!k_scales || !v_scales))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] fp8 pools need both k_scales and v_scales");
  if (kv8 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(PAL_ERR_RUNTIME, "[paged_attention_decode] no fp8 kernel for head_dim %d (supported: 64, 128, 256)",
                head_dim);
  if (!valid_dtype(dtype))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] unsupported dtype code %d", dtype);
  if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || tokens_per_page <= 0 ||
      num_pages < 0 || page_table_width < 0)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] negative or zero dimension");
  if (num_q_heads % num_kv_heads != 0)
    return fail(PAL_ERR_RUNTIME, "num_q_heads must be divisible by num_kv_heads (%d %% %d != 0)",
                num_q_heads, num_kv_heads);
  if (!decode_head_dim_supported(head_dim))
    return fail(PAL_ERR_RUNTIME, "[paged_attention_decode] no kernel for head_dim %d (supported: 32, 64, 80, 96, 128, 256)", head_dim);
  if (tokens_per_page != 16 && tokens_per_page != 32)
    return fail(PAL_ERR_RUNTIME, "[paged_attention_decode] no kernel for tokens_per_page %d (supported: 16, 32)", tokens_per_page);
  if (!decode_partition_ok(partition_size))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] partition_size %d not in {0, 128, 256, 512}",
                partition_size);
  if (num_query_rows < num_seqs)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] %lld query rows for %lld sequences",
                static_cast<long long>(num_query_rows), static_cast<long long>(num_seqs));
  if (num_seqs == 0) return ok();
  if (num_pages == 0) page_table_width = 0;  // no page to read: every sequence is empty
  const int group = num_q_heads / num_kv_heads;
  const int chunks = (group + 15) / 16;
  const int hg_max = group < 16 ? group : 16;
  int resident = 0;
  int64_t vw = 0;
  const int st = decode_workers(dtype, head_dim, tokens_per_page, num_seqs, num_kv_heads, chunks, page_table_width,
                                partition_size, false, kv8, &resident, &vw);
  if (st != PAL_OK) return st;
  const DecodeLayout lay = decode_layout(num_seqs, head_dim, hg_max, vw);
  if (use_scratch) {
    if (lay.total > pal::kScratchBytes)
      return fail(PAL_ERR_INVALID_ARGUMENT,
                  "[paged_attention_decode_noalloc] these shapes need %zu bytes of scratch; the library holds %zu "
                  "per device (use pal_paged_attention_decode with a caller workspace)",
                  lay.total, pal::kScratchBytes);
  }
  if (!queries || !sequence_lengths || !out || (num_pages > 0 && (!k_pool || !v_pool)) ||
      (page_table_width > 0 && !page_table))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] null pointer argument");
  if (!aligned16(queries) || !aligned16(k_pool) || !aligned16(v_pool) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(PAL_ERR_INVALID_ARGUMENT,
                "[paged_attention_decode] queries and pools must be 16-byte aligned, out 8-byte aligned");
  if (use_scratch) {
    const hipError_t err = pal::scratch_buffer(&workspace);
    if (err != hipSuccess) return hip_status(err, "paged_attention_decode_noalloc");
    workspace_bytes = pal::kScratchBytes;
  }
  if (workspace == nullptr || workspace_bytes < lay.total)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] workspace of %zu bytes needed, %zu given",
                lay.total, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] workspace must be 256-byte aligned");

  pal::DecodeParams p = decode_params(queries, k_pool, v_pool, page_table, sequence_lengths, out,
                                      static_cast<char*>(workspace), lay, num_seqs, num_pages, page_table_width,
                                      num_q_heads, num_kv_heads, head_dim, resident, partition_size);
  p.k_scales = k_scales;
  p.v_scales = v_scales;
  PAL_LOG("paged_attention_decode seqs=%lld Hq=%d Hkv=%d HD=%d TPP=%d W=%lld dtype=%d fp8=%d partition=%d "
          "workers=%d virtual=%lld ws=%zu scratch=%d stream=%p",
          static_cast<long long>(num_seqs), num_q_heads, num_kv_heads, head_dim, tokens_per_page,
          static_cast<long long>(page_table_width), dtype, kv8 ? 1 : 0, partition_size, resident,
          static_cast<long long>(vw), lay.total, use_scratch ? 1 : 0, static_cast<void*>(stream));
  return hip_status(pal::launch_decode(p, dtype, head_dim, tokens_per_page, stream),
                    "paged_attention_decode");
}

}  // namespace

extern "C" {

const char* pal_last_error(void) { return pal::last_error(); }

const char* pal_version(void) { return "2025.06.4+gfx950"; }

int pal_get_k_cache_stripe_size(int dtype) {
  if (!valid_pool_dtype(dtype)) return fail(PAL_ERR_INVALID_ARGUMENT, "unsupported dtype code %d", dtype);
  ok();
  return 16 / pool_elem_bytes(dtype);
}

int pal_get_optimal_page_size(void) { return 16; }

int pal_get_k_cache_shape(int64_t num_pages, int num_kv_heads, int head_dim, int tokens_per_page,
                          int dtype, int64_t out_shape[5]) {
  if (!valid_pool_dtype(dtype)) return fail(PAL_ERR_INVALID_ARGUMENT, "unsupported dtype code %d", dtype);
  const int x = 16 / pool_elem_bytes(dtype);
  out_shape[0] = num_pages;
  out_shape[1] = num_kv_heads;
  out_shape[2] = head_dim / x;
  out_shape[3] = tokens_per_page;
  out_shape[4] = x;
  return ok();
}

int pal_get_v_cache_shape(int64_t num_pages, int num_kv_heads, int head_dim, int tokens_per_page,
                          int dtype, int64_t out_shape[4]) {
  if (!valid_pool_dtype(dtype)) return fail(PAL_ERR_INVALID_ARGUMENT, "unsupported dtype code %d", dtype);
  out_shape[0] = num_pages;
  out_shape[1] = num_kv_heads;
  out_shape[2] = head_dim;
  out_shape[3] = tokens_per_page;
  return ok();
}

int pal_fill_kv_pages(const void* new_keys, const void* new_values, void* k_pool, void* v_pool,
                      const uint32_t* page_table, const int32_t* write_positions,
                      const uint32_t* query_to_seq_map, int dtype, int64_t num_tokens,
                      int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages,
                      int64_t num_seqs, int64_t page_table_width, void* stream) {
  if (!valid_dtype(dtype)) return fail(PAL_ERR_INVALID_ARGUMENT, "[fill_kv_pages] unsupported dtype code %d", dtype);
  FillArgs a;
  a.new_keys = new_keys;
  a.new_values = new_values;
  a.src_dtype = dtype;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.kv_dtype = dtype;
  a.page_table = page_table;
  a.write_positions = write_positions;
  a.query_to_seq_map = query_to_seq_map;
  a.num_tokens = num_tokens;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.tokens_per_page = tokens_per_page;
  a.num_pages = num_pages;
  a.num_seqs = num_seqs;
  a.page_table_width = page_table_width;
  return fill_call("fill_kv_pages", a, static_cast<hipStream_t>(stream));
}

int pal_fill_kv_pages_fp8(const void* new_keys, const void* new_values, int src_dtype, void* k_pool, void* v_pool,
                          const float* k_scales, const float* v_scales, const uint32_t* page_table,
                          const int32_t* write_positions, const uint32_t* query_to_seq_map, int64_t num_tokens,
                          int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages, int64_t num_seqs,
                          int64_t page_table_width, void* stream) {
  FillArgs a;
  a.new_keys = new_keys;
  a.new_values = new_values;
  a.src_dtype = src_dtype;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.kv_dtype = PAL_DTYPE_FP8_E4M3;
  a.k_scales = k_scales;
  a.v_scales = v_scales;
  a.page_table = page_table;
  a.write_positions = write_positions;
  a.query_to_seq_map = query_to_seq_map;
  a.num_tokens = num_tokens;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.tokens_per_page = tokens_per_page;
  a.num_pages = num_pages;
  a.num_seqs = num_seqs;
  a.page_table_width = page_table_width;
  return fill_call("fill_kv_pages_fp8", a, static_cast<hipStream_t>(stream));
}

int pal_rope_fill_kv_pages(const void* new_keys, const void* new_values, int src_dtype, void* k_pool, void* v_pool,
                           int kv_dtype, const float* k_scales, const float* v_scales, const uint32_t* page_table,
                           const int32_t* write_positions, const uint32_t* query_to_seq_map, int64_t num_tokens,
                           int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages, int64_t num_seqs,
                           int64_t page_table_width, const float* cos_sin_cache, int64_t cos_sin_rows,
                           int rotary_dim, int rope_style, const void* queries, void* queries_out,
                           int num_q_heads, int q_out_dtype, void* stream) {
  FillArgs a;
  a.new_keys = new_keys;
  a.new_values = new_values;
  a.src_dtype = src_dtype;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.kv_dtype = kv_dtype;
  a.k_scales = k_scales;
  a.v_scales = v_scales;
  a.page_table = page_table;
  a.write_positions = write_positions;
  a.query_to_seq_map = query_to_seq_map;
  a.num_tokens = num_tokens;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.tokens_per_page = tokens_per_page;
  a.num_pages = num_pages;
  a.num_seqs = num_seqs;
  a.page_table_width = page_table_width;
  a.cos_sin = cos_sin_cache;
  a.cos_sin_rows = cos_sin_rows;
  a.rotary_dim = rotary_dim;
  a.rope_style = rope_style;
  a.queries = queries;
  a.queries_out = queries_out;
  a.num_q_heads = num_q_heads;
  a.q_out_dtype = q_out_dtype;
  return fill_call("rope_fill_kv_pages", a, static_cast<hipStream_t>(stream));
}

size_t pal_paged_attention_decode_workspace_size(int dtype, int64_t num_seqs, int num_q_heads,
                                                 int num_kv_heads, int head_dim, int tokens_per_page,
                                                 int64_t page_table_width, int partition_size) {
  return decode_workspace_size(dtype, num_seqs, num_q_heads, num_kv_heads, head_dim, tokens_per_page,
                               page_table_width, partition_size, false);
}

size_t pal_paged_attention_decode_fp8_workspace_size(int dtype, int64_t num_seqs, int num_q_heads, int num_kv_heads,
                                                     int head_dim, int tokens_per_page, int64_t page_table_width,
                                                     int partition_size) {
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
  return decode_workspace_size(dtype, num_seqs, num_q_heads, num_kv_heads, head_dim, tokens_per_page,
                               page_table_width, partition_size, true);
}

int pal_paged_attention_decode(const void* queries, const void* k_pool, const void* v_pool,
                               const uint32_t* page_table, const int32_t* sequence_lengths,
                               void* out, int dtype, int64_t num_query_rows, int64_t num_seqs,
                               int num_q_heads, int num_kv_heads, int head_dim,
                               int tokens_per_page, int64_t num_pages, int64_t page_table_width,
                               int partition_size, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return decode_call(queries, k_pool, v_pool, nullptr, nullptr, page_table, sequence_lengths, out, dtype,
                     num_query_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tokens_per_page, num_pages,
                     page_table_width, partition_size, workspace, workspace_bytes, false,
                     static_cast<hipStream_t>(stream));
}

int pal_paged_attention_decode_noalloc(const void* queries, const void* k_pool, const void* v_pool,
                                       const uint32_t* page_table, const int32_t* sequence_lengths, void* out,
                                       int dtype, int64_t num_query_rows, int64_t num_seqs, int num_q_heads,
                                       int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages,
                                       int64_t page_table_width, int partition_size, void* stream) {
  return decode_call(queries, k_pool, v_pool, nullptr, nullptr, page_table, sequence_lengths, out, dtype,
                     num_query_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tokens_per_page, num_pages,
                     page_table_width, partition_size, nullptr, 0, true, static_cast<hipStream_t>(stream));
}

int pal_paged_attention_decode_fp8(const void* queries, const void* k_pool, const void* v_pool,
                                   const float* k_scales, const float* v_scales, const uint32_t* page_table,
                                   const int32_t* sequence_lengths, void* out, int dtype, int64_t num_query_rows,
                                   int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                   int tokens_per_page, int64_t num_pages, int64_t page_table_width,
                                   int partition_size, void* workspace, size_t workspace_bytes, void* stream) {
  if (!k_scales || !v_scales)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_decode] fp8 pools need both k_scales and v_scales");
  return decode_call(queries, k_pool, v_pool, k_scales, v_scales, page_table, sequence_lengths, out, dtype,
                     num_query_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tokens_per_page, num_pages,
                     page_table_width, partition_size, workspace, workspace_bytes, false,
                     static_cast<hipStream_t>(stream));
}

int pal_paged_attention_prefill(const void* q_prompt, const void* k_prompt, const void* v_prompt,
                                const void* k_cache_paged, const void* v_cache_paged, const uint32_t* page_table,
                                const int32_t* context_lens, void* out, int dtype, int64_t num_query_rows,
                                int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                int tokens_per_page, int64_t num_pages, int64_t page_table_width, void* stream) {
  return prefill_call(q_prompt, k_prompt, v_prompt, k_cache_paged, v_cache_paged, nullptr, nullptr, page_table,
                      context_lens, out, dtype, num_query_rows, num_seqs, num_q_heads, num_kv_heads, head_dim,
                      tokens_per_page, num_pages, page_table_width, static_cast<hipStream_t>(stream));
}

int pal_paged_attention_prefill_fp8(const void* q_prompt, const void* k_prompt, const void* v_prompt,
                                    const void* k_cache_paged, const void* v_cache_paged, const float* k_scales,
                                    const float* v_scales, const uint32_t* page_table, const int32_t* context_lens,
                                    void* out, int dtype, int64_t num_query_rows, int64_t num_seqs, int num_q_heads,
                                    int num_kv_heads, int head_dim, int tokens_per_page, int64_t num_pages,
                                    int64_t page_table_width, void* stream) {
  if (!k_scales || !v_scales)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention_prefill] fp8 pools need both k_scales and v_scales");
  return prefill_call(q_prompt, k_prompt, v_prompt, k_cache_paged, v_cache_paged, k_scales, v_scales, page_table,
                      context_lens, out, dtype, num_query_rows, num_seqs, num_q_heads, num_kv_heads, head_dim,
                      tokens_per_page, num_pages, page_table_width, static_cast<hipStream_t>(stream));
}

size_t pal_paged_attention_workspace_size(int dtype, int64_t num_query_rows, int num_q_heads, int num_kv_heads,
                                          int head_dim, int tokens_per_page) {
  return fused_workspace_size(dtype, num_query_rows, num_q_heads, num_kv_heads, head_dim, tokens_per_page, false);
}

size_t pal_paged_attention_fp8_workspace_size(int dtype, int64_t num_query_rows, int num_q_heads, int num_kv_heads,
                                              int head_dim, int tokens_per_page) {
  return fused_workspace_size(dtype, num_query_rows, num_q_heads, num_kv_heads, head_dim, tokens_per_page, true);
}

int pal_paged_attention(const void* queries, const void* k_pool, const void* v_pool, const uint32_t* page_table,
                        const int32_t* sequence_lengths, const uint32_t* query_to_seq_map,
                        const int32_t* query_token_offset, void* out, int dtype, int64_t num_query_rows,
                        int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim, int tokens_per_page,
                        int64_t num_pages, int64_t page_table_width, void* workspace, size_t workspace_bytes,
                        void* stream) {
  return fused_call(queries, k_pool, v_pool, nullptr, nullptr, page_table, sequence_lengths, query_to_seq_map,
                    query_token_offset, out, dtype, num_query_rows, num_seqs, num_q_heads, num_kv_heads, head_dim,
                    tokens_per_page, num_pages, page_table_width, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

int pal_paged_attention_fp8(const void* queries, const void* k_pool, const void* v_pool, const float* k_scales,
                            const float* v_scales, const uint32_t* page_table, const int32_t* sequence_lengths,
                            const uint32_t* query_to_seq_map, const int32_t* query_token_offset, void* out, int dtype,
                            int64_t num_query_rows, int64_t num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                            int tokens_per_page, int64_t num_pages, int64_t page_table_width, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!k_scales || !v_scales)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[paged_attention] fp8 pools need both k_scales and v_scales");
  return fused_call(queries, k_pool, v_pool, k_scales, v_scales, page_table, sequence_lengths, query_to_seq_map,
                    query_token_offset, out, dtype, num_query_rows, num_seqs, num_q_heads, num_kv_heads, head_dim,
                    tokens_per_page, num_pages, page_table_width, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

int pal_copy_pages(void* k_pool, void* v_pool, float* k_scales, float* v_scales, int64_t num_pages, int num_kv_heads,
                   int64_t page_bytes, const uint32_t* src, const uint32_t* dst, int64_t num_moves, void* stream) {
  const char* op = "copy_pages";
  if (num_moves < 0 || num_pages < 0 || num_kv_heads <= 0 || num_kv_heads > 256 || page_bytes <= 0 ||
      page_bytes % 16 != 0)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] bad dimensions (page_bytes must be a positive multiple of 16)", op);
  if (num_moves == 0) return ok();
  if (!k_pool || !v_pool || !src || !dst || (!k_scales != !v_scales))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] null pointer argument", op);
  if (!aligned16(k_pool) || !aligned16(v_pool))
    return fail(PAL_ERR_INVALID_ARGUMENT, "[%s] pools must be 16-byte aligned", op);
  pal::PageCopyParams p;
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.k_scales = k_scales;
  p.v_scales = v_scales;
  p.src = src;
  p.dst = dst;
  p.num_moves = num_moves;
  p.num_pages = num_pages;
  p.page_bytes = page_bytes;
  p.num_kv_heads = num_kv_heads;
  return hip_status(pal::launch_copy_pages(p, static_cast<hipStream_t>(stream)), op);
}

int pal_remap_pages(uint32_t* page_table, int64_t num_entries, const uint32_t* remap, int64_t remap_len,
                    void* stream) {
  if (num_entries < 0 || remap_len < 0)
    return fail(PAL_ERR_INVALID_ARGUMENT, "[remap_pages] negative size");
  if (num_entries == 0) return ok();
  if (!page_table || !remap) return fail(PAL_ERR_INVALID_ARGUMENT, "[remap_pages] null pointer argument");
  return hip_status(pal::launch_remap_pages(page_table, num_entries, remap, remap_len, static_cast<hipStream_t>(stream)),
                    "remap_pages");
}

int pal_debug_flags(int reset, uint32_t* flags) {
  if (!flags) return fail(PAL_ERR_INVALID_ARGUMENT, "[debug_flags] null output");
#ifdef PAL_DEBUG_CHECKS
  uint32_t a = 0, b = 0, c = 0;
  hipError_t err = pal::decode_debug_flags(&a, reset != 0);
  if (err == hipSuccess) err = pal::prefill_debug_flags(&b, reset != 0);
  if (err == hipSuccess) err = pal::fill_debug_flags(&c, reset != 0);
  if (err != hipSuccess) return hip_status(err, "debug_flags");
  *flags = a | b | c;
  return ok();
#else
  (void)reset;
  *flags = 0;
  return fail(PAL_ERR_RUNTIME, "[debug_flags] this library was built without PAL_DEBUG_CHECKS");
#endif
}

}  // extern "C"
