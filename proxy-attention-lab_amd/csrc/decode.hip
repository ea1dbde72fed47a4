// Paged-attention decode for gfx950: the KV stream of the whole batch is split
// into 16-token blocks, shared out to a resident set of wavefront workers
// (equal static shares, or static runs of fixed chunks when a partition size
// is given), and the pieces of sequences that several workers shared are
// merged with a log-sum-exp pass.
//
// Reference behaviour: kernels/paged_attention/decode/paged_attention_decode.h.metal
// (one query row per sequence, GQA map h -> h / (Hq/Hkv) at :64-65, scale
// 1/sqrt(HD) at :115, length mask at :125-131 and :298-306) and the two-pass
// merge of decode/paged_reduce_decode.h.metal:79-128.
//
// Design (MI355X):
//  * Work is the flat list of (sequence, kv head, head chunk) "segments", each
//    a run of 16-token blocks (one page for TPP=16, half a page for TPP=32).
//    All query heads sharing a kv head (up to 16 per chunk) are processed
//    together, so a K/V page block is read from HBM once per GQA group.
//  * The global block list [0, T) is cut into "virtual workers": equal
//    static ranges (one per resident wavefront), or, in the fixed-chunk mode
//    (partition_size > 0), chunks of C blocks, each wavefront streaming a
//    static run of consecutive chunks.  Because the cut is fixed, which
//    wavefront computes a chunk changes nothing in the result.
//  * Each workgroup scans the sequence lengths into LDS (batches of up to
//    1024 sequences; larger ones are scanned once by decode_plan_kernel into
//    the workspace) and locates the sequence of a range by binary search.
//  * A wavefront streams blocks with a software pipeline: the K and V loads
//    of the next PF blocks are in flight while the current block is computed.
//    The K block is read in the pool's striped [HD/8][TPP][8] layout, which is
//    exactly the A operand of v_mfma_f32_16x16x32 for S^T = K * Q^T (lane l
//    loads the 16-byte stripe (l/16 + 4kk) of token l%16: 1 KiB contiguous
//    per instruction).  The result holds head l%16 and tokens 4(l/16)..+3 in
//    lane l, which is the B operand of v_mfma_f32_16x16x16 for
//    O^T = V^T * P^T; V is read as 8-byte runs of 4 tokens from the [HD][TPP]
//    layout as its A operand.  In O^T the head is the lane, so the online
//    softmax rescale is a per-lane multiply.
//  * Row mode (the decode rows of the fused op): item i is query row i of
//    sequence q2seq[i], seeing min(len, q_offset[i]) keys, when the row is
//    alone in its run of same-sequence rows; rows of longer runs belong to
//    the prefill kernel and are skipped here.  Plain decode: item i is query
//    row i of sequence i.
//  * A segment that lies wholly inside one virtual worker writes the
//    normalised output directly.  Split segments leave partials (fp32 max
//    and exp-sum, O / exp-sum in the 16-bit dtype) in one of two slots per
//    virtual worker, combined by decode_merge_kernel.  The worker holding the
//    first piece of a split segment writes it into its own slot of a merge
//    list, so the merge grid does not grow with the batch.
#include <mutex>
#include <unordered_map>

#include "pal_device.h"

namespace pal {

// flag word of this translation unit's debug checks (see pal_device.h)
PAL_DEBUG_FLAGS_DEFINE(decode_debug_flags)

}  // namespace pal

#include "prefill_tile.h"  // the fused kernel's prefill tiles

namespace pal {

namespace {

constexpr int kWorkersPerGroup = 4;  // independent wavefront workers per workgroup
constexpr int kPrefetch = 2;         // blocks whose loads are in flight ahead of the one being computed
constexpr float kLazyMax = 8.f;      // log2 headroom before a decode worker's running max moves

// A K/V load of a 16-token block.  With 32-token pages a block reads half of
// each V row and of each K stripe row of its page, and the next block (the
// same wavefront, one step later) the other half; when a (page, kv head)
// block holds 8 KiB or more (16-bit pools from head dim 128, fp8 pools at
// head dim 256) the loads are cacheable so that half stays in L2 for it
// (config 2's shape over 32-token pages: head dim 128 138 -> 118 us, 256 288
// -> 228 us, fp8 head dim 256 146 -> 126 us); smaller blocks, and 16-token
// pages, whose blocks read whole rows, stream non-temporally.
template <int TPP, int kBlockBytes, typename T>
__device__ __forceinline__ T page_load(const T* p) {
  if constexpr (TPP == 32 && kBlockBytes >= 8192) return *p;
  else return __builtin_nontemporal_load(p);
}
constexpr int kGroupThreads = kWorkersPerGroup * kWave;
constexpr int kPlanThreads = 1024;
constexpr int kInlinePlanSeqs = 1024;  // largest batch scanned into LDS by each workgroup
constexpr int64_t kMergeGroups = 2048;  // merge grid (at most): workgroups stride over the list

struct Item {
  int64_t row;  // query / output row
  int64_t seq;  // page-table row
  int64_t len;  // visible keys, clamped to [0, W * TPP]
  bool skip;    // row mode: a row of a multi-row run (not ours to write)
};

__device__ __forceinline__ Item item_at(const DecodeParams& p, int64_t i, int tpp) {
  Item it;
  int64_t len;
  it.row = i;
  it.skip = false;
  if (p.q2seq) {
    const uint32_t sq = p.q2seq[i];
    it.skip = (i > 0 && p.q2seq[i - 1] == sq) || (i + 1 < p.num_seqs && p.q2seq[i + 1] == sq);
    if (sq < p.num_pt_rows && !it.skip) {
      it.seq = sq;
      len = p.seq_lens[sq];
      const int64_t off = p.q_offset[i];
      len = off < len ? off : len;
    } else {  // no such sequence, or a prefill row: nothing to attend to here
      it.seq = 0;
      len = 0;
    }
  } else {
    it.seq = i;
    len = p.seq_lens[i];
  }
  const int64_t max_tokens = p.page_table_width * tpp;
  PAL_DEBUG_FLAG(len > max_tokens, kDebugLength);
  it.len = len < 0 ? 0 : (len > max_tokens ? max_tokens : len);
  return it;
}

// The fixed cut of the global block list into virtual workers.
// Equal shares: [0, T) split evenly over nws = min(resident workers, T)
// virtual workers (none empty).  Fixed chunks: nc chunks of `chunk` blocks,
// virtual ids nws + k with nws = 0.  (A dynamically claimed tail of chunks
// after static shares measured much slower: each claimed range restarts the
// load pipeline and writes its own partials.)
struct Sched {
  int64_t total;  // T: blocks of all segments
  int64_t ts;     // static region [0, ts), split evenly over nws workers
  int64_t nws;    // static virtual workers
  int64_t chunk;  // blocks per chunk
  int64_t nc;     // chunks covering [ts, total); virtual ids nws .. nws + nc - 1
};

__device__ __forceinline__ Sched make_sched(int64_t total, int64_t nw, int tokens_per_worker) {
  Sched sc;
  sc.total = total;
  if (tokens_per_worker <= 0) {  // equal shares: no division on the start-up path
    sc.ts = total;
    sc.chunk = 1;
    sc.nws = total < nw ? total : nw;
    sc.nc = 0;
    return sc;
  }
  // fixed-size chunks (the reference's CHUNK_SIZE mode)
  sc.ts = 0;
  sc.chunk = tokens_per_worker / 16 > 0 ? tokens_per_worker / 16 : 1;
  sc.nws = 0;
  sc.nc = (total + sc.chunk - 1) / sc.chunk;
  return sc;
}

// First global block of virtual worker v (v in [0, nws + nc]); every virtual
// worker owns at least one block.
__device__ __forceinline__ int64_t vstart(const Sched& sc, int64_t v) {
  if (v <= sc.nws) return sc.nws > 0 ? (v * sc.ts) / sc.nws : 0;
  const int64_t b = sc.ts + (v - sc.nws) * sc.chunk;
  return b < sc.total ? b : sc.total;
}

// Virtual worker whose range holds global block b.
__device__ __forceinline__ int64_t vworker_of(const Sched& sc, int64_t b) {
  if (b < sc.ts) return ((b + 1) * sc.nws + sc.ts - 1) / sc.ts - 1;
  return sc.nws + (b - sc.ts) / sc.chunk;
}

// Zeros for every head of an empty item (no visible key).  Run by the
// planner's thread that finds the item; such items are rare.
template <int HD>
__device__ __forceinline__ void zero_item_output(const DecodeParams& p, int64_t row) {
  u32x2* o = reinterpret_cast<u32x2*>(p.out + row * p.num_q_heads * HD);  // out is 8-byte aligned
  const int64_t n = static_cast<int64_t>(p.num_q_heads) * HD / 4;
  for (int64_t i = 0; i < n; ++i) o[i] = u32x2{0u, 0u};
}

// Sequence holding global block b: the largest s with cum[s] <= b.
__device__ __forceinline__ int64_t locate_seq(const int64_t* cum, int64_t num_seqs, int64_t b) {
  int64_t lo = 0, hi = num_seqs - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (cum[mid] <= b) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Scan for batches larger than kInlinePlanSeqs: cum[s] = first global block of
// sequence s (all of its segments), cum[S] = hdr[0] = T.  Each thread takes
// kPlanPer consecutive items per pass, so their length loads go out together;
// it also writes the zeros of an empty item.
constexpr int kPlanPer = 16;

template <int HD, int TPP>
__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(const DecodeParams p) {
  __shared__ int64_t wave_sums[kPlanThreads / kWave];
  __shared__ int64_t carry_sh;
  const int64_t segs = static_cast<int64_t>(p.num_kv_heads) * p.head_chunks;
  const int tid = threadIdx.x;
  int64_t carry = 0;
  const int64_t n = p.num_seqs;
  for (int64_t base = 0; base < n; base += static_cast<int64_t>(kPlanThreads) * kPlanPer) {
    int64_t vals[kPlanPer];
    int64_t tsum = 0;
#pragma unroll
    for (int k = 0; k < kPlanPer; ++k) {
      const int64_t s = base + static_cast<int64_t>(tid) * kPlanPer + k;
      vals[k] = 0;
      if (s < n) {
        const Item it = item_at(p, s, TPP);
        vals[k] = ((it.len + 15) >> 4) * segs;
        if (it.len == 0 && !it.skip) zero_item_output<HD>(p, it.row);
      }
      tsum += vals[k];
    }
    const int64_t inc = block_inclusive_scan<kPlanThreads>(tsum, wave_sums);
    int64_t c = carry + inc - tsum;
#pragma unroll
    for (int k = 0; k < kPlanPer; ++k) {
      const int64_t s = base + static_cast<int64_t>(tid) * kPlanPer + k;
      if (s < n) p.cum[s] = c;
      c += vals[k];
    }
    if (tid == kPlanThreads - 1) carry_sh = inc;
    __syncthreads();
    carry += carry_sh;
    __syncthreads();
  }
  if (tid == 0) {
    p.cum[n] = carry;
    p.hdr[0] = carry;
  }
}

// Item table of the in-LDS plan: length and page-table row of every item,
// so a wavefront finds its next piece without a global round trip.
struct ItemLds {
  const int64_t* len;  // null: read items from global memory (item_at)
  const int32_t* seq;
  const int32_t* row;  // query / output row of each item (null: item s is row s)
};

// Streams the blocks of virtual workers v_begin .. v_end-1 (one wavefront;
// consecutive virtual workers own consecutive block ranges), with the loads
// of PF blocks in flight ahead of the one being computed.  The blocks form a
// run of pieces (the blocks of one segment inside one virtual worker's
// range); the pipeline runs through piece boundaries, including those
// between virtual workers: while the last blocks of a piece are computed,
// the first blocks of the next piece are already loading (its item, query
// and first page ids were fetched when the piece before it started).
template <int DT, int HD, int TPP, int PF, bool kMultiV, bool KV8>
__device__ __forceinline__ void process_range(const DecodeParams& p, const Sched& sc, const int64_t* cum,
                                              const ItemLds il, int64_t n_items, int64_t v_begin,
                                              int64_t v_end) {
  constexpr bool kK32 = (HD % 32) == 0;  // QK k-step of 32 (else 16)
  constexpr int KK = kK32 ? HD / 32 : HD / 16;
  constexpr int NT = HD / 16;            // output tiles of 16 dims
  constexpr int NBUF = PF + 1;
  // fp8 pools: a K stripe is 16 dims of one token (16 bytes); lane group g
  // loads stripes g + 4j, j < KL8, each feeding two k-steps of 8 dims
  constexpr int EB = KV8 ? 1 : 2;        // pool element bytes
  constexpr int KL8 = HD / 64;
  static_assert(!KV8 || (HD % 64 == 0), "fp8 pools: head_dim a multiple of 64");

  const int64_t b0 = vstart(sc, v_begin);
  const int64_t b_end = vstart(sc, v_end);
  // merge-list slot of each virtual worker: written exactly once per call
  // (the split segment whose first piece ends its range, or none), so the
  // slot never depends on what an earlier call left in the workspace
  int64_t list_g0 = -1, list_nb = 0, list_row = 0, list_seg = 0;  // g0 < 0: nothing to merge
  auto write_list = [&](int64_t v) {
    if (lane_id() == 0 && v < p.list_cap) {
      int64_t* slot = p.split_list + 4 * v;
      slot[0] = list_g0;
      slot[1] = list_nb;
      slot[2] = list_row;
      slot[3] = list_seg;
    }
  };
  if (b_end - b0 <= 0) {
    for (int64_t v = v_begin; v < v_end; ++v) write_list(v);
    return;
  }

  const int lane = lane_id();
  const int g = lane >> 4;
  const int r16 = lane & 15;
  const int segs = p.num_kv_heads * p.head_chunks;
  const int64_t head_block = static_cast<int64_t>(HD) * TPP * EB;  // bytes per (page, kv head)
  const int64_t page_stride = head_block * p.num_kv_heads;

  // A piece: item s (query row s of page-table row `seq`, `len` keys, nb
  // blocks per segment), segment `seg`, blocks [blk, blk + count) of the
  // segment, starting at global block gpos and ending at the latest at END
  // (its virtual worker's range end); r = block offset of the piece inside
  // the item's segments.  c_* is the piece being computed, x_* the
  // next one (kept in scalars: the pipeline state must stay in registers).
  int64_t c_s, c_r, c_gpos, c_seq, c_len, c_nb, c_blk, c_count;
  int c_seg;
  int64_t x_s, x_r, x_gpos, x_seq, x_len, x_nb, x_blk, x_count;
  int x_seg;
  // the piece at item s, offset r, global block gpos (items with no key
  // have no blocks and are skipped)
#define PAL_FIND_PIECE(P, S0, R0, G0, END)                                                         \
  do {                                                                                             \
    int64_t s_ = (S0), r_ = (R0), len_, seq_;                                                      \
    for (;;) {                                                                                     \
      if (il.len) {                                                                                \
        len_ = il.len[s_];                                                                         \
        seq_ = il.seq[s_];                                                                         \
      } else {                                                                                     \
        const Item it_ = item_at(p, s_, TPP);                                                      \
        len_ = it_.len;                                                                            \
        seq_ = it_.seq;                                                                            \
      }                                                                                            \
      if (len_ > 0) break;                                                                         \
      ++s_;                                                                                        \
      r_ = 0;                                                                                      \
    }                                                                                              \
    P##s = s_;                                                                                     \
    P##r = r_;                                                                                     \
    P##gpos = (G0);                                                                                \
    P##seq = seq_;                                                                                 \
    P##len = len_;                                                                                 \
    P##nb = (len_ + 15) >> 4;                                                                      \
    P##seg = static_cast<int>(r_ / P##nb);                                                         \
    P##blk = r_ - P##seg * P##nb;                                                                  \
    P##count = (P##nb - P##blk) < ((END) - P##gpos) ? (P##nb - P##blk) : ((END) - P##gpos);         \
  } while (0)

  // Q^T operand of a piece: lane holds Q[head r16][k-slice of this lane]
  // (padding heads zeroed).
  u32x4 qv4[kK32 ? KK : 1], qn4[kK32 ? KK : 1];
  u32x2 qv2[kK32 ? 1 : KK], qn2[kK32 ? 1 : KK];
  auto load_q = [&](int64_t s, int seg, u32x4 (&q4)[kK32 ? KK : 1], u32x2 (&q2)[kK32 ? 1 : KK]) {
    const int h0 = (seg % p.head_chunks) * 16;
    const int hg = min(16, p.group - h0);
    const int qh_base = (seg / p.head_chunks) * p.group + h0;
    const bool hv = r16 < hg;
    const uint32_t qmask = hv ? 0xFFFFFFFFu : 0u;
    const int64_t qr = il.row ? static_cast<int64_t>(il.row[s]) : s;
    const uint16_t* qrow = p.q + (qr * p.num_q_heads + qh_base + (hv ? r16 : 0)) * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if constexpr (KV8) {  // k-step kk = (stripe j = kk / 2, half): dims 16 (g + 4j) + 8 half .. +7
        q4[kk] = *reinterpret_cast<const u32x4*>(qrow + 16 * (g + 4 * (kk >> 1)) + 8 * (kk & 1)) & qmask;
      } else if constexpr (kK32) {
        q4[kk] = *reinterpret_cast<const u32x4*>(qrow + 32 * kk + 8 * g) & qmask;
      } else {
        q2[kk] = *reinterpret_cast<const u32x2*>(qrow + 16 * kk + 4 * g) & qmask;
      }
    }
  };
  // page ids of window wi (64 pages, one per lane) of a piece
  auto load_window = [&](int64_t seq, int64_t blk, int64_t wi) {
    const uint32_t* pt = p.page_table + seq * p.page_table_width;
    int64_t lp = (blk * 16) / TPP + wi * kWave + lane;
    if (lp >= p.page_table_width) lp = p.page_table_width - 1;
    return pt[lp];
  };

  int64_t c_v = v_begin, c_vend = vstart(sc, v_begin + 1);  // virtual worker of the piece, its range end
  int64_t x_v = c_v, x_vend = c_vend;
  {
    const int64_t s0 = locate_seq(cum, n_items, b0);  // the item holding block b0 (it has blocks)
    PAL_FIND_PIECE(c_, s0, b0 - cum[s0], b0, c_vend);
  }
  load_q(c_s, c_seg, qv4, qv2);
  // fp8 pools: the query as fp8 terms, the B operand of the fp8 MFMA
  QueryFp8<DT, KV8 ? KK : 1> q8;
  if constexpr (KV8) query_to_fp8<DT, KK>(qv4, q8);

  // Page ids in register windows of 64 pages (one id per lane): pid_cur
  // holds window wcur, the window of the block being computed, and pid_nxt
  // window wcur+1 (the loads run at most a few blocks ahead).  Every step
  // group also loads window wcur+2 (unconditionally, so the vector-memory
  // stream of the loop is the same every time and the compiler's counted
  // waits stay exact); when the computed block enters window wcur+1 the
  // windows move up by one, taking the window wcur+2 loaded a step group
  // earlier.
  int wcur = 0;
  uint32_t pid_cur = load_window(c_seq, c_blk, 0), pid_nxt = load_window(c_seq, c_blk, 1),
           pid_later = load_window(c_seq, c_blk, 2);

  u32x4 kb4[NBUF][KV8 ? KL8 : (kK32 ? KK : 1)];
  u32x2 kb2[NBUF][kK32 ? 1 : KK];
  u32x2 vb[NBUF][KV8 ? 1 : NT];
  u32x4 vq8[NBUF][KV8 ? NT / 4 : 1];
  float bks[NBUF], bvs[NBUF];  // fp8: the block's (page, kv head) scales
  bool bv[NBUF];

  bool first = true;     // the piece is its virtual worker's first
  bool prologue = true;  // the pipeline is empty
  bool has_next = false;
  x_s = c_s; x_r = c_r; x_gpos = c_gpos; x_seq = c_seq; x_len = c_len; x_nb = c_nb; x_blk = c_blk;
  x_count = c_count; x_seg = c_seg;
  uint32_t pidn0 = 0;  // window 0 of the next piece (a load in flight)
  // pidn0 once it has arrived: a copy made after the exact wait at the end of
  // a step group, so the issues of later groups select from it without
  // waiting on the load
  uint32_t pidn0_ready = 0;

  for (;;) {
    const int kvh = c_seg / p.head_chunks;
    const int h0 = (c_seg % p.head_chunks) * 16;
    const int hg = min(16, p.group - h0);
    const int qh_base = kvh * p.group + h0;
    const bool complete = (c_blk == 0) && (c_count == c_nb);
    // positions inside a piece fit 32 bits (a sequence holds fewer than 2^31
    // keys), so the per-block bookkeeping is 32-bit arithmetic
    const int len = static_cast<int>(c_len);
    const int n_blk = static_cast<int>(c_count);
    const int n_pad = (n_blk + NBUF - 1) / NBUF * NBUF;  // steps of the piece
    const int bstart = static_cast<int>(c_blk);        // first block of the piece
    const int pbase = (bstart * 16) / TPP;             // its page index
    const uint8_t* kbase = static_cast<const uint8_t*>(p.k_pool) + kvh * head_block;
    const uint8_t* vbase = static_cast<const uint8_t*>(p.v_pool) + kvh * head_block;
    const uint8_t* kbase_n = kbase;  // set once the next piece is known
    const uint8_t* vbase_n = vbase;
    int kvh_n = kvh;
    int nblk_n = 1;
    int bstart_n = 0, pbase_n = 0;  // first block of the next piece and its page index

    // Issue the K and V loads of step i of the piece into buffer `buf`:
    // block i of the piece (clamped to its last block), or, past the
    // piece's steps, block i - n_pad of the next piece (counted from its
    // first block bstart_n: block 0 of its segment, or a chunk boundary in
    // the fixed-chunk mode).  An out-of-range page id is replaced by page
    // 0 (in bounds) and the block is masked out when computed.  Every K/V
    // block is read exactly once per call, so the loads carry the
    // non-temporal hint: the stream does not displace other lines (page ids,
    // partials, the fused op's prefill tiles) from L2 and MALL.
    auto issue = [&](int i, int buf, uint32_t w_n0) {
      const bool to_next = has_next && i >= n_pad;
      const int j = to_next ? (i - n_pad < nblk_n - 1 ? i - n_pad : nblk_n - 1) : (i < n_blk - 1 ? i : n_blk - 1);
      const int b = (to_next ? bstart_n : bstart) + j;
      const int e = (b * 16) / TPP - (to_next ? pbase_n : pbase);  // page within the piece's windows
      // (selects of values, not of variables: a select of two variables'
      // addresses would push the whole pipeline state to scratch)
      const uint32_t w_c = pid_cur, w_x = pid_nxt;
      const uint32_t win = to_next ? w_n0 : ((e >> 6) == wcur ? w_c : w_x);
      const uint32_t pg = __builtin_amdgcn_readlane(win, static_cast<int>(e & 63));
      bv[buf] = pg < p.num_pages;
      PAL_DEBUG_FLAG(!bv[buf] && (to_next ? i - n_pad < nblk_n : i < n_blk), kDebugPageId);
      const uint32_t page = bv[buf] ? pg : 0u;
      const int slot0 = static_cast<int>((b * 16) % TPP);
      const uint8_t* kb_x = kbase_n;
      const uint8_t* vb_x = vbase_n;
      const uint8_t* kp = (to_next ? kb_x : kbase) + static_cast<int64_t>(page) * page_stride;
      const uint8_t* vp = (to_next ? vb_x : vbase) + static_cast<int64_t>(page) * page_stride + (slot0 + 4 * g) * EB;
      if constexpr (KV8) {
        const int kvh_b = to_next ? kvh_n : kvh;
        const int64_t si = static_cast<int64_t>(page) * p.num_kv_heads + kvh_b;
        bks[buf] = p.k_scales[si];
        bvs[buf] = p.v_scales[si];
#pragma unroll
        for (int j = 0; j < KL8; ++j) {
          const int c = g + 4 * j;  // stripe of dims 16c .. 16c+15
          kb4[buf][j] =
              page_load<TPP, HD * TPP * EB>(reinterpret_cast<const u32x4*>(kp + (c * TPP + slot0 + r16) * 16));
        }
        // V: lane 16g + i reads the block's 16 codes of dim row 64q + 16g + i
        // (one 16-byte load per 64 rows instead of four 4-byte ones); compute
        // transposes them across the lane groups
        const uint8_t* vrow = (to_next ? vb_x : vbase) + static_cast<int64_t>(page) * page_stride + slot0;
#pragma unroll
        for (int q = 0; q < NT / 4; ++q)
          vq8[buf][q] =
              page_load<TPP, HD * TPP * EB>(reinterpret_cast<const u32x4*>(vrow + (64 * q + 16 * g + r16) * TPP));
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          if constexpr (kK32) {
            const int c = 4 * kk + g;  // stripe holding dims 32kk + 8g .. +7
            kb4[buf][kk] =
                page_load<TPP, HD * TPP * EB>(reinterpret_cast<const u32x4*>(kp + (c * TPP + slot0 + r16) * 16));
          } else {
            const int d = 16 * kk + 4 * g;  // dims d .. d+3
            kb2[buf][kk] = page_load<TPP, HD * TPP * EB>(
                reinterpret_cast<const u32x2*>(kp + (((d >> 3) * TPP + slot0 + r16) * 8 + (d & 7)) * 2));
          }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n)
          vb[buf][n] =
              page_load<TPP, HD * TPP * EB>(reinterpret_cast<const u32x2*>(vp + (16 * n + r16) * TPP * 2));
      }
    };

    float m_run = -INFINITY;  // running max of head r16, in log2 units (score * scale_log2)
    float l_run = 0.f;        // this lane's share of the exp-sum of head r16
    f32x4 o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int i, int buf) {
      const int b = bstart + i;
      const bool live = bv[buf] && i < n_blk;  // steps past the piece end are fully masked
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (KV8) {
        // the K codes as loaded are the A operand (stripes g + 8m and
        // g + 8m + 4, 32 bytes), the query's fp8 terms the B operand
#pragma unroll
        for (int m = 0; m < q8.kOps; ++m) {
          const u32x4 a0 = kb4[buf][2 * m];
          const u32x4 a1 = 2 * m + 1 < KL8 ? kb4[buf][2 * m + 1] : u32x4{0u, 0u, 0u, 0u};
          const i32x8 a = {static_cast<int>(a0.x), static_cast<int>(a0.y), static_cast<int>(a0.z),
                           static_cast<int>(a0.w), static_cast<int>(a1.x), static_cast<int>(a1.y),
                           static_cast<int>(a1.z), static_cast<int>(a1.w)};
#pragma unroll
          for (int t = 0; t < q8.kTerms; ++t) acc = mma_fp8_16x16x128(a, q8.w[t][m], acc, q8.s_hi - 4 * t);
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          if constexpr (kK32) {
            acc = Dt<DT>::mma16x16x32(kb4[buf][kk], qv4[kk], acc);
          } else {
            acc = Dt<DT>::mma16x16x16(kb2[buf][kk], qv2[kk], acc);
          }
        }
      }
      // scores in log2 units (fp8: with the block's K scale in the same
      // multiply), so each exponent below is score - max: exactly 0 for the
      // max key whatever the scores' size (an fma of score * scale_log2
      // against a rounded max * scale_log2 leaves that product's rounding
      // error, which overflows exp2 once scores pass ~2^31)
      acc *= KV8 ? bks[buf] * p.scale_log2 : p.scale_log2;
      // tokens past the end (and whole invalid blocks) are masked: token
      // 4g + e of the block is a key when e < kl (the block's key count is
      // uniform, so the 64-bit part is scalar)
      const int left = live ? len - b * 16 : 0;
      const int kl = static_cast<int>(left < 16 ? left : 16) - 4 * g;
      float sc4[4];
      float bm = -INFINITY;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sc4[e] = e < kl ? acc[e] : -INFINITY;
        bm = fmaxf(bm, sc4[e]);
      }
      // The running max of a head moves only when one of its scores passes it
      // by more than kLazyMax (log2 units), so a block's exponents stay below
      // 2^kLazyMax and the max over the 4 lane groups and the rescale run
      // only then; otherwise the block pays one wavefront-uniform test.
      if (__ballot(bm > m_run + kLazyMax)) {  // (always for a head's first key: m_run = -inf)
        const float m_new = fmaxf(m_run, max_xor32(max_xor16(bm)));  // scores are finite or -inf
        // a head with no key yet has l = 0 and O = 0 (alpha 0 keeps them so)
        const float alpha = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int n = 0; n < NT; ++n) o[n] *= alpha;
        m_run = m_new;
      }
      const float mref = (m_run == -INFINITY) ? 0.f : m_run;  // a head with no key yet: every exponent is -inf
      float pe[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pe[e] = __builtin_amdgcn_exp2f(sc4[e] - mref);
        l_run += pe[e];
      }
      // fp8: the block's V scale rides on the probabilities (the exp-sum stays unscaled)
      const float pvs = KV8 ? bvs[buf] : 1.f;
      const u32x2 pb = {Dt<DT>::pack2(pe[0] * pvs, pe[1] * pvs), Dt<DT>::pack2(pe[2] * pvs, pe[3] * pvs)};
      // slots past the end may hold anything, NaN bits included: zero their
      // V (branch-free: two ANDs per tile, or one on the fp8 codes)
      const uint32_t mlo = (kl > 0 ? 0x0000FFFFu : 0u) | (kl > 1 ? 0xFFFF0000u : 0u);
      const uint32_t mhi = (kl > 2 ? 0x0000FFFFu : 0u) | (kl > 3 ? 0xFFFF0000u : 0u);
      const uint32_t m8 = kl >= 4 ? 0xFFFFFFFFu : (kl <= 0 ? 0u : (0xFFFFFFFFu >> (32 - 8 * kl)));
      // fp8: lane (g, i) gets codes of tokens 4g .. 4g+3 of dim rows 16n + i
      u32x4 vt[KV8 ? NT / 4 : 1];
      if constexpr (KV8) {
#pragma unroll
        for (int q = 0; q < NT / 4; ++q) vt[q] = transpose_lane_groups4(vq8[buf][q]);
      }
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        u32x2 vv;
        if constexpr (KV8) {
          const uint32_t codes = vt[n >> 2][n & 3] & m8;  // a zero code is +0
          vv = u32x2{Dt<DT>::fp8x2(codes, false), Dt<DT>::fp8x2(codes, true)};
        } else {
          vv = u32x2{vb[buf][n].x & mlo, vb[buf][n].y & mhi};
        }
        o[n] = Dt<DT>::mma16x16x16(vv, pb, o[n]);
      }
    };

    // The first piece fills the pipeline; a later piece finds its first PF
    // blocks in flight already.
    if (prologue) {
#pragma unroll
      for (int q = 0; q < PF; ++q) issue(q, q, pidn0);  // (never the next piece)
    }

    // The next piece: its item, query and first page ids load now, while
    // this piece streams.  (With no next piece the current one is loaded
    // again, so these loads are unconditional.)
    {
      const int64_t gpos_n = c_gpos + c_count;
      has_next = gpos_n < b_end;
      int64_t s_n = c_s, r_n = c_r + c_count;
      if (r_n >= c_nb * segs) {
        ++s_n;
        r_n = 0;
      }
      x_v = c_v;
      x_vend = c_vend;
      if constexpr (kMultiV) {
        if (has_next && gpos_n >= c_vend) {  // the next piece is the next virtual worker's first
          x_v = c_v + 1;
          x_vend = vstart(sc, x_v + 1);
        }
      }
      if (has_next) {
        PAL_FIND_PIECE(x_, s_n, r_n, gpos_n, x_vend);
      } else {
        x_s = c_s; x_r = c_r; x_gpos = c_gpos; x_seq = c_seq; x_len = c_len; x_nb = c_nb; x_blk = c_blk;
        x_count = c_count; x_seg = c_seg;
      }
      load_q(x_s, x_seg, qn4, qn2);
      pidn0 = load_window(x_seq, x_blk, 0);
    }
    const uint32_t pidn1 = load_window(x_seq, x_blk, 1);
    {
      const int kvh_x = x_seg / p.head_chunks;
      kbase_n = static_cast<const uint8_t*>(p.k_pool) + kvh_x * head_block;
      vbase_n = static_cast<const uint8_t*>(p.v_pool) + kvh_x * head_block;
      kvh_n = kvh_x;
      nblk_n = static_cast<int>(x_count);
      bstart_n = static_cast<int>(x_blk);
      pbase_n = (bstart_n * 16) / TPP;
    }

    // Every step issues and computes unconditionally (steps past the end
    // re-read the last block, an L2 hit, and compute it fully masked): with
    // no load under a branch the compiler's wait counts stay exact, so the
    // PF blocks in flight are never drained early.
    //
    // A step group's issues select their page-id window by value, the next
    // piece's window 0 included.  Selecting pidn0 itself would make the
    // compiler wait for that load (issued just before the first group) at the
    // top of every group, draining the pipeline each time; the groups of a
    // piece with two or more of them select pidn0_ready instead, which the end
    // of each group refreshes (in the first group no issue reaches the next
    // piece: its issues stop at block NBUF + PF - 1 < n_pad).  A piece of one
    // group selects pidn0 and waits once.
    auto step_group = [&](int i0, uint32_t w_n0) {
      const uint32_t pid_ahead = load_window(c_seq, c_blk, wcur + 2);
#pragma unroll
      for (int u = 0; u < NBUF; ++u) {
        const int i = i0 + u;
        issue(i + PF, (u + PF) % NBUF, w_n0);
        compute(i, u);
      }
      // entered window wcur+1: move the windows up (at most NBUF + PF pages
      // past its start, so no issue has needed window wcur+2 yet)
      const int e_last = ((bstart + i0 + NBUF - 1) * 16) / TPP - pbase;
      const bool up = (e_last >> 6) > wcur;
      pid_cur = up ? pid_nxt : pid_cur;
      pid_nxt = up ? pid_later : pid_nxt;
      wcur += up ? 1 : 0;
      pid_later = pid_ahead;
      // The next piece's query and page ids must have arrived by the end of
      // the first step group (they are older than its loads): consume them
      // here, where the wait count is exact, so neither the later groups nor
      // the piece hand-over below wait on the loads in flight.
#pragma unroll
      for (int kk = 0; kk < (kK32 ? KK : 1); ++kk) asm volatile("" ::"v"(qn4[kk]));
#pragma unroll
      for (int kk = 0; kk < (kK32 ? 1 : KK); ++kk) asm volatile("" ::"v"(qn2[kk]));
      asm volatile("" ::"v"(pidn1));
      asm volatile("v_mov_b32 %0, %1" : "=v"(pidn0_ready) : "v"(pidn0));
    };
    if (n_pad == NBUF) {
      step_group(0, pidn0);
    } else {
      int i0 = 0;
      do {
        step_group(i0, pidn0_ready);
        i0 += NBUF;
      } while (i0 < n_pad);
    }

    // ---- finish the segment piece: exp-sum of head r16 over the 4 lane groups
    const float l = sum_xor32(sum_xor16(l_run));
    if (r16 < hg) {
      const int64_t row = (il.row ? static_cast<int64_t>(il.row[c_s]) : c_s) * p.num_q_heads + qh_base + r16;
      if (complete) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const u32x2 pk = {Dt<DT>::pack2(o[n][0] * inv, o[n][1] * inv), Dt<DT>::pack2(o[n][2] * inv, o[n][3] * inv)};
          *reinterpret_cast<u32x2*>(p.out + row * HD + 16 * n + 4 * g) = pk;
        }
      } else {
        // partial: (max, exp-sum) in fp32 and O / exp-sum in the 16-bit
        // dtype (half the bytes of fp32 O; the rounding is that of one more
        // output store)
        const int64_t slot = (c_v * 2 + (first ? 0 : 1)) * p.hg_max + r16;
        const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const u32x2 pk = {Dt<DT>::pack2(o[n][0] * inv, o[n][1] * inv), Dt<DT>::pack2(o[n][2] * inv, o[n][3] * inv)};
          *reinterpret_cast<u32x2*>(p.part_o + slot * HD + 16 * n + 4 * g) = pk;
        }
        if (g == 0) {
          const f32x2 ml = {m_run, l};  // the max is in log2 units already
          *reinterpret_cast<f32x2*>(p.part_ml + slot * 2) = ml;
        }
      }
    }

    // the first piece of a split segment can only end a virtual worker's
    // range (a range ends inside one segment): that segment goes on the
    // worker's merge-list slot
    if (!complete && c_blk == 0) {
      list_g0 = c_gpos;  // the piece starts the segment
      list_nb = c_nb;
      list_row = il.row ? static_cast<int64_t>(il.row[c_s]) : c_s;
      list_seg = c_seg;
    }
    prologue = false;
    first = false;
    if (!has_next) break;
    if constexpr (kMultiV) {
      if (x_v != c_v) {  // leaving virtual worker c_v
        write_list(c_v);
        list_g0 = -1;
        list_nb = list_row = list_seg = 0;
        first = true;
        c_v = x_v;
        c_vend = x_vend;
      }
    }

    // the next piece becomes current: its first PF blocks are in flight,
    // in buffers 0 .. PF-1 (n_pad is a multiple of NBUF)
    c_s = x_s; c_r = x_r; c_gpos = x_gpos; c_seq = x_seq; c_len = x_len; c_nb = x_nb; c_blk = x_blk;
    c_count = x_count; c_seg = x_seg;
#pragma unroll
    for (int kk = 0; kk < (kK32 ? KK : 1); ++kk) qv4[kk] = qn4[kk];
#pragma unroll
    for (int kk = 0; kk < (kK32 ? 1 : KK); ++kk) qv2[kk] = qn2[kk];
    if constexpr (KV8) query_to_fp8<DT, KK>(qv4, q8);
    wcur = 0;
    pid_cur = pidn0;
    pid_nxt = pidn1;
    pid_later = load_window(c_seq, c_blk, 2);
  }
  write_list(c_v);
#undef PAL_FIND_PIECE
}

template <int DT, int HD, int TPP, int PF, bool kChunks, bool KV8>
__device__ __forceinline__ void stream_body(const DecodeParams& p, int64_t* cum_lds, int64_t* len_lds,
                                            int32_t* seq_lds, int64_t* wave_sums) {
  const bool lds_plan = p.num_seqs <= kInlinePlanSeqs;
  const int64_t* cum = p.cum;
  int64_t total = 0;
  const int64_t n_items = p.num_seqs;
  if (lds_plan) {
    // Every workgroup scans the (at most 1024) sequence lengths into LDS:
    // thread t owns sequences 4t .. 4t+3.
    constexpr int kPer = kInlinePlanSeqs / kGroupThreads;
    const int64_t segs = static_cast<int64_t>(p.num_kv_heads) * p.head_chunks;
    const int tid = threadIdx.x;
    int64_t vals[kPer];
    int64_t tsum = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int64_t s = static_cast<int64_t>(tid) * kPer + k;
      vals[k] = 0;
      if (s < n_items) {
        const Item it = item_at(p, s, TPP);
        vals[k] = ((it.len + 15) >> 4) * segs;
        len_lds[s] = it.len;
        seq_lds[s] = static_cast<int32_t>(it.seq);
        // empty items get zeros, written once, by workgroup 0
        if (it.len == 0 && !it.skip && blockIdx.x == 0) zero_item_output<HD>(p, it.row);
      }
      tsum += vals[k];
    }
    const int64_t incl = block_inclusive_scan<kGroupThreads>(tsum, wave_sums);
    int64_t c = incl - tsum;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int64_t s = static_cast<int64_t>(tid) * kPer + k;
      if (s < n_items) cum_lds[s] = c;
      c += vals[k];
    }
    if (tid == kGroupThreads - 1) cum_lds[n_items] = incl;
    __syncthreads();
    total = cum_lds[n_items];
    if (blockIdx.x == 0) {  // the merge kernel reads the scan from the workspace
      for (int64_t s = tid; s <= n_items; s += kGroupThreads) p.cum[s] = cum_lds[s];
      if (tid == 0) p.hdr[0] = total;
    }
    cum = cum_lds;
  } else {
    total = p.hdr[0];
  }
  if (total == 0) return;
  const ItemLds il = lds_plan ? ItemLds{len_lds, seq_lds, nullptr} : ItemLds{nullptr, nullptr, nullptr};
  const Sched sc = make_sched(total, p.num_workers, p.tokens_per_worker);
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kWorkersPerGroup + wave_id();
  if constexpr (kChunks) {
    // fixed chunks: wavefront w streams the run of consecutive chunks
    // [w nc / W, (w + 1) nc / W) with one unbroken pipeline; each chunk is
    // still its own virtual worker (its own partials and merge-list slot)
    const int64_t nw = p.num_workers;
    const int64_t va = w * sc.nc / nw, vb = (w + 1) * sc.nc / nw;
    if (va < vb) process_range<DT, HD, TPP, PF, true, KV8>(p, sc, cum, il, n_items, va, vb);
  } else {
    if (w < sc.nws) process_range<DT, HD, TPP, PF, false, KV8>(p, sc, cum, il, n_items, w, w + 1);
  }
}

// Plain decode: the whole GPU streams KV, one wavefront per SIMD.  (With
// the non-temporal loads a third block of prefetch, or two wavefronts per
// SIMD, measured slower.)  kChunks: the fixed-chunk mode (partition_size >
// 0), a separate instantiation so the equal-share kernel keeps its lower
// register count.
template <int DT, int HD, int TPP, bool kChunks, bool KV8>
__global__ __launch_bounds__(kGroupThreads) void decode_stream_kernel(const DecodeParams p) {
  __shared__ int64_t cum_lds[kInlinePlanSeqs + 1];
  __shared__ int64_t len_lds[kInlinePlanSeqs];
  __shared__ int32_t seq_lds[kInlinePlanSeqs];
  __shared__ int64_t wave_sums[kWorkersPerGroup];
  // Fixed chunks are 8, 16 or 32 blocks: three blocks of prefetch make the
  // steps of a chunk a whole number of step groups (no padded step per
  // chunk; measured 2 % faster in the 512-token mode of config 3).
  // fp8 pools: a block is half the bytes and registers, so one more block
  // in flight keeps the bytes in flight per wavefront up
  constexpr int kPf = KV8 ? kPrefetch + 1 : (kChunks && HD <= 128 ? kPrefetch + 1 : kPrefetch);  // (bf16 head_dim 256 would spill)
  stream_body<DT, HD, TPP, kPf, kChunks, KV8>(p, cum_lds, len_lds, seq_lds, wave_sums);
}

// Decode rows of the fused op: one workgroup per CU, held to half of the
// register file (head_dim 128: one block of prefetch), so that a prefill tile
// wavefront fits on every SIMD beside it and the HBM-bound decode overlaps
// the MFMA-bound prefill instead of taking turns with it.
// Head dims above 128 run the two halves one after the other: their prefill
// tiles need more than half of the register file themselves.
constexpr bool shares_cu(int hd) { return hd <= 128; }

template <int HD, int TPP>
constexpr int shared_cu_prefetch() {
  return HD == 128 ? kPrefetch - 1 : kPrefetch;
}

// The decode rows of the fused op, found and scheduled inside the fused
// kernel (no planning launch): every decode workgroup scans the query rows,
// keeps the rows alone in their run of same-sequence rows that have keys
// ("lone rows"; the prefill tiles take every other row), and compacts up to
// kFusedLone of them -- row, page-table row, length and first global block --
// into LDS.  The scan is a pure function of the inputs, so every workgroup
// builds the same list.  The lone rows' blocks are then cut into the equal
// static shares of the resident workers, as in decode_stream_kernel, and
// the merge kernel combines the split segments.  With more lone rows than
// the list holds, each wavefront instead claims batches of 64 rows from the
// claim counter and computes every lone row of a batch whole (no split,
// nothing to merge; with that many rows the claims balance the load).
// Workgroup 0 writes the zeros of lone rows without keys and the total the
// merge kernel schedules from (0 in the claiming mode).
constexpr int kFusedLone = 2048;
constexpr int kFusedScanPer = 16;  // rows per thread per scan pass

struct FusedDecodeLds {
  int64_t cum[kFusedLone + 1];
  int64_t len[kFusedLone];
  int32_t seq[kFusedLone];
  int32_t row[kFusedLone];
  int64_t wave_sums[2][kWorkersPerGroup];
  int64_t totals[2];
  int64_t one_cum[kWorkersPerGroup][2];  // claiming mode: a one-row list per wavefront
  int64_t one_len[kWorkersPerGroup];
  int32_t one_seq[kWorkersPerGroup];
  int32_t one_row[kWorkersPerGroup];
  int64_t batch_len[kWorkersPerGroup][kWave];  // claiming mode: keys of the batch's rows
};

// The claiming mode of fused_decode_body: batches of 64 rows from the claim
// counter, each lone row of a batch computed whole on a one-row list.
template <int DT, int HD, int TPP, int PF, bool KV8, typename LoneRow>
__device__ __forceinline__ void fused_claim_rows(const DecodeParams& p, FusedDecodeLds& L,
                                                          const LoneRow& lone_row) {
  if (blockIdx.x == 0 && threadIdx.x == 0) p.hdr[0] = 0;  // nothing to merge
  const int64_t n_rows = p.num_seqs;
  const int64_t segs = static_cast<int64_t>(p.num_kv_heads) * p.head_chunks;
  const int wv = wave_id();
  const int lane = lane_id();
  for (;;) {
    uint32_t k = 0;
    if (lane == 0) k = atomicAdd(p.claim, 1u);
    const int64_t batch = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(k)) * kWave;
    if (batch >= n_rows) break;
    const int64_t r = batch + lane;
    int32_t len = 0;
    bool keep = false;
    if (r < n_rows) {
      const uint32_t prev = r > 0 ? p.q2seq[r - 1] : 0xFFFFFFFFu;
      const uint32_t next = r + 1 < n_rows ? p.q2seq[r + 1] : 0xFFFFFFFFu;
      keep = lone_row(r, prev, p.q2seq[r], next, len);
    }
    L.batch_len[wv][lane] = len;
    uint64_t bits = __ballot(keep);
    while (bits) {
      const int j = __builtin_ctzll(bits);
      bits &= bits - 1;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int64_t lj = L.batch_len[wv][j];
      if (lane == 0) {
        L.one_cum[wv][0] = 0;
        L.one_cum[wv][1] = ((lj + 15) >> 4) * segs;
        L.one_len[wv] = lj;
        L.one_seq[wv] = static_cast<int32_t>(p.q2seq[batch + j]);
        L.one_row[wv] = static_cast<int32_t>(batch + j);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const Sched sc = make_sched(((lj + 15) >> 4) * segs, 1, 0);
      process_range<DT, HD, TPP, PF, false, KV8>(p, sc, L.one_cum[wv],
                                                 ItemLds{&L.one_len[wv], &L.one_seq[wv], &L.one_row[wv]}, 1, 0, 1);
      // every lane is done with this row's list before the next one is written
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

template <int DT, int HD, int TPP, int PF, bool KV8>
__device__ __forceinline__ void fused_decode_body(const DecodeParams& p, FusedDecodeLds& L) {
  const int tid = threadIdx.x;
  const int64_t n_rows = p.num_seqs;  // row mode: one item per query row
  const int64_t segs = static_cast<int64_t>(p.num_kv_heads) * p.head_chunks;
  const int64_t max_tokens = p.page_table_width * TPP;
  // a row's sequence, keys and whether it is a lone row with keys
  auto lone_row = [&](int64_t r, uint32_t prev, uint32_t sq, uint32_t next, int32_t& len) {
    len = 0;
    if ((r > 0 && prev == sq) || (r + 1 < n_rows && next == sq)) return false;  // a prefill row
    if (sq < p.num_pt_rows) {
      const int64_t l = p.seq_lens[sq];
      const int64_t off = p.q_offset[r];
      const int64_t k = off < l ? off : l;
      PAL_DEBUG_FLAG(k > max_tokens, kDebugLength);
      len = static_cast<int32_t>(k < 0 ? 0 : (k > max_tokens ? max_tokens : k));
    }
    if (len == 0 && blockIdx.x == 0) zero_item_output<HD>(p, r);  // no key: zeros, once
    return len > 0;
  };

  // Quick pass: is any row alone in its run?  Lane t of a pass reads rows
  // 4t .. 4t+3 as one 16-byte load (when the map is 16-byte aligned) and
  // their two neighbours; a batch with none (a prefill-only batch) ends here.
  {
    bool any = false;
    const bool vec = (reinterpret_cast<uintptr_t>(p.q2seq) & 15u) == 0;
    for (int64_t base = 0; base < n_rows; base += 4 * kGroupThreads) {
      const int64_t r0 = base + 4 * static_cast<int64_t>(tid);
      if (r0 >= n_rows) continue;
      uint32_t q[6];
      q[0] = r0 > 0 ? p.q2seq[r0 - 1] : 0xFFFFFFFFu;
      if (vec && r0 + 4 <= n_rows) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(p.q2seq + r0);
        q[1] = v.x;
        q[2] = v.y;
        q[3] = v.z;
        q[4] = v.w;
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) q[1 + k] = r0 + k < n_rows ? p.q2seq[r0 + k] : 0xFFFFFFFFu;
      }
      q[5] = r0 + 4 < n_rows ? p.q2seq[r0 + 4] : 0xFFFFFFFFu;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t r = r0 + k;
        if (r < n_rows && (r == 0 || q[k] != q[k + 1]) && (r + 1 == n_rows || q[k + 2] != q[k + 1])) any = true;
      }
    }
    if (!__syncthreads_or(any)) {
      if (blockIdx.x == 0 && tid == 0) p.hdr[0] = 0;  // nothing to merge
      return;
    }
  }

  int64_t n_lone = 0, n_blocks = 0;  // running totals (uniform)
  for (int64_t base = 0; base < n_rows; base += static_cast<int64_t>(kGroupThreads) * kFusedScanPer) {
    const int64_t r0 = base + static_cast<int64_t>(tid) * kFusedScanPer;
    uint32_t sq[kFusedScanPer + 2];  // q2seq of rows r0 - 1 .. r0 + kFusedScanPer
#pragma unroll
    for (int k = 0; k < kFusedScanPer + 2; ++k) {
      const int64_t r = r0 - 1 + k;
      sq[k] = (r >= 0 && r < n_rows) ? p.q2seq[r] : 0xFFFFFFFFu;
    }
    int32_t lens[kFusedScanPer];  // keys (< 2^31: a page-table row holds fewer tokens)
    int64_t cnt = 0, blk = 0;
#pragma unroll
    for (int k = 0; k < kFusedScanPer; ++k) {
      const int64_t r = r0 + k;
      lens[k] = 0;
      if (r < n_rows && lone_row(r, sq[k], sq[k + 1], sq[k + 2], lens[k])) {
        cnt += 1;
        blk += ((lens[k] + 15) >> 4) * segs;
      }
    }
    const int64_t inc_c = block_inclusive_scan<kGroupThreads>(cnt, L.wave_sums[0]);
    const int64_t inc_b = block_inclusive_scan<kGroupThreads>(blk, L.wave_sums[1]);
    int64_t ci = n_lone + inc_c - cnt, bi = n_blocks + inc_b - blk;
#pragma unroll
    for (int k = 0; k < kFusedScanPer; ++k) {
      if (lens[k] > 0) {
        if (ci < kFusedLone) {
          L.cum[ci] = bi;
          L.len[ci] = lens[k];
          L.seq[ci] = static_cast<int32_t>(sq[k + 1]);
          L.row[ci] = static_cast<int32_t>(r0 + k);
        }
        ci += 1;
        bi += ((lens[k] + 15) >> 4) * segs;
      }
    }
    if (tid == kGroupThreads - 1) {
      L.totals[0] = inc_c;
      L.totals[1] = inc_b;
    }
    __syncthreads();
    n_lone += L.totals[0];
    n_blocks += L.totals[1];
    __syncthreads();  // totals and wave sums are rewritten by the next pass
  }

  const int64_t w = static_cast<int64_t>(blockIdx.x) * kWorkersPerGroup + wave_id();
  if (n_lone <= kFusedLone) {
    if (tid == 0) L.cum[n_lone] = n_blocks;
    if (blockIdx.x == 0 && tid == 0) p.hdr[0] = n_blocks;  // the merge kernel's schedule
    __syncthreads();
    if (n_blocks == 0) return;
    const ItemLds il{L.len, L.seq, L.row};
    const Sched sc = make_sched(n_blocks, p.num_workers, 0);
    if (w < sc.nws) process_range<DT, HD, TPP, PF, false, KV8>(p, sc, L.cum, il, n_lone, w, w + 1);
    return;
  }
  fused_claim_rows<DT, HD, TPP, PF, KV8>(p, L, lone_row);
}

// The fused mixed batch in one launch (head dims up to 128).  Blocks
// [0, n_dec) are the decode workers of the lone rows (one workgroup per CU,
// equal static shares of the rows' KV blocks, as in decode_stream_kernel),
// the other blocks the prefill tiles of the windows of rows.  The decode
// blocks have the lowest ids, so the dispatcher places them first: they hold
// one slot on every CU from the start instead of waiting for tiles to drain
// (equal static shares started late would end late), and the tiles take the
// other slot, then both once the decode workers are done.  The two roles
// share one LDS allocation.
static_assert(kPfThreads == kGroupThreads, "decode workers and prefill tiles share the workgroup shape");
template <int DT, int HD, int TPP, bool KV8>
__global__ __launch_bounds__(kGroupThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fused_kernel(const DecodeParams dp, const PrefillParams pp, const unsigned n_dec) {
  __shared__ union {
    FusedDecodeLds d;
    PrefillLds<HD, KV8> f;
  } lds;
  if (blockIdx.x < n_dec)
    fused_decode_body<DT, HD, TPP, shared_cu_prefetch<HD, TPP>(), KV8>(dp, lds.d);
  else
    prefill_block<DT, HD, TPP, KV8, false>(pp, blockIdx.x - n_dec, lds.f);
}

// Walks the merge list, slot v for virtual worker v (first block < 0:
// nothing to merge; every slot of the live range was written by this call's
// workers, with the segment's first block, block count, output row and
// segment index, so the merge needs no other lookup); a workgroup per slot
// at a time, the grid striding over the live workers.  A split segment
// (sequence, kv head, head chunk) is merged head by head, a wavefront per
// head: M = max_c m_c, w_c = 2^(m_c - M) l_c, out = sum_c w_c Y_c / sum_c w_c
// over the virtual workers c that shared it (Y_c = O_c / l_c, the stored
// normalised partial).
//
// The worker that wrote slot v holds the segment's first piece, so the
// contributors are v, v+1, ...: the list slot, the header and the partials of
// the first contributors are all fetched in one round trip, before the slot
// says how many there are.  A wavefront fetches one head's four candidate
// rows at once -- both partial slots of v (its piece may be v's first or its
// last) and the first-piece slots of v+1 and v+2 -- one row per 16 lanes,
// 8 dims (16 bytes) per lane, plus each row's (max, exp-sum): two load
// instructions per head instead of one per element.  A segment with more
// than three contributors is finished by the general loop.  Workgroup 0
// re-arms the claim counter.
template <int DT, int HD, int TPP>
__global__ __launch_bounds__(kGroupThreads) void decode_merge_kernel(const DecodeParams p) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.claim = 0u;
  const int lane = lane_id();
  const int wv = wave_id();
  constexpr int kCh = (HD + 127) / 128;                 // 8-dim chunks of a row per lane (16 lanes per row)
  constexpr int kHpw = 16 / kWorkersPerGroup;           // heads per wavefront (hg_max <= 16)
  constexpr int kBatch = 8;                             // general path: O loads in flight
  const int64_t last_w = p.list_cap - 1;                // partial slots exist for workers < list_cap
  const int cand = lane >> 4;                           // candidate row: 0, 1 = slots of e; 2, 3 = slot 0 of e+1, e+2
  const int rl16 = lane & 15;

  int64_t sg0 = 0, snb = 0, srow = 0, sseg = 0;
  f32x2 pml[kHpw];
  u32x4 po[kHpw][kCh];
  auto fetch = [&](int64_t e) {
    const int64_t* slot = p.split_list + 4 * e;
    sg0 = slot[0];
    snb = slot[1];
    srow = slot[2];
    sseg = slot[3];
    int64_t u = cand < 2 ? e : e + cand - 1;
    u = u < last_w ? u : last_w;
#pragma unroll
    for (int j = 0; j < kHpw; ++j) {
      const int h = wv + kWorkersPerGroup * j;
      if (h < p.hg_max) {
        const int64_t sl = (u * 2 + (cand == 1 ? 1 : 0)) * p.hg_max + h;
        pml[j] = *reinterpret_cast<const f32x2*>(p.part_ml + sl * 2);
#pragma unroll
        for (int c = 0; c < kCh; ++c) {
          const int d = 8 * rl16 + 128 * c;
          po[j][c] = d < HD ? *reinterpret_cast<const u32x4*>(p.part_o + sl * HD + d) : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
  };

  int64_t e = blockIdx.x;  // < list_cap: the grid is at most list_cap workgroups
  const int64_t total = p.hdr[0];
  fetch(e);
  if (total == 0) return;
  const Sched sc = make_sched(total, p.num_workers, p.tokens_per_worker);
  const int64_t n_slots = sc.nws + sc.nc < p.list_cap ? sc.nws + sc.nc : p.list_cap;
  while (e < n_slots) {
    const int64_t g0 = sg0;
    if (g0 >= 0) {
      const int64_t nb = snb;
      const int64_t out_row = srow;
      const int seg = static_cast<int>(sseg);
      const int kvh = seg / p.head_chunks;
      const int h0 = (seg % p.head_chunks) * 16;
      const int hg = min(16, p.group - h0);
      const int64_t v0 = vworker_of(sc, g0);
      const int64_t v1 = vworker_of(sc, g0 + nb - 1);
      const int64_t nc = v1 - v0 + 1;
      if (v0 == e && nc <= 3) {
        // the common case: every contributor's row is in registers already.
        // Contributor 0 is candidate t0 (slot 0 of e if the segment starts
        // e's range, else slot 1), contributors 1 and 2 candidates 2 and 3.
        const int t0 = vstart(sc, e) >= g0 ? 0 : 1;
        const bool live = cand == t0 || (cand >= 2 && cand - 1 < nc);
#pragma unroll
        for (int j = 0; j < kHpw; ++j) {
          const int h = wv + kWorkersPerGroup * j;
          if (h >= hg) continue;
          const float m = live ? pml[j].x : -INFINITY;
          float big_m = fmaxf(m, shfl_xor(m, 16));
          big_m = fmaxf(big_m, shfl_xor(big_m, 32));
          const float base_m = (big_m == -INFINITY) ? 0.f : big_m;
          // dead candidates may hold anything (an earlier call's rows, or
          // never-written bytes): their weight and products are zero by select
          float w = live ? __builtin_amdgcn_exp2f(m - base_m) * pml[j].y : 0.f;
          float lsum = w + shfl_xor(w, 16);
          lsum += shfl_xor(lsum, 32);
          const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
          const int64_t row = out_row * p.num_q_heads + kvh * p.group + h0 + h;  // output row
#pragma unroll
          for (int c = 0; c < kCh; ++c) {
            const int d = 8 * rl16 + 128 * c;
            float acc[8];
#pragma unroll
            for (int e8 = 0; e8 < 8; ++e8) {
              const uint32_t word = po[j][c][e8 >> 1];
              const float y = Dt<DT>::to_f32(static_cast<uint16_t>((e8 & 1) ? (word >> 16) : (word & 0xFFFFu)));
              acc[e8] = live ? w * y : 0.f;
              acc[e8] += shfl_xor(acc[e8], 16);
              acc[e8] += shfl_xor(acc[e8], 32);
            }
            if (cand == 0 && d < HD) {  // out is 8-byte aligned: two 8-byte stores
              uint16_t* dst = p.out + row * HD + d;
              const u32x2 lo = {Dt<DT>::pack2(acc[0] * inv, acc[1] * inv), Dt<DT>::pack2(acc[2] * inv, acc[3] * inv)};
              const u32x2 hi = {Dt<DT>::pack2(acc[4] * inv, acc[5] * inv), Dt<DT>::pack2(acc[6] * inv, acc[7] * inv)};
              *reinterpret_cast<u32x2*>(dst) = lo;
              *reinterpret_cast<u32x2*>(dst + 4) = hi;
            }
          }
        }
      } else {
        // General path: a lane group of kLpr lanes holds one contributor's
        // row (8 dims per lane, one 16-byte load), so one load instruction
        // covers kRpi contributors and kBatch instructions are in flight;
        // the row groups' sums are combined with shuffles at the end.
        // Contributor 0 is worker v0's piece in partial slot t0; every later
        // contributor's piece is its first (slot 0).
        constexpr int kLpr = HD <= 32 ? 4 : (HD <= 64 ? 8 : (HD <= 128 ? 16 : 32));  // >= HD / 8
        constexpr int kRpi = kWave / kLpr;
        const int rl = lane % kLpr;  // 8-dim slice of the row
        const int rg = lane / kLpr;  // row within one load instruction
        const bool dl = rl * 8 < HD;
        const int t0 = vstart(sc, v0) >= g0 ? 0 : 1;
        auto slot_j = [&](int64_t j, int h) { return ((v0 + j) * 2 + (j == 0 ? t0 : 0)) * p.hg_max + h; };
        for (int h = wv; h < hg; h += kWorkersPerGroup) {
          const int64_t row = out_row * p.num_q_heads + kvh * p.group + h0 + h;  // output row
          float big_m = -INFINITY;
          for (int64_t base = 0; base < nc; base += kWave) {
            const int64_t j = base + lane;
            const float m = j < nc ? p.part_ml[slot_j(j, h) * 2] : -INFINITY;
            big_m = fmaxf(big_m, m);
          }
#pragma unroll
          for (int off = 1; off < kWave; off <<= 1) big_m = fmaxf(big_m, shfl_xor(big_m, off));
          const float base_m = (big_m == -INFINITY) ? 0.f : big_m;

          float lsum = 0.f;  // this row group's share
          float acc[8];
#pragma unroll
          for (int e8 = 0; e8 < 8; ++e8) acc[e8] = 0.f;
          for (int64_t c0 = 0; c0 < nc; c0 += static_cast<int64_t>(kRpi) * kBatch) {
            u32x4 ob[kBatch];
            float mb[kBatch], lb[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
              const int64_t j = c0 + static_cast<int64_t>(u) * kRpi + rg;
              const bool jl = j < nc;
              const int64_t sl = slot_j(jl ? j : nc - 1, h);  // padding re-reads the last row
              mb[u] = p.part_ml[sl * 2];
              lb[u] = jl ? p.part_ml[sl * 2 + 1] : 0.f;
              ob[u] = dl ? *reinterpret_cast<const u32x4*>(p.part_o + sl * HD + rl * 8) : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
              const float w = __builtin_amdgcn_exp2f(mb[u] - base_m) * lb[u];
              lsum += w;
#pragma unroll
              for (int e8 = 0; e8 < 8; ++e8) {
                const uint32_t word = ob[u][e8 >> 1];
                acc[e8] += w * Dt<DT>::to_f32(static_cast<uint16_t>((e8 & 1) ? (word >> 16) : (word & 0xFFFFu)));
              }
            }
          }
          // combine the row groups (lanes kLpr, 2 kLpr, ... apart)
#pragma unroll
          for (int off = kLpr; off < kWave; off <<= 1) {
            lsum += shfl_xor(lsum, off);
#pragma unroll
            for (int e8 = 0; e8 < 8; ++e8) acc[e8] += shfl_xor(acc[e8], off);
          }
          const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
          if (rg == 0 && dl) {  // out is 8-byte aligned: two 8-byte stores
            uint16_t* dst = p.out + row * HD + rl * 8;
            const u32x2 lo = {Dt<DT>::pack2(acc[0] * inv, acc[1] * inv), Dt<DT>::pack2(acc[2] * inv, acc[3] * inv)};
            const u32x2 hi = {Dt<DT>::pack2(acc[4] * inv, acc[5] * inv), Dt<DT>::pack2(acc[6] * inv, acc[7] * inv)};
            *reinterpret_cast<u32x2*>(dst) = lo;
            *reinterpret_cast<u32x2*>(dst + 4) = hi;
          }
        }
      }
    }
    e += gridDim.x;
    if (e >= n_slots) break;
    fetch(e);
  }
}

// The merge for batches with few segments per worker (plain decode in the
// fixed-chunk mode, or with fewer segments than a quarter of the resident
// workers -- long contexts, where one segment has tens to thousands of
// contributors).  Instead of walking the merge list one workgroup per slot
// (a chain of round trips per segment), the grid enumerates the merge's
// outputs: workgroup b is unit (item s, segment k, head h, slice of
// kSegDims dims).  It finds the segment's blocks from the length scan
// (cum[s] + k nb .. + nb), hence its contributors v0 .. v1 by the fixed cut;
// its 256 threads are 64 contributor lanes x 4 groups of 8 dims, each lane
// loading (max, exp-sum) and 16 bytes of O of a batch of kBatch
// contributors per round trip (512 contributors per round trip per
// workgroup).  Each thread keeps a running max (rescaling its sums when it
// grows), and the lanes' sums are combined by the same log-sum-exp rule,
// across lanes with shuffles and across the wavefronts through LDS.
constexpr int kSegDims = 32;

template <int DT, int HD, int TPP>
__global__ __launch_bounds__(kGroupThreads) void decode_merge_seg_kernel(const DecodeParams p) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.claim = 0u;
  constexpr int kDs = HD < kSegDims ? HD : kSegDims;
  constexpr int kSlices = (HD + kDs - 1) / kDs;
  constexpr int kDg = kDs / 8;                 // 8-dim groups per slice
  constexpr int kCl = kGroupThreads / kDg;     // contributor lanes of the workgroup
  constexpr int kClw = kWave / kDg;            // of one wavefront
  constexpr int kBatch = 8;
  static_assert(kDs % 8 == 0, "slices of whole 8-dim groups");
  __shared__ float red[kWorkersPerGroup][kDg][10];
  const int tid = threadIdx.x;
  const int dg = tid % kDg;
  const int cl = tid / kDg;
  int64_t u = blockIdx.x;
  const int slice = static_cast<int>(u % kSlices);
  u /= kSlices;
  const int h = static_cast<int>(u % p.hg_max);
  u /= p.hg_max;
  const int segs = p.num_kv_heads * p.head_chunks;
  const int k = static_cast<int>(u % segs);
  const int64_t s = u / segs;
  const int kvh = k / p.head_chunks;
  const int h0 = (k % p.head_chunks) * 16;
  const int hg = min(16, p.group - h0);
  // every return below is uniform over the workgroup (before its barrier)
  if (s >= p.num_seqs || h >= hg) return;
  const Item it = item_at(p, s, TPP);
  const int64_t nb = (it.len + 15) >> 4;
  if (nb == 0) return;
  const int64_t total = p.hdr[0];  // > 0: this item has blocks
  const Sched sc = make_sched(total, p.num_workers, p.tokens_per_worker);
  const int64_t g0 = p.cum[s] + static_cast<int64_t>(k) * nb;
  const int64_t v0 = vworker_of(sc, g0);
  const int64_t nc = vworker_of(sc, g0 + nb - 1) - v0 + 1;
  if (nc <= 1) return;  // a whole segment: its worker wrote the output
  const int t0 = vstart(sc, v0) >= g0 ? 0 : 1;  // contributor 0's partial slot
  const int d = slice * kDs + dg * 8;
  const bool dl = d < HD;

  float m_loc = -INFINITY, l_loc = 0.f;
  float acc[8];
#pragma unroll
  for (int e8 = 0; e8 < 8; ++e8) acc[e8] = 0.f;
  for (int64_t c0 = 0; c0 < nc; c0 += static_cast<int64_t>(kCl) * kBatch) {
    f32x2 mlb[kBatch];
    u32x4 ob[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int64_t j = c0 + static_cast<int64_t>(b) * kCl + cl;
      const int64_t jj = j < nc ? j : nc - 1;  // padding re-reads the last row, with weight 0
      const int64_t sl = ((v0 + jj) * 2 + (jj == 0 ? t0 : 0)) * p.hg_max + h;
      mlb[b] = *reinterpret_cast<const f32x2*>(p.part_ml + sl * 2);
      if (j >= nc) mlb[b] = f32x2{-INFINITY, 0.f};
      ob[b] = dl ? *reinterpret_cast<const u32x4*>(p.part_o + sl * HD + d) : u32x4{0u, 0u, 0u, 0u};
    }
    float bm = m_loc;
#pragma unroll
    for (int b = 0; b < kBatch; ++b) bm = fmaxf(bm, mlb[b].x);
    if (bm > m_loc) {  // the running max grew: rescale this lane's sums
      const float a = m_loc == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_loc - bm);
      l_loc *= a;
#pragma unroll
      for (int e8 = 0; e8 < 8; ++e8) acc[e8] *= a;
      m_loc = bm;
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const float w = mlb[b].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mlb[b].x - m_loc) * mlb[b].y;
      l_loc += w;
#pragma unroll
      for (int e8 = 0; e8 < 8; ++e8) {
        const uint32_t word = ob[b][e8 >> 1];
        acc[e8] += w * Dt<DT>::to_f32(static_cast<uint16_t>((e8 & 1) ? (word >> 16) : (word & 0xFFFFu)));
      }
    }
  }
  // (m, l, acc) of two lanes -> their log-sum-exp combination
  auto combine = [&](float m2, float l2, const float (&a2)[8]) {
    const float mm = fmaxf(m_loc, m2);
    const float f1 = m_loc == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_loc - mm);
    const float f2 = m2 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m2 - mm);
    l_loc = f1 * l_loc + f2 * l2;
#pragma unroll
    for (int e8 = 0; e8 < 8; ++e8) acc[e8] = f1 * acc[e8] + f2 * a2[e8];
    m_loc = mm;
  };
  // across the contributor lanes of a wavefront (lane = cl_w * kDg + dg)
#pragma unroll
  for (int off = kDg; off < kWave; off <<= 1) {
    const float m2 = shfl_xor(m_loc, off);
    const float l2 = shfl_xor(l_loc, off);
    float a2[8];
#pragma unroll
    for (int e8 = 0; e8 < 8; ++e8) a2[e8] = shfl_xor(acc[e8], off);
    combine(m2, l2, a2);
  }
  const int wv = wave_id();
  const int lane = lane_id();
  if (lane < kDg) {
    red[wv][dg][0] = m_loc;
    red[wv][dg][1] = l_loc;
#pragma unroll
    for (int e8 = 0; e8 < 8; ++e8) red[wv][dg][2 + e8] = acc[e8];
  }
  __syncthreads();
  if (wv != 0 || lane >= kDg) return;
#pragma unroll
  for (int w2 = 1; w2 < kWorkersPerGroup; ++w2) {
    float a2[8];
#pragma unroll
    for (int e8 = 0; e8 < 8; ++e8) a2[e8] = red[w2][dg][2 + e8];
    combine(red[w2][dg][0], red[w2][dg][1], a2);
  }
  static_assert(kClw >= 1, "a wavefront holds whole 8-dim groups");
  if (!dl) return;
  const float inv = l_loc > 0.f ? 1.f / l_loc : 0.f;
  const int64_t row = it.row * p.num_q_heads + kvh * p.group + h0 + h;
  uint16_t* dst = p.out + row * HD + d;  // out is 8-byte aligned: two 8-byte stores
  const u32x2 lo = {Dt<DT>::pack2(acc[0] * inv, acc[1] * inv), Dt<DT>::pack2(acc[2] * inv, acc[3] * inv)};
  const u32x2 hi = {Dt<DT>::pack2(acc[4] * inv, acc[5] * inv), Dt<DT>::pack2(acc[6] * inv, acc[7] * inv)};
  *reinterpret_cast<u32x2*>(dst) = lo;
  *reinterpret_cast<u32x2*>(dst + 4) = hi;
}

// The merge of split segments, after the stream kernel.  Plain decode with
// few segments per worker (the fixed-chunk mode, or fewer segments than a
// quarter of the resident workers): the segment-enumerating merge, one
// workgroup per (item, segment, head, dim slice).  Otherwise the merge list:
// one slot per static share (at most num_workers) with equal shares, up to
// list_cap in the fixed-chunk mode.  A workgroup with no live slot still
// pays one fetch round trip, so the equal-share grid is not padded beyond
// the workers (it then fits the GPU in one round).
constexpr int64_t kMaxSegMergeGroups = 1 << 16;

template <int DT, int HD, int TPP>
hipError_t launch_merge(const DecodeParams& p, hipStream_t stream) {
  if (!p.q2seq) {
    const int64_t segments = p.num_seqs * p.num_kv_heads * p.head_chunks;
    constexpr int64_t slices = (HD + kSegDims - 1) / (HD < kSegDims ? HD : kSegDims);
    const int64_t units = segments * p.hg_max * slices;
    // The segment merge pays one workgroup per (segment, head, dim slice),
    // worth it once a segment has many contributors (its 64 contributor lanes
    // busy); otherwise the slot merge is faster (config 2 in partition-512
    // mode: 142 -> 116 us with the slot merge; 8 seqs of 32-128K in equal
    // shares, 16 per segment: the same; 4 seqs, 32 per segment: the segment
    // merge 1 us faster).  Fixed chunks: the most contributors a sequence can
    // have (page-table capacity / partition size); equal shares: the average.
    const int64_t contrib = p.tokens_per_worker > 0
                                ? (p.page_table_width * TPP + p.tokens_per_worker - 1) / p.tokens_per_worker
                                : p.num_workers / (segments > 0 ? segments : 1);
    if (contrib >= (p.tokens_per_worker > 0 ? 64 : 32) && units > 0 && units <= kMaxSegMergeGroups) {
      hipLaunchKernelGGL((decode_merge_seg_kernel<DT, HD, TPP>), dim3(static_cast<unsigned>(units)),
                         dim3(kGroupThreads), 0, stream, p);
      return hipGetLastError();
    }
  }
  int64_t merge_groups = p.tokens_per_worker == 0 ? p.num_workers : kMergeGroups;
  if (merge_groups > p.list_cap) merge_groups = p.list_cap;
  hipLaunchKernelGGL((decode_merge_kernel<DT, HD, TPP>), dim3(static_cast<unsigned>(merge_groups)),
                     dim3(kGroupThreads), 0, stream, p);
  return hipGetLastError();
}

// The scan of batches above kInlinePlanSeqs items, before the stream kernel.
template <int HD, int TPP>
hipError_t launch_plan(const DecodeParams& p, hipStream_t stream) {
  if (p.num_seqs <= kInlinePlanSeqs) return hipSuccess;
  hipLaunchKernelGGL((decode_plan_kernel<HD, TPP>), dim3(1), dim3(kPlanThreads), 0, stream, p);
  return hipGetLastError();
}

template <int DT, int HD, int TPP, bool KV8>
hipError_t launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  hipError_t err = launch_plan<HD, TPP>(p, stream);
  if (err != hipSuccess) return err;
  const int64_t groups = (static_cast<int64_t>(p.num_workers) + kWorkersPerGroup - 1) / kWorkersPerGroup;
  if (p.tokens_per_worker > 0)
    hipLaunchKernelGGL((decode_stream_kernel<DT, HD, TPP, true, KV8>), dim3(static_cast<unsigned>(groups)),
                       dim3(kGroupThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_stream_kernel<DT, HD, TPP, false, KV8>), dim3(static_cast<unsigned>(groups)),
                       dim3(kGroupThreads), 0, stream, p);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  return launch_merge<DT, HD, TPP>(p, stream);
}

template <int DT, int HD, bool KV8>
hipError_t dispatch_tpp(const DecodeParams& p, int tpp, hipStream_t stream) {
  switch (tpp) {
    case 16: return launch_decode_t<DT, HD, 16, KV8>(p, stream);
    case 32: return launch_decode_t<DT, HD, 32, KV8>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t dispatch_hd(const DecodeParams& p, int hd, int tpp, bool kv8, hipStream_t stream) {
  if (kv8) {  // fp8 pools: head dims that are whole 64-dim stripe rounds
    switch (hd) {
      case 64: return dispatch_tpp<DT, 64, true>(p, tpp, stream);
      case 128: return dispatch_tpp<DT, 128, true>(p, tpp, stream);
      case 256: return dispatch_tpp<DT, 256, true>(p, tpp, stream);
      default: return hipErrorInvalidValue;
    }
  }
  switch (hd) {
    case 32: return dispatch_tpp<DT, 32, false>(p, tpp, stream);
    case 64: return dispatch_tpp<DT, 64, false>(p, tpp, stream);
    case 80: return dispatch_tpp<DT, 80, false>(p, tpp, stream);
    case 96: return dispatch_tpp<DT, 96, false>(p, tpp, stream);
    case 128: return dispatch_tpp<DT, 128, false>(p, tpp, stream);
    case 256: return dispatch_tpp<DT, 256, false>(p, tpp, stream);
    default: return hipErrorInvalidValue;
  }
}

// The fused op: the fused kernel, then the merge; head dims above 128: the
// decode rows' kernels, then the prefill tiles.
template <int DT, int HD, int TPP, bool KV8>
hipError_t launch_fused_t(const DecodeParams& dp, const PrefillParams& pp, hipStream_t stream) {
  if constexpr (shares_cu(HD)) {
    hipError_t err;
    const int64_t n_dec = (static_cast<int64_t>(dp.num_workers) + kWorkersPerGroup - 1) / kWorkersPerGroup;
    const int64_t n_pf = static_cast<int64_t>(pp.num_units) * pp.num_kv_heads * pp.head_chunks;
    if (n_dec + n_pf > 0x7FFFFFFFll) return hipErrorInvalidValue;
    hipLaunchKernelGGL((fused_kernel<DT, HD, TPP, KV8>), dim3(static_cast<unsigned>(n_dec + n_pf)),
                       dim3(kGroupThreads), 0, stream, dp, pp, static_cast<unsigned>(n_dec));
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_merge<DT, HD, TPP>(dp, stream);
  } else {
    const hipError_t err = launch_decode_t<DT, HD, TPP, KV8>(dp, stream);
    if (err != hipSuccess) return err;
    return launch_prefill(pp, DT, HD, TPP, stream);
  }
}

template <int DT, int HD, bool KV8>
hipError_t fused_tpp(const DecodeParams& dp, const PrefillParams& pp, int tpp, hipStream_t stream) {
  switch (tpp) {
    case 16: return launch_fused_t<DT, HD, 16, KV8>(dp, pp, stream);
    case 32: return launch_fused_t<DT, HD, 32, KV8>(dp, pp, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t fused_hd(const DecodeParams& dp, const PrefillParams& pp, int hd, int tpp, bool kv8, hipStream_t stream) {
  if (kv8) {
    switch (hd) {
      case 64: return fused_tpp<DT, 64, true>(dp, pp, tpp, stream);
      case 128: return fused_tpp<DT, 128, true>(dp, pp, tpp, stream);
      case 256: return fused_tpp<DT, 256, true>(dp, pp, tpp, stream);
      default: return hipErrorInvalidValue;
    }
  }
  switch (hd) {
    case 32: return fused_tpp<DT, 32, false>(dp, pp, tpp, stream);
    case 64: return fused_tpp<DT, 64, false>(dp, pp, tpp, stream);
    case 96: return fused_tpp<DT, 96, false>(dp, pp, tpp, stream);
    case 128: return fused_tpp<DT, 128, false>(dp, pp, tpp, stream);
    case 256: return fused_tpp<DT, 256, false>(dp, pp, tpp, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int DT, int HD, int TPP, bool KV8>
const void* stream_kernel_ptr(bool chunks) {
  return chunks ? reinterpret_cast<const void*>(&decode_stream_kernel<DT, HD, TPP, true, KV8>)
                : reinterpret_cast<const void*>(&decode_stream_kernel<DT, HD, TPP, false, KV8>);
}

template <int DT, int HD, bool KV8>
const void* stream_kernel_tpp(int tpp, bool chunks) {
  return tpp == 32 ? stream_kernel_ptr<DT, HD, 32, KV8>(chunks) : stream_kernel_ptr<DT, HD, 16, KV8>(chunks);
}

template <int DT>
const void* stream_kernel_for(int hd, int tpp, bool chunks, bool kv8) {
  if (kv8) {
    switch (hd) {
      case 64: return stream_kernel_tpp<DT, 64, true>(tpp, chunks);
      case 128: return stream_kernel_tpp<DT, 128, true>(tpp, chunks);
      case 256: return stream_kernel_tpp<DT, 256, true>(tpp, chunks);
      default: return nullptr;
    }
  }
  switch (hd) {
    case 32: return stream_kernel_tpp<DT, 32, false>(tpp, chunks);
    case 64: return stream_kernel_tpp<DT, 64, false>(tpp, chunks);
    case 80: return stream_kernel_tpp<DT, 80, false>(tpp, chunks);
    case 96: return stream_kernel_tpp<DT, 96, false>(tpp, chunks);
    case 128: return stream_kernel_tpp<DT, 128, false>(tpp, chunks);
    case 256: return stream_kernel_tpp<DT, 256, false>(tpp, chunks);
    default: return nullptr;
  }
}

}  // namespace

hipError_t decode_resident_workers(int dtype, int head_dim, int tokens_per_page, bool shared_cu, bool chunks,
                                   bool kv8, int* workers) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  // The answer depends only on the device and the kernel instance: it is
  // computed once (an occupancy query and an attribute read) and cached.
  const bool shared = shared_cu && shares_cu(head_dim);
  const uint64_t key = (static_cast<uint64_t>(dev) << 32) | (static_cast<uint64_t>(dtype & 0xff) << 24) |
                       (static_cast<uint64_t>(head_dim & 0xfff) << 12) | (static_cast<uint64_t>(tokens_per_page & 0xff) << 4) |
                       (kv8 ? 4u : 0u) | (shared ? 2u : 0u) | (chunks ? 1u : 0u);
  static std::mutex mu;
  static std::unordered_map<uint64_t, int> cache;
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) {
      *workers = it->second;
      return hipSuccess;
    }
  }
  int cus = 0;
  err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err != hipSuccess) return err;
  int res = 0;
  if (shared) {  // one workgroup per CU; the prefill tiles take the rest
    res = cus * kWorkersPerGroup;
  } else {
    const void* fn = dtype == kBF16 ? stream_kernel_for<kBF16>(head_dim, tokens_per_page, chunks, kv8)
                                    : stream_kernel_for<kF16>(head_dim, tokens_per_page, chunks, kv8);
    if (!fn) return hipErrorInvalidValue;
    int groups_per_cu = 0;
    err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&groups_per_cu, fn, kGroupThreads, 0);
    if (err != hipSuccess) return err;
    if (groups_per_cu < 1) return hipErrorInvalidConfiguration;  // the kernel does not fit a CU
    // One workgroup per CU (one wavefront per SIMD, PF blocks in flight
    // each), whatever else the registers would allow: a second workgroup per
    // CU measured slower and doubles the split segments to merge.
    res = cus * kWorkersPerGroup;
  }
  {
    std::lock_guard<std::mutex> lock(mu);
    cache[key] = res;
  }
  *workers = res;
  return hipSuccess;
}

int64_t decode_virtual_workers(int64_t resident, int64_t max_blocks, int partition_size) {
  if (partition_size > 0) {  // one virtual worker per fixed chunk of the page-table capacity
    const int64_t chunk = partition_size / 16;
    return resident + (max_blocks + chunk - 1) / chunk;
  }
  return resident + 1;  // equal static shares
}

hipError_t launch_decode(const DecodeParams& p, int dtype, int head_dim, int tokens_per_page, hipStream_t stream) {
  const bool kv8 = p.k_scales != nullptr;
  if (dtype == kBF16) return dispatch_hd<kBF16>(p, head_dim, tokens_per_page, kv8, stream);
  return dispatch_hd<kF16>(p, head_dim, tokens_per_page, kv8, stream);
}

bool fused_shares_cu(int head_dim) { return shares_cu(head_dim); }

hipError_t launch_fused(const DecodeParams& dp, const PrefillParams& pp, int dtype, int head_dim, int tokens_per_page,
                        hipStream_t stream) {
  const bool kv8 = dp.k_scales != nullptr;
  if (dtype == kBF16) return fused_hd<kBF16>(dp, pp, head_dim, tokens_per_page, kv8, stream);
  return fused_hd<kF16>(dp, pp, head_dim, tokens_per_page, kv8, stream);
}

}  // namespace pal
