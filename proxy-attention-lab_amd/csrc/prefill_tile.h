// Paged causal attention for query tiles (prefill and the prefill rows of the
// fused mixed batch) on gfx950 MFMA.
//
// Reference behaviour: kernels/paged_attention/prefill/paged_attention_prefill.h.metal
// -- a prompt token attends to the cached history and to prompt tokens at or
// before it (:147-234, :251-360), scores scaled by 1/sqrt(HD) after the dot
// product (:178, :302), output rows (token, head) (:379-381).  In the fused
// op every key is read from pages: row r of sequence s sees keys
// [0, min(len[s], q_offset[r])), which is exactly the causal mask when the
// new tokens were written to the pages first.
//
// Design (MI355X):
//  * One workgroup (4 wavefronts) owns a tile of 128 "M-rows": QT consecutive
//    query tokens of one sequence times the (up to 16) query heads sharing a
//    kv head, so one K/V tile in LDS serves the whole GQA group.
//  * Per 32-key step the K and V tiles reach LDS by direct-to-LDS copies
//    (global_load_lds_dwordx4, no registers), issued three steps ahead into four
//    LDS buffers, with counted waits and one barrier per step.  Page ids come
//    from an LDS copy of the tile's page-table slice.  Steps of dense prompt
//    keys are copied the same way from the prompt rows (V rows untransposed,
//    read back with transposing LDS reads); fp8 pages in window mode as fp8
//    bytes, converted in the operand reads.  Steps across the history /
//    prompt boundary, with invalid page ids, or of fp8 pages in prompt mode
//    take a synchronous register path.
//  * Each wavefront computes S^T = K * Q^T with v_mfma_f32_32x32x16 (A = K
//    from LDS, B = Q^T held in registers) and O^T += V^T * P^T with the same
//    instruction.  In the transposed products a lane owns one M-row, so the
//    softmax max / sum need one cross-half exchange (v_permlane32_swap) and
//    the probabilities go into the PV MFMA without leaving the lane.  K is
//    stored in the QK operand's row order and V rows are swizzled, so every
//    operand read is one conflict-free 16-byte LDS access.
//  * Steps are software-pipelined inside a wavefront: the QK MFMAs of step
//    st+1 are issued among the exponentials of step st.
//  * Online softmax in log2 units with a lazy rescale: the running max is only
//    moved when a score exceeds it by more than 2^8, so O is rescaled rarely.
//  * Causal skipping: the key loop stops at the tile's largest limit, and key
//    steps below every row's limit skip the mask arithmetic.
//  * Two ways to name the work, both without a planning pass: the reference
//    prefill's uniform prompt (S sequences x P prompt rows; tiles are pure
//    arithmetic; keys [0, hist[s]) come from pages and keys hist[s] + i from
//    the dense prompt K/V rows s*P + i, as prefill.h.metal:147-234 reads
//    them), or windows of consecutive query rows (the fused op), each run of
//    rows of one sequence in a window being a tile.
//
// This header holds the device code of a tile (prefill_tile) so that both the
// prefill kernel (prefill.hip) and the fused mixed-batch kernel (decode.hip)
// compile it; a translation unit includes it after defining its debug-check
// flag word (PAL_DEBUG_FLAGS_DEFINE).
#pragma once

#include <type_traits>

#include "pal_device.h"

namespace pal {
namespace {


constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kMRows = kPfWaves * 32;  // M-rows (token, head) per workgroup
constexpr int kKeys = 32;              // keys per step
constexpr int kNBuf = 4;               // LDS step buffers (read by stragglers, computed, two in flight)
constexpr int kPidChunk = 512;         // page ids staged per chunk; two chunks live in LDS
static_assert(kPidChunk % kPfThreads == 0, "a page-id chunk is a whole number of loads per thread");
constexpr float kLazyRescale = 8.f;    // log2 headroom before the running max moves

// A step moves 4*HD items of 16 bytes of K and as many of V.
template <int HD>
struct StepGeo {
  static constexpr int kItems = 4 * HD;
  static constexpr int kLoads = (kItems + kPfThreads - 1) / kPfThreads;  // per thread, per K (or V)
};

// Item <-> (page, offset) maps.  LDS holds each step's items in item order,
// so one direct-to-LDS load per wavefront fills 1 KiB of consecutive slots
// (lane l -> slot base + l).  With TPP 16 the items are page-major (2*HD per
// page), which also makes each load instruction read a single page.
//   K item i: stripe c, slot t of the step holds key kperm(t):  page offset (c*TPP + kperm(t) % TPP) * 8
//   V item i: row d, 8-key group g' = g ^ swz(d) of the row:     page offset d*TPP + 8 g'
// K keys are stored in the QK operand's row order (kperm, an involution
// swapping bits 2 and 3 of the key index), so the operand reads are
// contiguous; the V groups are swizzled by row so that the PV operand reads
// (one 16-byte chunk per lane and row) spread over all banks.
__device__ __forceinline__ int kperm(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }
// fp8 steps: QK operand row m holds key 16 b2 + 8 b4 + 4 b3 + (m & 3) (b_i:
// bit i of m), so that the scores a lane holds after the QK product are
// the 16 consecutive keys 16 h .. 16 h + 15 (h: its lane half) in register
// order, and one 16-byte V item (16 keys of one row) feeds both PV k-steps.
__device__ __forceinline__ int kperm_f8(int m) {
  return ((m & 4) << 2) | ((m & 16) >> 1) | ((m & 8) >> 1) | (m & 3);
}

template <int HD, int TPP>
struct ItemMap {
  static __device__ __forceinline__ int k_page_half(int i) { return TPP == 16 ? i / (2 * HD) : 0; }
  // K item i: stripe c and the key (within the step) it carries
  static __device__ __forceinline__ void k_item(int i, int& c, int& key) {
    if (TPP == 16) {
      const int rem = i % (2 * HD);
      c = rem / 16;
      key = (i / (2 * HD)) * 16 + kperm(rem % 16);
    } else {
      c = i / 32;
      key = kperm(i % 32);
    }
  }
  static __device__ __forceinline__ int k_offset(int i) {  // element offset inside the (page, kv head) block
    int c, key;
    k_item(i, c, key);
    return (c * TPP + key % TPP) * 8;
  }
  // Conflict-free for 8-lane groups over 32 banks and 16-lane groups over 64
  // banks: within any 8 (and any 16) consecutive rows the 16-byte chunk each
  // lane reads lands on a distinct bank group.
  static __device__ __forceinline__ int v_swz(int d) {
    return TPP == 16 ? ((d >> 2) ^ (d >> 3)) & 1 : ((d >> 1) ^ (d >> 3)) & 3;
  }
  // V item i: row d and the group g stored in its slot (key offset in the step)
  static __device__ __forceinline__ void v_item(int i, int& d, int& key) {
    if (TPP == 16) {
      const int rem = i % (2 * HD);
      d = rem / 2;
      key = (i / (2 * HD)) * 16 + 8 * ((rem % 2) ^ v_swz(d));
    } else {
      d = i / 4;
      key = 8 * ((i % 4) ^ v_swz(d));
    }
  }
  // LDS slot of K operand row m (key kperm(m) of the step), stripe c
  static __device__ __forceinline__ int k_slot(int m, int c) {
    return TPP == 16 ? (m / 16) * (2 * HD) + c * 16 + m % 16 : c * 32 + m;
  }
  // LDS slot holding V row d, keys kg .. kg+7 of the step (kg multiple of 8)
  static __device__ __forceinline__ int v_slot(int d, int kg) {
    return TPP == 16 ? (kg / 16) * (2 * HD) + d * 2 + (((kg / 8) % 2) ^ v_swz(d)) : d * 4 + ((kg / 8) ^ v_swz(d));
  }
  // v_slot(d + 32 n, kg) - v_slot(d, kg): v_swz depends on bits 1..3 of d only
  static constexpr int kVRowTile = TPP == 16 ? 64 : 128;
};

// One query tile: rows [row0, row0 + nrows) of sequence s (nrows <= tokens
// per tile), query heads h0 .. h0+15 of kv head kvh.  PROMPT: the
// uniform-prompt mode (keys below the history length from pages, the rest
// from the dense prompt rows of sequence s); otherwise every key from pages.
template <int DT, int HD, int TPP, bool PROMPT, bool KV8>
__device__ __forceinline__ void prefill_tile(const PrefillParams& p, int row0, int nrows, int64_t s, int kvh, int h0,
                                             uint16_t* k_lds_base, uint16_t* v_lds_base, uint16_t* junk_lds,
                                             uint32_t* pid_lds, int* lim_lds, float* scl_lds) {
  // TPP 0: the page size is p.tokens_per_page, known at run time (a
  // multiple of 8; the reference prefill takes any, paged_attention_prefill.h.metal:
  // 243-263).  Steps of history keys then take the register path, reading
  // each key's page id from the page table; steps of dense prompt keys are
  // copied as for the other page sizes.  LDS holds every step in the
  // 32-key-page item order.
  constexpr int TP = TPP == 0 ? 32 : TPP;  // page size of the LDS item order
  const int tpp = TPP == 0 ? p.tokens_per_page : TPP;
  static_assert(TPP != 0 || (PROMPT && !KV8), "run-time page sizes: uniform-prompt mode, 16-bit pools");
  static_assert(HD % 32 == 0, "prefill needs head_dim % 32 == 0");
  static_assert(2 * StepGeo<HD>::kLoads <= HD / 16, "a step's copies fit in its PV chunks");
  constexpr int KS = HD / 16;  // QK k-steps of 16
  constexpr int DT32 = HD / 32;  // O^T row tiles of 32 dims
  constexpr int NI = StepGeo<HD>::kItems;
  constexpr int NL = StepGeo<HD>::kLoads;
  using IM = ItemMap<HD, TP>;
  // fp8 pools in window mode: steps are copied as fp8 bytes (16-byte items:
  // 16 dims of one key for K, 16 keys of one row for V; 2 HD items each, in
  // item order) and converted in the operand reads, each lane reading whole
  // items: a K item gives the 8 dims of two QK k-steps, a V item the 8 keys
  // of both PV k-steps (the keys of an fp8 step are in kperm_f8 order, the
  // query operand permuted to match).  A copy instruction must stay in one
  // page: with TP 16 that needs HD % 64 == 0 (every fp8 pool's head dim).
  constexpr bool F8 = KV8 && !PROMPT && (TP == 32 || HD % 64 == 0);
  constexpr int NI8 = 2 * HD;
  constexpr int NL8 = (NI8 + kPfThreads - 1) / kPfThreads;
  constexpr int NC = F8 ? NL8 : NL;  // copies per thread per step, K (and V)
  float* ks_lds = scl_lds;                   // fp8: K scale of page-table entry e in slot e % 1024
  float* vs_lds = scl_lds + 2 * kPidChunk;   // and V scale
  auto k_lds = [&](int b) { return k_lds_base + b * NI * 8; };
  auto v_lds = [&](int b) { return v_lds_base + b * NI * 8; };

  // tile coordinates are workgroup-uniform: keep them in scalar registers
  row0 = __builtin_amdgcn_readfirstlane(row0);
  nrows = __builtin_amdgcn_readfirstlane(nrows);
  s = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(s)));
  const int hg = min(16, p.group - h0);  // heads of this chunk
  const int qt = kMRows / p.hg_max;      // tokens per tile (hg_max = min(group, 16))
  constexpr bool prompt_mode = PROMPT;
  const bool seq_ok = s < p.num_seqs;  // a row naming no sequence attends to nothing
  if (!seq_ok) s = 0;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int w = wave_id();
  const int col = lane & 31;  // this lane's M-row within the wave
  const int half = lane >> 5;

  const int64_t max_tokens = p.page_table_width * tpp;
  int64_t hist = 0;  // prompt mode: keys below hist come from pages
  int64_t slen;
  if (prompt_mode) {
    hist = p.seq_lens[s];
    PAL_DEBUG_FLAG(hist > max_tokens, kDebugLength);
    hist = hist < 0 ? 0 : (hist > max_tokens ? max_tokens : hist);
    slen = hist + p.prompt_len;
  } else {
    slen = seq_ok ? p.seq_lens[s] : 0;
    PAL_DEBUG_FLAG(slen > max_tokens, kDebugLength);
    slen = slen < 0 ? 0 : (slen > max_tokens ? max_tokens : slen);
  }

  // Loads that need nothing but the tile's coordinates go out first, so
  // their latency overlaps the row-limit round trip: the query operand and
  // the first kPidChunk page-table entries of the row (staged into LDS once
  // the limits say how many the tile reads; entries past the sequence's
  // pages are never used).
  const int m_row = w * 32 + col;  // this lane's M-row
  const int my_t = m_row / p.hg_max;
  const int my_h = m_row % p.hg_max;
  const bool row_ok = my_t < nrows && my_t < qt && my_h < hg;
  // Q^T operand: lane holds Q[M-row col][16kk + 8 half .. +7] for all k-steps.
  u32x4 qv[KS];
  {
    const int64_t qrow = static_cast<int64_t>(row0 + (row_ok ? my_t : 0)) * p.num_q_heads + kvh * p.group + h0 +
                         (row_ok ? my_h : 0);
    const uint32_t qmask = row_ok ? 0xFFFFFFFFu : 0u;
    if constexpr (F8) {
      // fp8 steps read 16 dims of stripe 2j + half per K item: k-step 2j + e
      // of this lane half takes dims 16 (2j + half) + 8e .. +7
      const uint16_t* qp = p.q + qrow * HD + 16 * half;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        qv[kk] = *reinterpret_cast<const u32x4*>(qp + 32 * (kk / 2) + 8 * (kk % 2)) & qmask;
    } else {
      const uint16_t* qp = p.q + qrow * HD + 8 * half;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) qv[kk] = *reinterpret_cast<const u32x4*>(qp + 16 * kk) & qmask;
    }
  }
  const uint32_t* pt = p.page_table + s * p.page_table_width;
  constexpr int kPidPre = kPidChunk / kPfThreads;  // entries of chunk 0 per thread
  uint32_t pid_pre[kPidPre];
#pragma unroll
  for (int j = 0; j < kPidPre; ++j) {
    const int e = tid + j * kPfThreads;
    pid_pre[j] = e < p.page_table_width ? pt[e] : 0u;
  }

  // Row limits: M-row m = token * hg_max + head.  The previous tile's last
  // reads of the min / max words passed a barrier since.
  if (tid == 0) {
    lim_lds[kMRows] = 0;
    lim_lds[kMRows + 1] = 1 << 30;
  }
  __syncthreads();  // the previous tile is done with every LDS array
  if (tid < kMRows) {
    const int t = tid / p.hg_max;
    const int hh = tid % p.hg_max;
    int lim = 0;
    if (t < nrows && t < qt && hh < hg) {
      int64_t off = prompt_mode ? hist + (row0 + t - s * p.prompt_len) + 1 : p.q_offset[row0 + t];
      off = off < 0 ? 0 : off;
      lim = static_cast<int>(off < slen ? off : slen);
    }
    lim_lds[tid] = lim;
    if (t < nrows && t < qt && hh < hg) {
      atomicMax(&lim_lds[kMRows], lim);
      atomicMin(&lim_lds[kMRows + 1], lim);
    }
  }
  // fp8: the scales of those page-table entries, behind the page ids
  float ks_pre[kPidPre], vs_pre[kPidPre];
#pragma unroll
  for (int j = 0; j < kPidPre; ++j) {
    ks_pre[j] = 0.f;
    vs_pre[j] = 0.f;
    if constexpr (F8) {
      const int e = tid + j * kPfThreads;
      if (e < p.page_table_width && pid_pre[j] < p.num_pages) {
        const int64_t si = static_cast<int64_t>(pid_pre[j]) * p.num_kv_heads + kvh;
        ks_pre[j] = p.k_scales[si];
        vs_pre[j] = p.v_scales[si];
      }
    }
  }
  __syncthreads();
  // largest and smallest limit over the tile's rows (LDS atomics, two
  // words after the per-row limits, reset before the first barrier above)
  const int max_lim = __builtin_amdgcn_readfirstlane(lim_lds[kMRows]);
  const int min_lim = __builtin_amdgcn_readfirstlane(lim_lds[kMRows + 1]);
  const int my_lim = lim_lds[m_row];

  const int64_t head_block = static_cast<int64_t>(HD) * tpp;
  const int64_t page_stride = head_block * p.num_kv_heads;
  const int64_t page_stride8 = page_stride;            // fp8 pools: bytes per page (one byte per element)
  const int64_t kv_head_off8 = kvh * head_block;       // and of a kv head's block
  const int64_t dense_row0 = s * p.prompt_len - hist;  // dense row of key token tok: dense_row0 + tok
  const int64_t dense_stride = static_cast<int64_t>(p.num_kv_heads) * HD;
  const int64_t kv_head_off = kvh * head_block;
  const int nsteps = (max_lim + kKeys - 1) / kKeys;
  // page-table entries the tile reads: keys below max_lim, and in prompt mode
  // only those below the history (the rest are dense) -- never past the width
  const int paged_keys = prompt_mode ? min(max_lim, static_cast<int>(hist)) : max_lim;
  const int n_pid = TPP == 0 ? 0 : (paged_keys + TP - 1) / TP;  // runtime page size: no staged ids

  // Page ids live in LDS (two chunks of 512 entries, entry e in slot e % 1024):
  // reading them is an LDS broadcast, so the only vector-memory traffic in the
  // step loop is the K/V copies, whose count the waits below rely on.
  // fp8: the (page, kv head) scales of entry e, beside its page id (0 for an
  // invalid id: such a step takes the register path, which reads none)
  auto stage_scales = [&](int e, uint32_t pg) {
    if constexpr (F8) {
      const bool ok = pg < p.num_pages;
      const int64_t si = static_cast<int64_t>(ok ? pg : 0) * p.num_kv_heads + kvh;
      ks_lds[e % (2 * kPidChunk)] = ok ? p.k_scales[si] : 0.f;
      vs_lds[e % (2 * kPidChunk)] = ok ? p.v_scales[si] : 0.f;
    }
  };
  auto stage_pids = [&](int chunk) {  // synchronous; callers hold a barrier after it
    for (int e = chunk * kPidChunk + tid; e < min((chunk + 1) * kPidChunk, n_pid); e += kPfThreads) {
      const uint32_t pg = pt[e];
      pid_lds[e % (2 * kPidChunk)] = pg;
      stage_scales(e, pg);
    }
  };

  // Fast step: its first key below the tile's largest limit (the last step
  // may end past it), in valid pages (and, in prompt mode, all 32 keys below
  // the history, or all of them prompt keys): one direct-to-LDS copy per
  // item, no registers, nothing to wait for here.  Every wavefront issues exactly
  // 2*NL copies (items past the step go to a junk slot), so the wait counts
  // are the same on every wavefront.
  // Slow step (invalid pages, history / prompt boundary, fp8 in prompt mode): register loads,
  // masked, then LDS stores -- synchronous, so it also drains the copies in
  // flight, which keeps the counted waits safe.
  // pg0 / pg1: the pages of the step's first and (TP 16) second 16 keys.
  constexpr bool kAllItems = NI % kPfThreads == 0;  // no wavefront has a padding copy
  __builtin_assume(w >= 0 && w < kPfWaves);
  // page ids >= 2^32 - 1 cannot occur with fewer pages; such an id takes the slow path
  const uint32_t np32 = p.num_pages > 0xFFFFFFFFll ? 0xFFFFFFFFu : static_cast<uint32_t>(p.num_pages);
  // Copy q of a fast step into buffer buf: the K items (q < NL) or the V
  // items (q >= NL) of this thread's load q % NL, off0 / off1 the (page,
  // kv head) blocks of the step's two pages.
  auto copy_one = [&](int q, int buf, int64_t off0, int64_t off1) {
    const int jj = q % NL;
    const int i = tid + jj * kPfThreads;
    const int ib = w * kWave + jj * kPfThreads;  // first item of this wavefront's load
    const bool ok = kAllItems || ib < NI;
    if (q < NL) {
      const uint16_t* page = p.k_pool + (IM::k_page_half(ok ? ib : 0) ? off1 : off0);
      const uint32_t src = 2u * static_cast<uint32_t>(ok ? IM::k_offset(i) : 0);
      copy_to_lds16(page, src, lds_addr(ok ? k_lds(buf) + ib * 8 : junk_lds));
    } else {
      const uint16_t* page = p.v_pool + (IM::k_page_half(ok ? ib : 0) ? off1 : off0);
      int d = 0, key = 0;
      if (ok) IM::v_item(i, d, key);
      const uint32_t src = 2u * static_cast<uint32_t>(d * TP + key % TP);
      copy_to_lds16(page, src, lds_addr(ok ? v_lds(buf) + ib * 8 : junk_lds));
    }
  };
  // fp8 items.  K item i: page half ph (TP 16), stripe c (dims 16c ..
  // 16c+15), key of the step; V item i: page half ph (TP 16) or 16-key half
  // of the page row (TP 32), row d.  Item i is LDS slot i.
  auto k8_item = [](int i, int& ph, int& c, int& key) {
    if (TP == 16) {  // page-major; page 1's keys at positions XOR 12, so a 16-lane operand read spans all banks
      ph = i / HD;
      c = (i % HD) / 16;
      key = 16 * ph + ((i % 16) ^ (ph ? 12 : 0));
    } else {  // operand row order: slot 32 c + m holds key kperm_f8(m)
      ph = 0;
      c = i / 32;
      key = kperm_f8(i % 32);
    }
  };
  auto v8_item = [](int i, int& ph, int& d, int& kb) {  // kb: the item's first key in the step
    ph = TP == 16 ? i / HD : 0;
    d = i % HD;
    kb = 16 * (i / HD);
  };
  const uint8_t* k8_pool = reinterpret_cast<const uint8_t*>(p.k_pool) + kv_head_off8;
  const uint8_t* v8_pool = reinterpret_cast<const uint8_t*>(p.v_pool) + kv_head_off8;
  // Copy q of an fp8 fast step: K items (q < NL8) or V items of load q % NL8;
  // boff0 / boff1: byte offsets of the step's two pages' blocks.
  auto copy8 = [&](int q, int buf, int64_t boff0, int64_t boff1) {
    const int jj = q % NL8;
    const int i = tid + jj * kPfThreads;
    const int ib = w * kWave + jj * kPfThreads;  // first item of this wavefront's load
    const bool ok = ib < NI8;
    int ph = 0, a = 0, b = 0;
    uint32_t src = 0;
    if (q < NL8) {
      if (ok) k8_item(i, ph, a, b);
      src = static_cast<uint32_t>((a * TP + b % TP) * 16);
    } else {
      if (ok) v8_item(i, ph, a, b);
      src = static_cast<uint32_t>(a * TP + b % TP);
    }
    const int phw = (TP == 16 && ok) ? ib / HD : 0;  // the load's page half (one page per instruction)
    const uint8_t* page = (q < NL8 ? k8_pool : v8_pool) + (phw ? boff1 : boff0);
    copy_to_lds16(page, ok ? src : 0u, lds_addr(ok ? (q < NL8 ? k_lds(buf) : v_lds(buf)) + ib * 8 : junk_lds));
  };
  // An fp8 step on the register path (a page id out of range): the same
  // items, zero for invalid pages, V keys past max_lim cleared.
  auto slow8 = [&](int j, uint32_t pg0, uint32_t pg1) {
    const int buf = j % kNBuf;
    const int k0 = j * kKeys;
#pragma unroll
    for (int jj = 0; jj < NL8; ++jj) {
      const int i = tid + jj * kPfThreads;
      if (i >= NI8) continue;
      {
        int ph, c, key;
        k8_item(i, ph, c, key);
        const uint32_t pg = ph ? pg1 : pg0;
        PAL_DEBUG_FLAG(pg >= p.num_pages && k0 + key < max_lim, kDebugPageId);
        u32x4 val = {0u, 0u, 0u, 0u};
        if (pg < p.num_pages && k0 + key < max_lim)
          val = *reinterpret_cast<const u32x4*>(k8_pool + static_cast<int64_t>(pg) * page_stride8 +
                                                (c * TP + key % TP) * 16);
        *reinterpret_cast<u32x4*>(k_lds(buf) + i * 8) = val;
      }
      {
        int ph, d, kb;
        v8_item(i, ph, d, kb);
        const uint32_t pg = ph ? pg1 : pg0;
        u32x4 val = {0u, 0u, 0u, 0u};
        const int valid = max_lim - (k0 + kb);
        if (pg < p.num_pages && valid > 0) {
          val = *reinterpret_cast<const u32x4*>(v8_pool + static_cast<int64_t>(pg) * page_stride8 + d * TP + kb % TP);
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int bb = 0; bb < 4; ++bb)
              if (4 * e + bb >= valid) val[e] &= ~(0xFFu << (8 * bb));
        }
        *reinterpret_cast<u32x4*>(v_lds(buf) + i * 8) = val;
      }
    }
  };
  // step j takes the fast path (fp8 pools only in window mode, as fp8 items;
  // the 16-bit copies cannot dequantize)
  // (the tile's last step may end past max_lim: its copies then read keys
  // no row sees, from valid pages, and fix_tail clears their V entries)
  auto is_fast = [&](int j, uint32_t pg0, uint32_t pg1) {
    const int k0 = j * kKeys;
    return TPP != 0 && (!KV8 || F8) && k0 < max_lim && pg0 < np32 && pg1 < np32 && (!prompt_mode || k0 + kKeys <= hist);
  };
  // Prompt mode: a step whose 32 keys are all prompt keys below the tile's
  // largest limit copies them from the dense prompt rows (16-bit in every
  // pool dtype): K into its operand layout, V rows untransposed (V items of
  // the row layout are 16 contiguous bytes of one key; the PV operand reads
  // of such a step transpose).
  auto is_dense = [&](int j) {
    const int k0 = j * kKeys;
    return PROMPT && k0 >= hist && k0 < max_lim;
  };
  // Untransposed V rows, read back with transposing reads: each 16-lane
  // group reads 32 bytes of each of 4 consecutive keys, the other group of
  // its half-wavefront the next 32 bytes.  16-byte chunk c of key k is stored
  // at chunk c ^ vd_swz(k), which puts a 16-lane group on distinct banks in a
  // 32-bank pass and a half-wavefront on distinct banks in a 64-bank pass
  // (HD 96 rows are not swizzled).
  auto vd_swz = [](int key) {
    const int r = key & 3;
    return HD % 128 == 0 ? 4 * r + 2 * (r >> 1) : (HD == 64 ? 2 * r : (HD == 32 ? 2 * (r >> 1) : 0));
  };
  auto copy_dense = [&](int q, int buf, int j) {
    const int jj = q % NL;
    const int i = tid + jj * kPfThreads;
    const int ib = w * kWave + jj * kPfThreads;
    const bool ok = kAllItems || ib < NI;
    const int64_t row0 = (dense_row0 + j * kKeys) * dense_stride + kvh * HD;  // key 0 of the step, this kv head
    const int last = max_lim - 1 - j * kKeys;  // keys past it (tile's last step) read this key's row instead
    if (q < NL) {  // K in its operand layout, as from pages
      int c = 0, key = 0;
      if (ok) IM::k_item(i, c, key);
      const uint32_t src = 2u * static_cast<uint32_t>(min(key, last) * dense_stride + c * 8);
      copy_to_lds16(p.k_dense + row0, src, lds_addr(ok ? k_lds(buf) + ib * 8 : junk_lds));
    } else {
      // raw rows: slot i = (key, 8-dim chunk c ^ vd_swz(key))
      const int key = ok ? i / (HD / 8) : 0, c = ok ? (i % (HD / 8)) ^ vd_swz(key) : 0;
      const uint32_t src = 2u * static_cast<uint32_t>(min(key, last) * dense_stride + c * 8);
      copy_to_lds16(p.v_dense + row0, src, lds_addr(ok ? v_lds(buf) + ib * 8 : junk_lds));
    }
  };
  auto issue = [&](int j, uint32_t pg0, uint32_t pg1) {
    const int buf = j % kNBuf;
    const int k0 = j * kKeys;
    if (is_dense(j)) {
#pragma unroll
      for (int q = 0; q < 2 * NL; ++q) copy_dense(q, buf, j);
      return;
    }
    if (TP != 16) pg1 = pg0;
    const bool fast = is_fast(j, pg0, pg1);
    if constexpr (F8) {
      if (fast) {
#pragma unroll
        for (int q = 0; q < 2 * NL8; ++q)
          copy8(q, buf, static_cast<int64_t>(pg0) * page_stride8, static_cast<int64_t>(pg1) * page_stride8);
      } else {
        slow8(j, pg0, pg1);
      }
      return;
    }
    if (fast) {
      const int64_t off0 = static_cast<int64_t>(pg0) * page_stride + kv_head_off;
      const int64_t off1 = static_cast<int64_t>(pg1) * page_stride + kv_head_off;
#pragma unroll
      for (int q = 0; q < 2 * NL; ++q) copy_one(q, buf, off0, off1);
      return;
    }
    if constexpr (TPP == 0) {
      // run-time page size: each key's page from the page table (8 keys
      // of a V group share a page: the size is a multiple of 8)
#pragma unroll
      for (int jj = 0; jj < NL; ++jj) {
        const int i = tid + jj * kPfThreads;
        if (i >= NI) continue;
        {
          int kj, c;
          IM::k_item(i, c, kj);
          const int tok = k0 + kj;
          u32x4 val = {0u, 0u, 0u, 0u};
          if (tok < max_lim) {
            if (tok < hist) {
              const uint32_t pg = pt[tok / tpp];
              PAL_DEBUG_FLAG(pg >= p.num_pages, kDebugPageId);
              if (pg < p.num_pages)
                val = *reinterpret_cast<const u32x4*>(p.k_pool + static_cast<int64_t>(pg) * page_stride + kv_head_off +
                                                      (static_cast<int64_t>(c) * tpp + tok % tpp) * 8);
            } else {
              val = *reinterpret_cast<const u32x4*>(p.k_dense + (dense_row0 + tok) * dense_stride + kvh * HD + c * 8);
            }
          }
          *reinterpret_cast<u32x4*>(k_lds(buf) + i * 8) = val;
        }
        {
          int d, key;
          IM::v_item(i, d, key);
          const int tok = k0 + key;
          u32x4 val = {0u, 0u, 0u, 0u};
          if (tok < max_lim) {
            const uint32_t pg = tok < hist ? pt[tok / tpp] : 0u;
            const bool pg_ok = pg < p.num_pages;
            const uint16_t* vrow = p.v_pool + static_cast<int64_t>(pg) * page_stride + kv_head_off +
                                   static_cast<int64_t>(d) * tpp + tok % tpp;
            if (tok + 8 <= hist) {
              if (pg_ok) val = *reinterpret_cast<const u32x4*>(vrow);
            } else {
              uint32_t e16[8];
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const int t2 = tok + e;
                uint16_t x = 0;
                if (t2 < max_lim) {
                  if (t2 >= hist)
                    x = p.v_dense[(dense_row0 + t2) * dense_stride + kvh * HD + d];
                  else if (pg_ok)
                    x = vrow[e];
                }
                e16[e] = x;
              }
              val = {e16[0] | (e16[1] << 16), e16[2] | (e16[3] << 16), e16[4] | (e16[5] << 16),
                     e16[6] | (e16[7] << 16)};
            }
            const int valid = max_lim - tok;  // keys past the largest limit may hold anything
            if (valid < 8) {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                val[e] &= (2 * e < valid ? 0x0000FFFFu : 0u) | (2 * e + 1 < valid ? 0xFFFF0000u : 0u);
            }
          }
          *reinterpret_cast<u32x4*>(v_lds(buf) + i * 8) = val;
        }
      }
      return;
    }
#pragma unroll
    for (int jj = 0; jj < NL; ++jj) {
      const int i = tid + jj * kPfThreads;
      if (i >= NI) continue;
      const uint32_t pg = IM::k_page_half(i) ? pg1 : pg0;
      const bool pg_ok = pg < p.num_pages;
      PAL_DEBUG_FLAG(!pg_ok && k0 + (IM::k_page_half(i) ? 16 : 0) < (prompt_mode ? min(max_lim, static_cast<int>(hist)) : max_lim),
                     kDebugPageId);
      // K: stripe c, key kj of the step
      {
        int kj, c;
        IM::k_item(i, c, kj);
        const int tok = k0 + kj;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (!prompt_mode || tok < hist) {
          if (pg_ok && tok < max_lim) {
            if constexpr (KV8) {  // dims 8c..8c+7: half of 16-dim stripe c / 2, times the page's K scale
              const uint8_t* kp8 = reinterpret_cast<const uint8_t*>(p.k_pool) + static_cast<int64_t>(pg) * page_stride8 +
                                   kv_head_off8 + ((c >> 1) * TP + kj % TP) * 16 + (c & 1) * 8;
              val = fp8x8_scaled<DT>(*reinterpret_cast<const u32x2*>(kp8),
                                     p.k_scales[static_cast<int64_t>(pg) * p.num_kv_heads + kvh]);
            } else {
              val = *reinterpret_cast<const u32x4*>(p.k_pool + static_cast<int64_t>(pg) * page_stride + kv_head_off +
                                                    IM::k_offset(i));
            }
          }
        } else if (tok < max_lim) {
          val = *reinterpret_cast<const u32x4*>(p.k_dense + (dense_row0 + tok) * dense_stride + kvh * HD + c * 8);
        }
        *reinterpret_cast<u32x4*>(k_lds(buf) + i * 8) = val;
      }
      // V: row d, keys key .. key+7 of the step
      {
        int d, key;
        IM::v_item(i, d, key);
        const int tok = k0 + key;
        const uint16_t* vpage = p.v_pool + static_cast<int64_t>(pg) * page_stride + kv_head_off + d * TP;
        const uint8_t* vpage8 = reinterpret_cast<const uint8_t*>(p.v_pool) + static_cast<int64_t>(pg) * page_stride8 +
                                kv_head_off8 + d * TP;
        const float vsc = KV8 && pg_ok ? p.v_scales[static_cast<int64_t>(pg) * p.num_kv_heads + kvh] : 1.f;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (!prompt_mode || tok + 8 <= hist) {
          if (pg_ok && tok < max_lim) {
            if constexpr (KV8) {
              val = fp8x8_scaled<DT>(*reinterpret_cast<const u32x2*>(vpage8 + key % TP), vsc);
            } else {
              val = *reinterpret_cast<const u32x4*>(vpage + key % TP);
            }
          }
        } else if (tok < max_lim) {
          // some of the 8 keys are prompt tokens (dense, strided by row)
          uint32_t e16[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int t2 = tok + e;
            const bool pgd = t2 < hist;
            uint16_t x = 0;
            if (t2 < max_lim && (!pgd || pg_ok)) {
              if (!pgd) {
                x = p.v_dense[(dense_row0 + t2) * dense_stride + kvh * HD + d];
              } else if constexpr (KV8) {
                const uint32_t code = vpage8[(key + e) % TP];
                x = static_cast<uint16_t>(fp8x8_scaled<DT>(u32x2{code, 0u}, vsc)[0] & 0xFFFFu);
              } else {
                x = vpage[(key + e) % TP];
              }
            }
            e16[e] = x;
          }
          val = {e16[0] | (e16[1] << 16), e16[2] | (e16[3] << 16), e16[4] | (e16[5] << 16), e16[6] | (e16[7] << 16)};
        }
        // keys past the largest limit may hold anything (NaN bits included)
        const int valid = max_lim - tok;
        if (valid < 8) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t keep = (2 * e < valid ? 0x0000FFFFu : 0u) | (2 * e + 1 < valid ? 0xFFFF0000u : 0u);
            val[e] &= keep;
          }
        }
        *reinterpret_cast<u32x4*>(v_lds(buf) + i * 8) = val;
      }
    }
  };
  // The tile's last step j, when it ends past max_lim and was copied: the
  // keys no row sees hold whatever the pages (or, in prompt mode, the row of
  // the last key) held, and a masked probability of 0 times a NaN there
  // would still be NaN, so their V entries are cleared.  Each thread clears
  // its own items, after the barrier that saw the copies land and before the
  // barrier preceding the step's V reads (a slow step's entries are zero
  // already).
  auto fix_tail = [&](int j) {
    const int valid0 = max_lim - j * kKeys;  // valid keys of the step, 1 .. 31
    uint16_t* vb = v_lds(j % kNBuf);
    if constexpr (F8) {  // fp8 items: 16 key bytes of one row
#pragma unroll
      for (int jj = 0; jj < NL8; ++jj) {
        const int i = tid + jj * kPfThreads;
        if (i >= NI8) continue;
        int ph, d, kb;
        v8_item(i, ph, d, kb);
        const int valid = valid0 - kb;
        if (valid < 16) {
          u32x4* slot = reinterpret_cast<u32x4*>(vb + i * 8);
          u32x4 val = *slot;
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int bb = 0; bb < 4; ++bb)
              if (4 * e + bb >= valid) val[e] &= ~(0xFFu << (8 * bb));
          *slot = val;
        }
      }
      return;
    }
    const bool dense = is_dense(j);
#pragma unroll
    for (int jj = 0; jj < NL; ++jj) {
      const int i = tid + jj * kPfThreads;
      if (i >= NI) continue;
      u32x4* slot = reinterpret_cast<u32x4*>(vb + i * 8);
      if (dense) {  // raw rows: slot i holds 8 dims of key i / (HD / 8)
        if (i / (HD / 8) >= valid0) *slot = u32x4{0u, 0u, 0u, 0u};
      } else {  // operand layout: 8 keys key .. key+7 of row d
        int d, key;
        IM::v_item(i, d, key);
        const int valid = valid0 - key;
        if (valid < 8) {
          u32x4 val = *slot;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            val[e] &= (2 * e < valid ? 0x0000FFFFu : 0u) | (2 * e + 1 < valid ? 0xFFFF0000u : 0u);
          *slot = val;
        }
      }
    }
  };
  const bool tail_partial = max_lim % kKeys != 0;  // the last step ends past max_lim
  // the page ids of step j (an LDS broadcast read; TP 32: one page)
  // fp8: the scales of step j's first and (TP 16) second page (LDS
  // broadcast); 0 for a page past the tile's last staged entry (the tail
  // step's keys past max_lim: their V bytes are cleared, and 0 x a stale
  // scale could be NaN)
  auto read_scales = [&](const float* arr, int j, float& s0, float& s1) {
    const int e = j * kKeys / TP;
    s0 = e < n_pid ? arr[e % (2 * kPidChunk)] : 0.f;
    s1 = TP == 16 ? (e + 1 < n_pid ? arr[(e + 1) % (2 * kPidChunk)] : 0.f) : s0;
  };
  // fp8: step j's scores times the K scale of each key's page (register r
  // holds key 16 (r / 8) + ..., so r < 8: the first page)
  auto scale_scores = [&](f32x16& sacc, int j) {
    if constexpr (F8) {
      float s0, s1;
      read_scales(ks_lds, j, s0, s1);
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] *= half ? s1 : s0;  // the lane's keys are 16 half .. +15
    }
  };
  auto read_pids = [&](int j) {
    const int e = (j * kKeys / TP) % (2 * kPidChunk);
    u32x2 v;
    if (TP == 16) {
      v = *reinterpret_cast<const u32x2*>(pid_lds + e);  // e is even: 8-byte aligned
    } else {
      v.x = pid_lds[e];
      v.y = v.x;
    }
    return v;
  };

  float m_run = -INFINITY;  // running max of this lane's M-row (raw score units)
  float l_run = 0.f;        // this lane's share of the exp-sum
  f32x16 o[DT32];
#pragma unroll
  for (int n = 0; n < DT32; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[n][r] = 0.f;

  // Key order inside a 32-key step.  The QK product's A operand takes key
  // kperm(m) as its row m (bits 2 and 3 of m swapped); then the 8 scores a
  // lane feeds into each PV k-step are 8 consecutive keys, and the V^T operand
  // is one 16-byte LDS read per lane.  LDS already holds K in this row order.

  // S^T[key][M-row] = sum_d K[key][d] Q[M-row][d] for step st (raw scores).
  auto read_k = [&](int st, u32x4 (&ka)[KS]) {
    const int buf = st % kNBuf;
    if constexpr (F8) {  // lane: key kperm_f8(col), all 16 dims of stripe 2j + half: k-steps 2j and 2j + 1
      const int key = kperm_f8(col);
      const uint8_t* kb = reinterpret_cast<const uint8_t*>(k_lds(buf));
#pragma unroll
      for (int j = 0; j < KS / 2; ++j) {
        const int c = 2 * j + half;
        const int slot = TP == 16 ? (key / 16) * HD + c * 16 + ((key % 16) ^ (key >= 16 ? 12 : 0)) : c * 32 + col;
        const u32x4 v = *reinterpret_cast<const u32x4*>(kb + slot * 16);
        // exact in 16 bits; the K scale goes on the scores
        ka[2 * j] = fp8x8_exact<DT>(u32x2{v.x, v.y});
        ka[2 * j + 1] = fp8x8_exact<DT>(u32x2{v.z, v.w});
      }
      return;
    }
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int c = 2 * kk + half;  // stripe of dims 16kk + 8 half .. +7
      ka[kk] = *reinterpret_cast<const u32x4*>(k_lds(buf) + IM::k_slot(col, c) * 8);
    }
  };
  // V^T operand bases: k-step kk takes keys 16kk + 8 half .. +7; row tile n
  // (dims 32n + col) sits kVRowTile slots further
  const int v_base[2] = {IM::v_slot(col, 8 * half), IM::v_slot(col, 16 + 8 * half)};
  // register r holds key k0 + 16 (r/8) + 8 half + 4 ((r/4)%2) + r%4 of
  // M-row col (fp8 steps: key k0 + 16 half + r).  Scores stay raw (the scale is positive, so maxima commute
  // with it); the exponent is one fma: s * scale_log2 - m * scale_log2.  The
  // rounding of m * scale_log2 is common to a step's keys and cancels in the
  // normalisation while that product stays below ~2^14 (log2 units; trained
  // models' logits are far below); it grows with the product and overflows
  // exp2 past ~2^31.  An exact (s - m) * scale_log2 costs 16 more VALU
  // instructions per step (a rarely taken branch to it: 3 % on config 4).
  auto mask_score = [&](f32x16& sacc, int r, int st) {
    const int key = F8 ? st * kKeys + 16 * half + r
                       : st * kKeys + 16 * (r >> 3) + 8 * half + 4 * ((r >> 2) & 1) + (r & 3);
    if (key >= my_lim) sacc[r] = -INFINITY;
  };
  // Given this lane's max bm of a step's scores: moves the running max to the
  // row max if it grew by more than the headroom (rescaling this row's O and
  // exp-sum), and returns the exponent offset of the step.
  auto update_max = [&](float bm) {
    bm = max_xor32(bm);
    if (__ballot(bm > m_run + kLazyRescale * p.scale_inv_log2)) {
      const bool grow = bm > m_run + kLazyRescale * p.scale_inv_log2;
      const float m_new = fmaxf(m_run, bm);
      const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((m_run - m_new) * p.scale_log2);
      // rows whose max did not grow by more than the headroom keep their scale
      const float a = grow ? alpha : 1.f;
      if (grow) m_run = m_new;
      l_run *= a;
#pragma unroll
      for (int n = 0; n < DT32; ++n) o[n] *= a;
    }
    return (m_run == -INFINITY) ? 0.f : -m_run * p.scale_log2;
  };

  // Pipeline.  Memory: three steps ahead.  Iteration st waits for step st+1
  // (step st+2 may still be in flight), passes the barrier, and then issues
  // the copies of step st+3 into the buffer of step st-1, which every
  // wavefront finished reading before the barrier; hence four buffers.
  // Compute, inside a wavefront: all operand reads of the iteration go out
  // first; the QK MFMAs of step st+1 run beside the exponentials of step st,
  // and the PV MFMAs of step st beside the exp-sum of step st and the row max
  // of step st+1, which gives the next iteration its exponent offset.
  if (nsteps > 0) {
#pragma unroll
    for (int j = 0; j < kPidPre; ++j) {  // chunk 0, loaded above
      const int e = tid + j * kPfThreads;
      if (e < n_pid) {
        pid_lds[e] = pid_pre[j];
        if constexpr (F8) {
          ks_lds[e] = ks_pre[j];
          vs_lds[e] = vs_pre[j];
        }
      }
    }
    if (n_pid > kPidChunk) stage_pids(1);
  }
  __syncthreads();
  auto wait_barrier = [&](int pending_steps) {  // all but the pending_steps youngest steps' copies landed
    compiler_fence();
    if (pending_steps >= 2)
      __builtin_amdgcn_s_waitcnt(vmcnt_only(4 * NC));
    else if (pending_steps == 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * NC));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __builtin_amdgcn_s_waitcnt(kLgkmZero);
    __builtin_amdgcn_s_barrier();
    compiler_fence();
  };
  f32x16 s_cur;
#pragma unroll
  for (int r = 0; r < 16; ++r) s_cur[r] = 0.f;
  float mb = 0.f;
  if (nsteps > 0) {
    for (int j = 0; j < 3 && j < nsteps; ++j) {
      const u32x2 pg = read_pids(j);
      issue(j, __builtin_amdgcn_readfirstlane(pg.x), __builtin_amdgcn_readfirstlane(pg.y));
    }
    wait_barrier(min(nsteps - 1, 2));  // step 0 has landed
    if (nsteps == 1 && tail_partial) fix_tail(0);
    u32x4 ka[KS];
    read_k(0, ka);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) s_cur = Dt<DT>::mma32x32x16(ka[kk], qv[kk], s_cur);
    scale_scores(s_cur, 0);
    float bm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (min_lim < kKeys) mask_score(s_cur, r, 0);
      bm = fmaxf(bm, s_cur[r]);
    }
    mb = update_max(bm);
  }
  // Steps whose next step needs no mask (every row sees all its keys) run
  // the unmasked body.  The last step is always in the masked part, whose
  // mask also discards the scores of the stale buffer it reads as "next".
  const int n_main = max(0, min(nsteps, min_lim / kKeys - 1));
  // dense_v: step st's V rows were copied untransposed (a dense prompt step);
  // each combination is its own loop body, so the operand reads carry no
  // per-chunk branch.
  auto step = [&](auto masked, auto dense_v, int st) {
    constexpr bool kMask = decltype(masked)::value;
    constexpr bool vdense = decltype(dense_v)::value;
    wait_barrier(st + 2 < nsteps ? 1 : 0);  // step st+1 has landed
    const int j = st + 3;
    const u32x2 pgv = read_pids(j);  // used after the MFMAs (in bounds whether or not step j exists)
    u32x4 ka[KS];
    read_k(st + 1, ka);
    if (kMask && st + 2 == nsteps && tail_partial) fix_tail(st + 1);
    float pe[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) pe[r] = fmaf(s_cur[r], p.scale_log2, mb);
    // The rest is written in issue order, chunk by chunk, with scheduling
    // fences between chunks (the compiler would otherwise keep two operand
    // reads in flight, wait before every MFMA and bunch the vector work):
    // each QK MFMA of step st+1 (K operands all read above) goes out with one
    // V operand read of step st and a share of step st's exponentials and
    // conversions; each PV MFMA of step st with a share of the exp-sum and of
    // the row max of step st+1.
    sched_fence();
    // Raised wave priority through the MFMA chunks: the other wavefront on
    // the SIMD is then more often in its vector/LDS phase while this one
    // issues MFMAs (measured +1 % on config 4, -1 to -3 % time on config 5).
    __builtin_amdgcn_s_setprio(1);
    const int vbuf = st % kNBuf;
    float vs0 = 1.f, vs1 = 1.f;  // fp8: V scales of step st's pages
    if constexpr (F8) read_scales(vs_lds, st, vs0, vs1);
    f32x16 s_next;
#pragma unroll
    for (int r = 0; r < 16; ++r) s_next[r] = 0.f;
    u32x4 va[KS];  // PV operand m: k-step m / DT32, row tile m % DT32 (KS == 2 * DT32)
    u32x4 v16[F8 ? DT32 : 1];  // fp8: row tile t's item (16 keys of one row), both PV k-steps
    uint32_t pp[8];  // packed probabilities of the lane's scores 2q, 2q+1
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      s_next = Dt<DT>::mma32x32x16(ka[kk], qv[kk], s_next);
      if constexpr (vdense) {
        // raw rows: V[key][d] in chunk (d / 8) ^ vd_swz(key) of row key.  Lane
        // 4r + c of a 16-lane group points at keys kg + 4t + r, dims d0 + 4c ..
        // +3 (d0 = 32 (kk % DT32) + (col & 16)); the transposing read hands
        // lane j dim d0 + j = col + 32 (kk % DT32) of those 4 keys.
        const int l16 = lane & 15;
        const int key = 16 * (kk / DT32) + 8 * half + (l16 >> 2);
        const int d = 32 * (kk % DT32) + (col & 16) + 4 * (l16 & 3);
        const uint16_t* vr = v_lds(vbuf) + key * HD + (((d >> 3) ^ vd_swz(key)) << 3) + (d & 7);
        const u32x2 lo = lds_read_tr16(vr);           // keys kg .. kg+3
        const u32x2 hi = lds_read_tr16(vr + 4 * HD);  // keys kg+4 .. kg+7 (vd_swz(key + 4) = vd_swz(key))
        va[kk] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      } else if constexpr (F8) {
        // chunk t < DT32 reads row tile t's item (half, d = col + 32 t): keys
        // 16 half .. +7 for k-step 0 (operand t), +8 .. +15 for k-step 1
        // (operand t + DT32).  Exact in 16 bits; the V scale is on P.  Each
        // half is converted in a later chunk than its read (the LDS read has
        // landed) and consumed there, so the conversions are not sunk to the
        // PV MFMAs.
        if (kk < DT32)
          v16[kk] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(v_lds(vbuf)) +
                                                    (half * HD + col + 32 * kk) * 16);
        if (kk >= 1 && kk <= DT32) {
          va[kk - 1] = fp8x8_exact<DT>(u32x2{v16[kk - 1].x, v16[kk - 1].y});
          asm volatile("" ::"v"(va[kk - 1]));
        }
        if (kk >= DT32) {
          va[kk] = fp8x8_exact<DT>(u32x2{v16[kk - DT32].z, v16[kk - DT32].w});
          asm volatile("" ::"v"(va[kk]));
        }
      } else {
        va[kk] = *reinterpret_cast<const u32x4*>(v_lds(vbuf) + (v_base[kk / DT32] + (kk % DT32) * IM::kVRowTile) * 8);
      }
#pragma unroll
      for (int r = kk * 16 / KS; r < (kk + 1) * 16 / KS; ++r) pe[r] = __builtin_amdgcn_exp2f(pe[r]);
#pragma unroll
      for (int q = kk * 8 / KS; q < (kk + 1) * 8 / KS; ++q) {
        if constexpr (F8) {  // the exp-sum of the probabilities, then P times its key's page V scale
          const float sv = half ? vs1 : vs0;  // the lane's keys 16 half .. +15: page half (TP 32: vs1 == vs0)
          l_run += pe[2 * q] + pe[2 * q + 1];
          pp[q] = Dt<DT>::pack2(pe[2 * q] * sv, pe[2 * q + 1] * sv);
        } else {
          pp[q] = Dt<DT>::pack2(pe[2 * q], pe[2 * q + 1]);
        }
        // consumed here, so the exponentials and the conversion stay in this
        // chunk beside its QK MFMA (the fences only bind the scheduler: code
        // motion would otherwise sink them to the PV MFMAs that use them,
        // past the copy branches)
        asm volatile("" ::"v"(pp[q]));
      }
      sched_fence();
    }
    const u32x4 pb[2] = {u32x4{pp[0], pp[1], pp[2], pp[3]}, u32x4{pp[4], pp[5], pp[6], pp[7]}};
    scale_scores(s_next, st + 1);
    // O^T[d][M-row] += sum_key V[key][d] P[M-row][key]; k-step kk takes
    // registers 8kk .. 8kk+7 = keys 16kk + 8 half .. +7.
    float bm = -INFINITY;
    // A fast step j issues its copies one per PV chunk (the first 2 NL
    // chunks), so the wavefront's MFMAs run while an issue waits for the
    // memory pipeline (measured 3 % on config 4 against issuing them all
    // after the chunks); other steps take the synchronous path below.
    const uint32_t jp0 = __builtin_amdgcn_readfirstlane(pgv.x);
    const uint32_t jp1 = TP == 16 ? __builtin_amdgcn_readfirstlane(pgv.y) : jp0;
    const bool jdense = j < nsteps && (vdense || is_dense(j));  // steps after a dense one are dense
    const bool jfast = j < nsteps && (jdense || is_fast(j, jp0, jp1));
    const int64_t joff0 = static_cast<int64_t>(jp0) * page_stride + kv_head_off;
    const int64_t joff1 = static_cast<int64_t>(jp1) * page_stride + kv_head_off;
#pragma unroll
    for (int m = 0; m < KS; ++m) {
      if (jfast && m < 2 * NC) {
        if constexpr (F8)
          copy8(m, j % kNBuf, static_cast<int64_t>(jp0) * page_stride8, static_cast<int64_t>(jp1) * page_stride8);
        else if (jdense)
          copy_dense(m, j % kNBuf, j);
        else
          copy_one(m, j % kNBuf, joff0, joff1);
      }
      o[m % DT32] = Dt<DT>::mma32x32x16(va[m], pb[m / DT32], o[m % DT32]);
      // the exp-sum adds the probabilities as rounded for the PV product
#pragma unroll
      for (int q = m * 8 / KS; q < (m + 1) * 8 / KS; ++q)
        if constexpr (!F8) l_run = Dt<DT>::sum2(pp[q], l_run);
#pragma unroll
      for (int r = m * 16 / KS; r < (m + 1) * 16 / KS; ++r) {
        if (kMask) mask_score(s_next, r, st + 1);
        bm = fmaxf(bm, s_next[r]);
      }
      sched_fence();
    }
    __builtin_amdgcn_s_setprio(0);
    mb = update_max(bm);
    if (j < nsteps) {
      // entering page-id chunk q (q >= 1): stage chunk q + 1 over chunk q - 1,
      // whose last reader finished before this iteration's barrier; the next
      // barriers publish it long before its first reader
      const int e0 = j * kKeys / TP;
      if (e0 % kPidChunk == 0 && e0 > 0 && e0 + kPidChunk < n_pid) stage_pids(e0 / kPidChunk + 1);
      if (!jfast) issue(j, jp0, jp1);
    }
    s_cur = s_next;
  };
  // prompt mode: steps from ceil(hist / 32) on are dense (the one across the
  // boundary, if any, is not)
  const int fd = PROMPT ? min(nsteps, static_cast<int>((hist + kKeys - 1) / kKeys)) : nsteps;
  int st = 0;
  for (; st < min(n_main, fd); ++st) step(std::false_type{}, std::false_type{}, st);
  if constexpr (PROMPT)
    for (; st < n_main; ++st) step(std::false_type{}, std::true_type{}, st);
  for (; st < fd; ++st) step(std::true_type{}, std::false_type{}, st);
  if constexpr (PROMPT)
    for (; st < nsteps; ++st) step(std::true_type{}, std::true_type{}, st);

  // ---- normalise and write: lane holds O[M-row col][32n + 8(r/4) + 4 half + r%4]
  float l = sum_xor32(l_run);
  if (row_ok) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int64_t orow = static_cast<int64_t>(row0 + my_t) * p.num_q_heads + kvh * p.group + h0 + my_h;
    uint16_t* op = p.out + orow * HD;
#pragma unroll
    for (int n = 0; n < DT32; ++n) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * n + 8 * q4 + 4 * half;
        const u32x2 pk = {Dt<DT>::pack2(o[n][4 * q4 + 0] * inv, o[n][4 * q4 + 1] * inv),
                          Dt<DT>::pack2(o[n][4 * q4 + 2] * inv, o[n][4 * q4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(op + d) = pk;
      }
    }
  }
}

// Rows [0, R) of the query batch alternate runs of one sequence.  Is row r
// alone in its run (a decode row, served by the decode kernels)?
__device__ __forceinline__ bool single_row(const uint32_t* q2seq, int64_t r, int64_t n) {
  const uint32_t sq = q2seq[r];
  return (r == 0 || q2seq[r - 1] != sq) && (r + 1 == n || q2seq[r + 1] != sq);
}

// LDS of a prefill workgroup: four K and four V step buffers, the target of
// padding copies, two chunks of page ids, the rows' key limits (with their
// max and min) and the run starts of a window.
template <int HD, bool KV8>
struct PrefillLds {
  __attribute__((aligned(16))) uint16_t k[kNBuf * StepGeo<HD>::kItems * 8];
  __attribute__((aligned(16))) uint16_t v[kNBuf * StepGeo<HD>::kItems * 8];
  __attribute__((aligned(16))) uint16_t junk[kWave * 8];
  uint32_t pid[2 * kPidChunk];
  float scl[KV8 ? 4 * kPidChunk : 1];  // fp8 pools: K then V scale of each staged page id
  int lim[kMRows + 2];
  int run_start[kMRows];
};

// The work of prefill block b (a 1-D grid, XCD-aware): head group
// g = b % G (G = kv heads x head chunks) and work unit b / G, so consecutive
// blocks -- which the dispatcher spreads over the 8 XCDs -- take different kv
// heads, and each kv head's K/V stay in few L2s.
//  * prompt mode: unit = (sequence, tile), the last tile of a sequence first
//    (it has the most keys);
//  * window mode (fused op): unit = window of `tokens per tile` rows, the
//    last window first (rows of a sequence usually come in position order,
//    so its later windows see more keys); every run of rows of one sequence
//    inside the window that is not a lone decode row is computed as a tile.
// kPromptMode false: the caller never runs the uniform-prompt mode (the
// fused kernel), which is then not compiled in.
template <int DT, int HD, int TPP, bool KV8, bool kPromptMode = true>
__device__ __forceinline__ void prefill_block(const PrefillParams& p, unsigned block, PrefillLds<HD, KV8>& L) {
  uint16_t* k_lds = L.k;
  uint16_t* v_lds = L.v;
  uint16_t* junk_lds = L.junk;
  uint32_t* pid_lds = L.pid;
  float* scl_lds = L.scl;
  int* lim_lds = L.lim;
  int* run_start = L.run_start;
  const int G = p.num_kv_heads * p.head_chunks;
  const int g = static_cast<int>(block % static_cast<unsigned>(G));
  const int unit = static_cast<int>(block / static_cast<unsigned>(G));
  const int kvh = g / p.head_chunks;
  const int h0 = (g % p.head_chunks) * 16;
  const int qt = kMRows / p.hg_max;
  if constexpr (kPromptMode) {
    if (p.prompt_len > 0) {
      const int tps = (p.prompt_len + qt - 1) / qt;
      const int s = unit / tps;
      const int j = tps - 1 - (unit - s * tps);
      const int row0 = s * p.prompt_len + j * qt;
      prefill_tile<DT, HD, TPP, true, KV8>(p, row0, min(qt, p.prompt_len - j * qt), s, kvh, h0, k_lds, v_lds,
                                           junk_lds, pid_lds, lim_lds, scl_lds);
      return;
    }
  }
  if constexpr (TPP != 0) {  // run-time page sizes: uniform-prompt mode only
    // windows in reverse row order: a sequence's later rows see more keys, so
    // its longest tiles start first and the grid ends on short ones
    const int w0 = (p.num_units - 1 - unit) * qt;
    const int w1 = static_cast<int>(min(static_cast<int64_t>(w0 + qt), p.num_rows));
    const int tid = threadIdx.x;
    if (tid < w1 - w0) run_start[tid] = (tid == 0 || p.q2seq[w0 + tid] != p.q2seq[w0 + tid - 1]) ? 1 : 0;
    __syncthreads();
    int cur = w0;
    while (cur < w1) {
      int end = cur + 1;
      while (end < w1 && !run_start[end - w0]) ++end;
      end = __builtin_amdgcn_readfirstlane(end);
      if (end - cur > 1 || !single_row(p.q2seq, cur, p.num_rows))
        prefill_tile<DT, HD, TPP, false, KV8>(p, cur, end - cur, p.q2seq[cur], kvh, h0, k_lds, v_lds, junk_lds, pid_lds,
                                         lim_lds, scl_lds);
      cur = end;
    }
  }
}

}  // namespace
}  // namespace pal
