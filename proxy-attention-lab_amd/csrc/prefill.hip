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
//  * Per 32-key step the workgroup stages K (as [HD/8][32][8], the page's own
//    striped layout) and V (as [HD][32 + pad]) in LDS, double buffered, with
//    the global loads of the next step held in registers during the compute
//    (one barrier per step); then
//    each wavefront computes S^T = K * Q^T with v_mfma_f32_32x32x16 (A = K
//    from LDS, B = Q^T held in registers) and O^T += V^T * P^T with the same
//    instruction.  In the transposed products a lane owns one M-row, so the
//    softmax max / sum need one cross-half exchange and the probabilities go
//    into the PV MFMA without leaving the lane.
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
#include "pal_device.h"

namespace pal {

namespace {

constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kMRows = kPfWaves * 32;  // M-rows (token, head) per workgroup
constexpr int kKeys = 32;              // keys per step
constexpr int kVPad = 8;               // extra elements per V row in LDS (bank spread)
constexpr float kLazyRescale = 8.f;    // log2 headroom before the running max moves

// Global -> register staging of one 32-key step: K as HD/8 stripes x 32 keys
// and V as HD rows x 4 groups of 8 keys, 16 bytes per load, spread over the
// workgroup's 256 threads.
template <int HD>
struct StepRegs {
  static constexpr int kLoads = (HD * 4 + kPfThreads - 1) / kPfThreads;  // K (and V) loads per thread
  u32x4 k[kLoads];
  u32x4 v[kLoads];
  int v_valid[kLoads];  // keys of the V group below the tile's largest limit (masked at store time)
};

// One query tile: rows [row0, row0 + nrows) of sequence s (nrows <= tokens
// per tile), query heads h0 .. h0+15 of kv head kvh.  `hist` >= 0 selects the
// uniform-prompt mode (keys below hist from pages, the rest from the dense
// prompt rows of sequence s); hist < 0: every key from pages.
template <int DT, int HD, int TPP, bool PROMPT>
__device__ __forceinline__ void prefill_tile(const PrefillParams& p, int row0, int nrows, int64_t s, int kvh, int h0,
                                             uint16_t* k_lds_base, uint16_t* v_lds_base, int* lim_lds) {
  static_assert(HD % 32 == 0, "prefill needs head_dim % 32 == 0");
  constexpr int KS = HD / 16;  // QK k-steps of 16
  constexpr int DT32 = HD / 32;  // O^T row tiles of 32 dims
  constexpr int kVRow = kKeys + kVPad;
  constexpr int NL = StepRegs<HD>::kLoads;
  auto k_lds = [&](int b) { return k_lds_base + b * HD * kKeys; };
  auto v_lds = [&](int b) { return v_lds_base + b * HD * kVRow; };

  // tile coordinates are workgroup-uniform: keep them in scalar registers so
  // page-table reads are scalar loads
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

  const int64_t max_tokens = p.page_table_width * TPP;
  int64_t hist = 0;  // prompt mode: keys below hist come from pages
  int64_t slen;
  if (prompt_mode) {
    hist = p.seq_lens[s];
    hist = hist < 0 ? 0 : (hist > max_tokens ? max_tokens : hist);
    slen = hist + p.prompt_len;
  } else {
    slen = seq_ok ? p.seq_lens[s] : 0;
    slen = slen < 0 ? 0 : (slen > max_tokens ? max_tokens : slen);
  }

  // Row limits: M-row m = token * hg_max + head.
  __syncthreads();  // the previous tile is done with lim_lds and the K/V buffers
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
  }
  __syncthreads();
  int max_lim = 0, min_lim = 1 << 30;
  for (int i = 0; i < kMRows; ++i) {  // uniform LDS broadcast reads
    const int t = i / p.hg_max;
    const int hh = i % p.hg_max;
    if (t < nrows && t < qt && hh < hg) {
      max_lim = max(max_lim, lim_lds[i]);
      min_lim = min(min_lim, lim_lds[i]);
    }
  }
  max_lim = __builtin_amdgcn_readfirstlane(max_lim);
  min_lim = __builtin_amdgcn_readfirstlane(min_lim);
  const int m_row = w * 32 + col;  // this lane's M-row
  const int my_t = m_row / p.hg_max;
  const int my_h = m_row % p.hg_max;
  const bool row_ok = my_t < nrows && my_t < qt && my_h < hg;
  const int my_lim = lim_lds[m_row];

  // Q^T operand: lane holds Q[M-row col][16kk + 8 half .. +7] for all k-steps.
  u32x4 qv[KS];
  {
    const int64_t qrow = static_cast<int64_t>(row0 + (row_ok ? my_t : 0)) * p.num_q_heads + kvh * p.group + h0 +
                         (row_ok ? my_h : 0);
    const uint16_t* qp = p.q + qrow * HD + 8 * half;
    const uint32_t qmask = row_ok ? 0xFFFFFFFFu : 0u;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qv[kk] = *reinterpret_cast<const u32x4*>(qp + 16 * kk) & qmask;
  }

  const int64_t head_block = static_cast<int64_t>(HD) * TPP;
  const int64_t page_stride = head_block * p.num_kv_heads;
  const uint32_t* pt = p.page_table + s * p.page_table_width;
  const int64_t dense_row0 = s * p.prompt_len - hist;  // dense row of key token tok: dense_row0 + tok
  const int64_t dense_stride = static_cast<int64_t>(p.num_kv_heads) * HD;

  // Page ids of the (at most two) pages holding keys [k0, k0+32): k0 is a
  // multiple of 32 and TPP of 16.  Loaded one pipeline stage before the K/V
  // loads that use them, so those never wait on a fresh load.
  auto load_pages = [&](int k0, uint32_t& pg0, uint32_t& pg1) {
    pg0 = pg1 = 0xFFFFFFFFu;
    if (p.page_table_width > 0) {
      const int64_t last = p.page_table_width - 1;
      const int64_t i0 = k0 / TPP;
      const int64_t i1 = (k0 + 16) / TPP;
      pg0 = pt[i0 < last ? i0 : last];
      pg1 = pt[i1 < last ? i1 : last];
    }
  };

  // A step moves 4*HD items of 16 bytes for K and as many for V; thread tid
  // takes items tid + 256 j.  With TPP = 16 the items are ordered page-major
  // (2*HD per page), and 2*HD is a multiple of 64, so every load instruction
  // of a wavefront reads one page: its base address is scalar and the
  // per-thread offset within the page never changes.
  //   K item: stripe c, key kj (0..31) -> LDS [c][kj][8]
  //   V item: row d, keys kg .. kg+7   -> LDS [d][kg .. kg+7]
  auto k_item = [&](int i, int& c, int& kj) {
    if (TPP == 16) {
      const int rem = i % (2 * HD);
      c = rem / 16;
      kj = (i / (2 * HD)) * 16 + rem % 16;
    } else {
      c = i / kKeys;
      kj = i % kKeys;
    }
  };
  auto v_item = [&](int i, int& d, int& kg) {
    if (TPP == 16) {
      const int rem = i % (2 * HD);
      d = rem / 2;
      kg = (i / (2 * HD)) * 16 + (rem % 2) * 8;
    } else {
      d = i / 4;
      kg = (i % 4) * 8;
    }
  };
  // page of load j of this wavefront (0: first page of the step, 1: second)
  auto load_page_sel = [&](int j) { return TPP == 16 ? (w * kWave + j * kPfThreads) / (2 * HD) : 0; };
  const int64_t kv_head_off = kvh * head_block;

  // Global loads of keys [k0, k0+32) into registers; keys past the tile's
  // largest limit read as zeros (and their scores are masked).
  auto load_step = [&](int k0, StepRegs<HD>& r, uint32_t pg0v, uint32_t pg1v) {
    const uint32_t pg0 = __builtin_amdgcn_readfirstlane(pg0v);
    const uint32_t pg1 = __builtin_amdgcn_readfirstlane(pg1v);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int i = tid + j * kPfThreads;
      const uint32_t pg = load_page_sel(j) ? pg1 : pg0;
      const bool pg_ok = pg < p.num_pages;
      const uint16_t* kpage = p.k_pool + static_cast<int64_t>(pg_ok ? pg : 0) * page_stride + kv_head_off;
      const uint16_t* vpage = p.v_pool + static_cast<int64_t>(pg_ok ? pg : 0) * page_stride + kv_head_off;
      int c, kj, d, kg;
      k_item(i, c, kj);
      v_item(i, d, kg);
      const bool item_ok = i < HD * 4;
      // K
      {
        u32x4 val = {0u, 0u, 0u, 0u};
        const int tok = k0 + kj;
        if (!prompt_mode || tok < hist) {
          if (item_ok && pg_ok && tok < max_lim)
            val = *reinterpret_cast<const u32x4*>(kpage + (c * TPP + kj % TPP) * 8);
        } else if (item_ok && tok < max_lim) {
          val = *reinterpret_cast<const u32x4*>(p.k_dense + (dense_row0 + tok) * dense_stride + kvh * HD + c * 8);
        }
        r.k[j] = val;
      }
      // V
      {
        u32x4 val = {0u, 0u, 0u, 0u};
        const int tok = k0 + kg;
        if (!prompt_mode || tok + 8 <= hist) {
          if (item_ok && pg_ok && tok < max_lim)
            val = *reinterpret_cast<const u32x4*>(vpage + d * TPP + kg % TPP);
        } else if (item_ok && tok < max_lim) {
          // some of the 8 keys are prompt tokens (dense, strided by row)
          uint32_t e16[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int t2 = tok + e;
            const bool pgd = t2 < hist;
            const uint16_t* src = pgd ? vpage + d * TPP + (kg + e) % TPP
                                      : p.v_dense + (dense_row0 + t2) * dense_stride + kvh * HD + d;
            uint16_t x = 0;
            if (t2 < max_lim && (!pgd || pg_ok)) x = *src;
            e16[e] = x;
          }
          val = {e16[0] | (e16[1] << 16), e16[2] | (e16[3] << 16), e16[4] | (e16[5] << 16), e16[6] | (e16[7] << 16)};
        }
        // keys past the largest limit may hold anything (NaN bits included);
        // they are zeroed when the registers go to LDS, so no wait here
        r.v_valid[j] = max_lim - tok;
        r.v[j] = val;
      }
    }
  };
  auto store_step = [&](const StepRegs<HD>& r, int buf) {
    uint16_t* kl = k_lds(buf);
    uint16_t* vl = v_lds(buf);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int i = tid + j * kPfThreads;
      if (i < HD * 4) {
        int c, kj, d, kg;
        k_item(i, c, kj);
        v_item(i, d, kg);
        *reinterpret_cast<u32x4*>(kl + (c * kKeys + kj) * 8) = r.k[j];
        u32x4 v = r.v[j];
        const int valid = r.v_valid[j];
        if (valid < 8) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t keep = (2 * e < valid ? 0x0000FFFFu : 0u) | (2 * e + 1 < valid ? 0xFFFF0000u : 0u);
            v[e] &= keep;
          }
        }
        *reinterpret_cast<u32x4*>(vl + d * kVRow + kg) = v;
      }
    }
  };

  float m_run = -INFINITY;  // running max of this lane's M-row (raw score units)
  float l_run = 0.f;        // this lane's share of the exp-sum
  f32x16 o[DT32];
#pragma unroll
  for (int n = 0; n < DT32; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[n][r] = 0.f;

  // Pipeline: while step st is computed from LDS, the K/V loads of step st+1
  // are in flight in registers and the page ids of step st+2 in two more;
  // after the compute the registers go to the other LDS buffer, the loads of
  // step st+2 and the page ids of step st+3 are issued, and one barrier ends
  // the step.
  const int nsteps = (max_lim + kKeys - 1) / kKeys;
  StepRegs<HD> regs;
  uint32_t pga = 0xFFFFFFFFu, pgb = 0xFFFFFFFFu;
  if (nsteps > 0) {
    load_pages(0, pga, pgb);
    load_step(0, regs, pga, pgb);
    store_step(regs, 0);
    if (nsteps > 1) {
      load_pages(kKeys, pga, pgb);
      load_step(kKeys, regs, pga, pgb);
      if (nsteps > 2) load_pages(2 * kKeys, pga, pgb);
    }
  }
  __syncthreads();
  for (int st = 0; st < nsteps; ++st) {
    const int buf = st & 1;
    const int k0 = st * kKeys;

    // S^T[key][M-row] = sum_d K[key][d] Q[M-row][d]
    f32x16 sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int c = 2 * kk + half;  // stripe of dims 16kk + 8 half .. +7
      const u32x4 ka = *reinterpret_cast<const u32x4*>(k_lds(buf) + (c * kKeys + col) * 8);
      sacc = Dt<DT>::mma32x32x16(ka, qv[kk], sacc);
    }
    // lane holds keys k0 + 8 (r/4) + 4 half + r%4 of M-row col.  Scores stay
    // raw (the scale is positive, so maxima commute with it); the exponent is
    // one fma: s * scale_log2 - m * scale_log2.
    float bm = -INFINITY;
    if (k0 + kKeys > min_lim) {  // some key of this step is masked for some row
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (key >= my_lim) sacc[r] = -INFINITY;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) bm = fmaxf(bm, sacc[r]);
    bm = fmaxf(bm, shfl_xor(bm, 32));
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
    const float mb = (m_run == -INFINITY) ? 0.f : -m_run * p.scale_log2;
    float pe[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      pe[r] = __builtin_amdgcn_exp2f(fmaf(sacc[r], p.scale_log2, mb));
      l_run += pe[r];
    }
    // O^T[d][M-row] += sum_key V[key][d] P[M-row][key]; k-step kk covers the
    // keys held in registers 8kk .. 8kk+7: {16kk + 4 half + e, 16kk + 8 + 4 half + e}.
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const u32x4 pb = {Dt<DT>::pack2(pe[8 * kk + 0], pe[8 * kk + 1]), Dt<DT>::pack2(pe[8 * kk + 2], pe[8 * kk + 3]),
                        Dt<DT>::pack2(pe[8 * kk + 4], pe[8 * kk + 5]), Dt<DT>::pack2(pe[8 * kk + 6], pe[8 * kk + 7])};
#pragma unroll
      for (int n = 0; n < DT32; ++n) {
        const int d = 32 * n + col;
        const uint16_t* vrow = v_lds(buf) + d * kVRow + 16 * kk + 4 * half;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
        const u32x4 va = {lo.x, lo.y, hi.x, hi.y};
        o[n] = Dt<DT>::mma32x32x16(va, pb, o[n]);
      }
    }
    if (st + 1 < nsteps) {
      store_step(regs, buf ^ 1);  // buffer buf^1 was last read in step st-1, before the last barrier
      if (st + 2 < nsteps) {
        load_step(k0 + 2 * kKeys, regs, pga, pgb);
        if (st + 3 < nsteps) load_pages(k0 + 3 * kKeys, pga, pgb);
      }
    }
    __syncthreads();
  }

  // ---- normalise and write: lane holds O[M-row col][32n + 8(r/4) + 4 half + r%4]
  float l = l_run + shfl_xor(l_run, 32);
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

// 1-D grid, XCD-aware: block b serves head group g = b % G (G = kv heads x
// head chunks) and work unit b / G, so consecutive blocks -- which the
// dispatcher spreads over the 8 XCDs -- take different kv heads, and each kv
// head's K/V stay in few L2s.
//  * prompt mode: unit = (sequence, tile), the last tile of a sequence first
//    (it has the most keys);
//  * window mode (fused op): unit = window of `tokens per tile` rows; every
//    run of rows of one sequence inside the window that is not a lone decode
//    row is computed as a tile.
template <int DT, int HD, int TPP>
__global__ __launch_bounds__(kPfThreads) void prefill_tile_kernel(const PrefillParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2 * HD * kKeys];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2 * HD * (kKeys + kVPad)];
  __shared__ int lim_lds[kMRows];
  __shared__ int run_start[kMRows];
  const int G = p.num_kv_heads * p.head_chunks;
  const int g = static_cast<int>(blockIdx.x % static_cast<unsigned>(G));
  const int unit = static_cast<int>(blockIdx.x / static_cast<unsigned>(G));
  const int kvh = g / p.head_chunks;
  const int h0 = (g % p.head_chunks) * 16;
  const int qt = kMRows / p.hg_max;
  if (p.prompt_len > 0) {
    const int tps = (p.prompt_len + qt - 1) / qt;
    const int s = unit / tps;
    const int j = tps - 1 - (unit - s * tps);
    const int row0 = s * p.prompt_len + j * qt;
    prefill_tile<DT, HD, TPP, true>(p, row0, min(qt, p.prompt_len - j * qt), s, kvh, h0, k_lds, v_lds, lim_lds);
    return;
  }
  const int w0 = unit * qt;
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
      prefill_tile<DT, HD, TPP, false>(p, cur, end - cur, p.q2seq[cur], kvh, h0, k_lds, v_lds, lim_lds);
    cur = end;
  }
}

template <int DT, int HD, int TPP>
hipError_t launch_prefill_t(const PrefillParams& p, hipStream_t stream) {
  const int64_t blocks = static_cast<int64_t>(p.num_units) * p.num_kv_heads * p.head_chunks;
  hipLaunchKernelGGL((prefill_tile_kernel<DT, HD, TPP>), dim3(static_cast<unsigned>(blocks)), dim3(kPfThreads), 0,
                     stream, p);
  return hipGetLastError();
}

template <int DT, int HD>
hipError_t prefill_tpp(const PrefillParams& p, int tpp, hipStream_t stream) {
  switch (tpp) {
    case 16: return launch_prefill_t<DT, HD, 16>(p, stream);
    case 32: return launch_prefill_t<DT, HD, 32>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t prefill_hd(const PrefillParams& p, int hd, int tpp, hipStream_t stream) {
  switch (hd) {
    case 32: return prefill_tpp<DT, 32>(p, tpp, stream);
    case 64: return prefill_tpp<DT, 64>(p, tpp, stream);
    case 96: return prefill_tpp<DT, 96>(p, tpp, stream);
    case 128: return prefill_tpp<DT, 128>(p, tpp, stream);
    case 256: return prefill_tpp<DT, 256>(p, tpp, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int prefill_tokens_per_tile(int group) { return kMRows / (group < 16 ? group : 16); }

hipError_t launch_prefill(const PrefillParams& p, int dtype, int head_dim, int tokens_per_page, hipStream_t stream) {
  if (p.num_units <= 0) return hipSuccess;
  if (dtype == kBF16) return prefill_hd<kBF16>(p, head_dim, tokens_per_page, stream);
  return prefill_hd<kF16>(p, head_dim, tokens_per_page, stream);
}

}  // namespace pal
