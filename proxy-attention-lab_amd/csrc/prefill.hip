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
//    striped layout) and V (as [HD][32 + pad]) in LDS, double buffered, then
//    each wavefront computes S^T = K * Q^T with v_mfma_f32_32x32x16 (A = K
//    from LDS, B = Q^T held in registers) and O^T += V^T * P^T with the same
//    instruction.  In the transposed products a lane owns one M-row, so the
//    softmax max / sum need one cross-half exchange and the probabilities go
//    into the PV MFMA without leaving the lane.
//  * Online softmax in log2 units with a lazy rescale: the running max is only
//    moved when a score exceeds it by more than 2^8, so O is rescaled rarely.
//  * Causal skipping: the key loop stops at the tile's largest limit, and key
//    steps below every row's limit skip the mask arithmetic.
//  * Two ways to name the work: a device-built list of tiles (the fused op;
//    a persistent grid walks it), or the reference prefill's uniform prompt
//    (S sequences x P prompt rows; tiles are pure arithmetic).  In the second
//    mode keys [0, hist[s]) come from pages and keys hist[s] + i from the
//    dense prompt K/V rows s*P + i, as prefill.h.metal:147-234 reads them.
#include "pal_device.h"

namespace pal {

namespace {

constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kMRows = kPfWaves * 32;  // M-rows (token, head) per workgroup
constexpr int kKeys = 32;              // keys per step
constexpr int kVPad = 8;               // extra elements per V row in LDS (bank spread)
constexpr float kLazyRescale = 8.f;    // log2 headroom before the running max moves

template <int DT, int HD, int TPP>
__device__ __forceinline__ void prefill_tile(const PrefillParams& p, int tile, int kvh, int h0, uint16_t* k_lds_base,
                                             uint16_t* v_lds_base, int* lim_lds) {
  static_assert(HD % 32 == 0, "prefill needs head_dim % 32 == 0");
  constexpr int KS = HD / 16;  // QK k-steps of 16
  constexpr int DT32 = HD / 32;  // O^T row tiles of 32 dims
  constexpr int kVRow = kKeys + kVPad;
  constexpr int NB = HD <= 128 ? 2 : 1;  // LDS buffers (double buffering up to HD 128)
  auto k_lds = [&](int b) { return k_lds_base + b * HD * kKeys; };
  auto v_lds = [&](int b) { return v_lds_base + b * HD * kVRow; };

  const int hg = min(16, p.group - h0);  // heads of this chunk
  const int qt = kMRows / p.hg_max;      // tokens per tile (hg_max = min(group, 16))
  int row0, nrows;
  int64_t s;
  int64_t hist = 0;  // uniform-prompt mode: keys below hist come from pages
  if (p.prompt_len > 0) {
    const int tps = (p.prompt_len + qt - 1) / qt;
    s = tile / tps;
    const int j = tile - static_cast<int>(s) * tps;
    row0 = static_cast<int>(s) * p.prompt_len + j * qt;
    nrows = min(qt, p.prompt_len - j * qt);
  } else {
    row0 = p.tiles[3 * tile + 0];
    nrows = p.tiles[3 * tile + 1];
    s = static_cast<uint32_t>(p.tiles[3 * tile + 2]);
  }
  const bool seq_ok = s < p.num_seqs;  // a row naming no sequence attends to nothing
  if (!seq_ok) s = 0;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int w = wave_id();
  const int col = lane & 31;  // this lane's M-row within the wave
  const int half = lane >> 5;

  const int64_t max_tokens = p.page_table_width * TPP;
  int64_t slen;
  if (p.prompt_len > 0) {
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
      int64_t off = p.prompt_len > 0 ? hist + (row0 + t - s * p.prompt_len) + 1 : p.q_offset[row0 + t];
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

  // Cooperative load of keys [k0, k0+32) into LDS buffer `buf`; keys past the
  // tile's largest limit get zeros (and their scores are masked).
  auto stage = [&](int k0, int buf) {
    uint16_t* kl = k_lds(buf);
    uint16_t* vl = v_lds(buf);
    // K: 32 keys x HD/8 stripes of 16 B; thread -> (stripe, key), keys fastest.
    for (int i = tid; i < kKeys * (HD / 8); i += kPfThreads) {
      const int j = i % kKeys;
      const int c = i / kKeys;
      const int tok = k0 + j;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (tok < max_lim) {
        if (tok < hist || p.prompt_len == 0) {
          const uint32_t pg = pt[tok / TPP];
          const int64_t off = kvh * head_block + (static_cast<int64_t>(c) * TPP + tok % TPP) * 8;
          if (pg < p.num_pages)
            val = *reinterpret_cast<const u32x4*>(p.k_pool + static_cast<int64_t>(pg) * page_stride + off);
        } else {
          val = *reinterpret_cast<const u32x4*>(p.k_dense + (dense_row0 + tok) * dense_stride + kvh * HD + c * 8);
        }
      }
      *reinterpret_cast<u32x4*>(kl + (c * kKeys + j) * 8) = val;
    }
    // V: HD rows x 32 keys; thread -> (row d, 8-key group), 16 B per load.
    for (int i = tid; i < HD * (kKeys / 8); i += kPfThreads) {
      const int grp = i % (kKeys / 8);
      const int d = i / (kKeys / 8);
      const int tok = k0 + grp * 8;  // 8 keys, all in one page (TPP % 8 == 0)
      u32x4 val = {0u, 0u, 0u, 0u};
      if (tok < max_lim) {
        if (tok + 8 <= hist || p.prompt_len == 0) {
          const uint32_t pg = pt[tok / TPP];
          const int64_t off = kvh * head_block + static_cast<int64_t>(d) * TPP + tok % TPP;
          if (pg < p.num_pages)
            val = *reinterpret_cast<const u32x4*>(p.v_pool + static_cast<int64_t>(pg) * page_stride + off);
        } else {
          // some of the 8 keys are prompt tokens (dense, strided by row)
          uint16_t e16[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int t2 = tok + e;
            uint16_t x = 0;
            if (t2 < max_lim) {
              if (t2 < hist) {
                const uint32_t pg = pt[t2 / TPP];
                const int64_t off = kvh * head_block + static_cast<int64_t>(d) * TPP + t2 % TPP;
                if (pg < p.num_pages) x = p.v_pool[static_cast<int64_t>(pg) * page_stride + off];
              } else {
                x = p.v_dense[(dense_row0 + t2) * dense_stride + kvh * HD + d];
              }
            }
            e16[e] = x;
          }
          val = {static_cast<uint32_t>(e16[0]) | (static_cast<uint32_t>(e16[1]) << 16),
                 static_cast<uint32_t>(e16[2]) | (static_cast<uint32_t>(e16[3]) << 16),
                 static_cast<uint32_t>(e16[4]) | (static_cast<uint32_t>(e16[5]) << 16),
                 static_cast<uint32_t>(e16[6]) | (static_cast<uint32_t>(e16[7]) << 16)};
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
      }
      *reinterpret_cast<u32x4*>(vl + d * kVRow + grp * 8) = val;
    }
  };

  float m_run = -INFINITY;  // running max of this lane's M-row, log2 units
  float l_run = 0.f;        // this lane's share of the exp-sum
  f32x16 o[DT32];
#pragma unroll
  for (int n = 0; n < DT32; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[n][r] = 0.f;

  const int nsteps = (max_lim + kKeys - 1) / kKeys;
  if (nsteps > 0) stage(0, 0);
  for (int st = 0; st < nsteps; ++st) {
    const int buf = NB == 2 ? (st & 1) : 0;
    const int k0 = st * kKeys;
    __syncthreads();  // buffer `buf` is staged; the other one is free
    if (NB == 2 && st + 1 < nsteps) stage(k0 + kKeys, buf ^ 1);

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
    // lane holds keys k0 + 8 (r/4) + 4 half + r%4 of M-row col
    float sv[16];
    float bm = -INFINITY;
    const bool need_mask = k0 + kKeys > min_lim;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
      float x = sacc[r] * p.scale_log2;
      if (need_mask && key >= my_lim) x = -INFINITY;
      sv[r] = x;
      bm = fmaxf(bm, x);
    }
    bm = fmaxf(bm, shfl_xor(bm, 32));
    if (__ballot(bm > m_run + kLazyRescale)) {
      const float m_new = fmaxf(m_run, bm);
      const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
      // rows whose max did not grow keep alpha = 1 via m_new == m_run
      const float a = (bm > m_run + kLazyRescale) ? alpha : 1.f;
      if (bm > m_run + kLazyRescale) m_run = m_new;
      l_run *= a;
#pragma unroll
      for (int n = 0; n < DT32; ++n) o[n] *= a;
    }
    const float mb = (m_run == -INFINITY) ? 0.f : m_run;
    float pe[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      pe[r] = __builtin_amdgcn_exp2f(sv[r] - mb);
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
    if (NB == 1 && st + 1 < nsteps) {
      __syncthreads();  // everyone is done reading the single buffer
      stage(k0 + kKeys, 0);
    }
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

// grid.y = kv heads x head chunks; grid.x walks the tiles (uniform-prompt
// mode: exactly one tile per workgroup; list mode: a persistent stride over
// the device-built list, whose length is read from the workspace).
template <int DT, int HD, int TPP>
__global__ __launch_bounds__(kPfThreads) void prefill_tile_kernel(const PrefillParams p) {
  constexpr int NB = HD <= 128 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[NB * HD * kKeys];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[NB * HD * (kKeys + kVPad)];
  __shared__ int lim_lds[kMRows];
  const int kvh = blockIdx.y / p.head_chunks;
  const int h0 = (blockIdx.y % p.head_chunks) * 16;
  const int n_tiles = p.prompt_len > 0 ? p.num_tiles : *p.num_tiles_dev;
  for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x)
    prefill_tile<DT, HD, TPP>(p, tile, kvh, h0, k_lds, v_lds, lim_lds);
}

template <int DT, int HD, int TPP>
hipError_t launch_prefill_t(const PrefillParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.num_tiles), static_cast<unsigned>(p.num_kv_heads * p.head_chunks));
  hipLaunchKernelGGL((prefill_tile_kernel<DT, HD, TPP>), grid, dim3(kPfThreads), 0, stream, p);
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

template <int DT>
const void* prefill_kernel_for(int hd, int tpp) {
  const bool t32 = tpp == 32;
  switch (hd) {
    case 32: return t32 ? (const void*)&prefill_tile_kernel<DT, 32, 32> : (const void*)&prefill_tile_kernel<DT, 32, 16>;
    case 64: return t32 ? (const void*)&prefill_tile_kernel<DT, 64, 32> : (const void*)&prefill_tile_kernel<DT, 64, 16>;
    case 96: return t32 ? (const void*)&prefill_tile_kernel<DT, 96, 32> : (const void*)&prefill_tile_kernel<DT, 96, 16>;
    case 128:
      return t32 ? (const void*)&prefill_tile_kernel<DT, 128, 32> : (const void*)&prefill_tile_kernel<DT, 128, 16>;
    case 256:
      return t32 ? (const void*)&prefill_tile_kernel<DT, 256, 32> : (const void*)&prefill_tile_kernel<DT, 256, 16>;
    default: return nullptr;
  }
}

}  // namespace

hipError_t prefill_resident_groups(int dtype, int head_dim, int tokens_per_page, int* groups) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  int cus = 0;
  err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err != hipSuccess) return err;
  const void* fn = dtype == kBF16 ? prefill_kernel_for<kBF16>(head_dim, tokens_per_page)
                                  : prefill_kernel_for<kF16>(head_dim, tokens_per_page);
  if (!fn) return hipErrorInvalidValue;
  int per_cu = 0;
  err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kPfThreads, 0);
  if (err != hipSuccess) return err;
  *groups = cus * (per_cu < 1 ? 1 : per_cu);
  return hipSuccess;
}

int prefill_tokens_per_tile(int group) { return kMRows / (group < 16 ? group : 16); }

hipError_t launch_prefill(const PrefillParams& p, int dtype, int head_dim, int tokens_per_page, hipStream_t stream) {
  if (p.num_tiles <= 0) return hipSuccess;
  if (dtype == kBF16) return prefill_hd<kBF16>(p, head_dim, tokens_per_page, stream);
  return prefill_hd<kF16>(p, head_dim, tokens_per_page, stream);
}

}  // namespace pal
