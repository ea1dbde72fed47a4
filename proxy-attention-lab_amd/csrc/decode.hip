// Split-K paged-attention decode for gfx950.
//
// Reference behaviour: kernels/paged_attention/decode/paged_attention_decode.h.metal
// (one query row per sequence, GQA map h -> h / (Hq/Hkv) at :64-65, scale
// 1/sqrt(HD) at :115, length mask at :125-131 and :298-306) and the two-pass
// merge of decode/paged_reduce_decode.h.metal:79-128.
//
// Design (MI355X):
//  * One workgroup = 4 wavefronts = one (partition, kv head, head chunk,
//    sequence).  All query heads that share the kv head (up to 16 per chunk)
//    are processed together, so every K/V page block is read from HBM once per
//    GQA group instead of once per query head.
//  * The unit of work is a 16-token block (one page for TPP=16, half a page
//    for TPP=32).  Wave w of the workgroup takes blocks w, w+4, w+8, ... of the
//    partition.
//  * QK^T runs on MFMA as S^T = K * Q^T with v_mfma_f32_16x16x32: the A operand
//    is the K page block exactly as it lies in the striped pool layout
//    [HD/8][TPP][8] -- lane l loads the 16-byte stripe (l/16 + 4kk) of token
//    l%16, so 64 lanes read 1 KiB contiguous per instruction.  The result
//    leaves head l%16 and tokens 4(l/16)..+3 in lane l, which is exactly the A
//    operand layout of v_mfma_f32_16x16x16 for P*V, so probabilities never
//    cross lanes.  V is read as 8-byte runs of 4 tokens from the [HD][TPP]
//    layout.
//  * Softmax: scores of all blocks of the partition stay in registers; the
//    workgroup max is exchanged once through LDS, so there is no running
//    rescale.  Each partition writes either the final output (single
//    partition) or fp32 partials (max, exp-sum, unnormalised O) that the merge
//    kernel combines with a log-sum-exp reduction.
#include "pal_device.h"

namespace pal {

namespace {

constexpr int kNW = 4;  // wavefronts per workgroup

template <int DT, int HD, int TPP, int BPW>
__global__ __launch_bounds__(kNW * kWave) void decode_partition_kernel(const DecodeParams p) {
  constexpr bool kK32 = (HD % 32) == 0;  // QK k-step of 32 (else 16)
  constexpr int KK = kK32 ? HD / 32 : HD / 16;
  constexpr int NT = HD / 16;            // PV output tiles of 16 dims
  extern __shared__ float smem[];        // [kNW][hg][HD] partial outputs
  __shared__ float red_m[kNW][16];
  __shared__ float red_l[kNW][16];

  const int part = blockIdx.x;
  const int kvh = blockIdx.y / p.head_chunks;
  const int h0 = (blockIdx.y % p.head_chunks) * 16;
  const int hg = min(16, p.group - h0);
  const int64_t s = blockIdx.z;
  const int qh_base = kvh * p.group + h0;
  const int64_t max_tokens = p.page_table_width * TPP;
  const int len = static_cast<int>(min<int64_t>(max<int32_t>(p.seq_lens[s], 0), max_tokens));

  const int lane = lane_id();
  const int g = lane >> 4;
  const int r16 = lane & 15;
  const int w = wave_id();

  const int blocks_seq = (len + 15) >> 4;
  constexpr int kBlocksPart = kNW * BPW;
  const int nparts = (blocks_seq + kBlocksPart - 1) / kBlocksPart;

  if (len == 0) {
    if (part == 0) {
      for (int idx = threadIdx.x; idx < hg * HD; idx += kNW * kWave) {
        p.out[(s * p.num_q_heads + qh_base + idx / HD) * HD + idx % HD] = 0;
      }
    }
    return;
  }
  if (part >= nparts) return;

  // Q^T operand: lane holds Q[head r16][k-slice of this lane] for every k-step.
  u32x4 qv4[kK32 ? KK : 1];
  u32x2 qv2[kK32 ? 1 : KK];
  {
    const bool hv = r16 < hg;
    const uint16_t* qrow = p.q + (s * p.num_q_heads + qh_base + (hv ? r16 : 0)) * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if constexpr (kK32) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        qv4[kk] = hv ? *reinterpret_cast<const u32x4*>(qrow + 32 * kk + 8 * g) : z;
      } else {
        const u32x2 z = {0u, 0u};
        qv2[kk] = hv ? *reinterpret_cast<const u32x2*>(qrow + 16 * kk + 4 * g) : z;
      }
    }
  }

  const int64_t head_block = static_cast<int64_t>(HD) * TPP;  // elements per (page, kv head)
  const int64_t page_stride = head_block * p.num_kv_heads;
  const uint16_t* kbase = p.k_pool + kvh * head_block;
  const uint16_t* vbase = p.v_pool + kvh * head_block;
  const uint32_t* pt = p.page_table + s * p.page_table_width;
  const int b_first = part * kBlocksPart;

  // ---- S^T = K * Q^T for every block of this wave -------------------------
  f32x4 sc[BPW];
  float mloc = -INFINITY;
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int b = b_first + j * kNW + w;
    const float ninf = -INFINITY;
    sc[j] = f32x4{ninf, ninf, ninf, ninf};
    if (b < blocks_seq) {
      const uint32_t page = pt[(b * 16) / TPP];
      if (page < p.num_pages) {
        const int slot0 = (b * 16) % TPP;
        const uint16_t* kp = kbase + static_cast<int64_t>(page) * page_stride;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          if constexpr (kK32) {
            const int c = 4 * kk + g;  // stripe holding dims 32kk + 8g .. +7
            const u32x4 kv = *reinterpret_cast<const u32x4*>(kp + (c * TPP + slot0 + r16) * 8);
            acc = Dt<DT>::mma16x16x32(kv, qv4[kk], acc);
          } else {
            const int d = 16 * kk + 4 * g;  // dims d .. d+3
            const u32x2 kv = *reinterpret_cast<const u32x2*>(
                kp + ((d >> 3) * TPP + slot0 + r16) * 8 + (d & 7));
            acc = Dt<DT>::mma16x16x16(kv, qv2[kk], acc);
          }
        }
        const int t0 = b * 16 + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[j][i] = (t0 + i < len) ? acc[i] : ninf;
          mloc = fmaxf(mloc, sc[j][i]);
        }
      }
    }
  }

  // ---- workgroup max per head ---------------------------------------------
  mloc = fmaxf(mloc, shfl_xor(mloc, 16));
  mloc = fmaxf(mloc, shfl_xor(mloc, 32));
  if (g == 0) red_m[w][r16] = mloc;
  __syncthreads();
  float m = red_m[0][r16];
#pragma unroll
  for (int ww = 1; ww < kNW; ++ww) m = fmaxf(m, red_m[ww][r16]);
  // A head whose every score is masked (all pages invalid) keeps m = -inf;
  // use 0 so that exp2 yields 0 instead of NaN.
  const float msc = (m == -INFINITY) ? 0.f : m * p.scale_log2;

  // ---- P = exp(S - m), O += P * V -----------------------------------------
  float lsum = 0.f;
  f32x4 o[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int b = b_first + j * kNW + w;
    if (b < blocks_seq) {
      const uint32_t page = pt[(b * 16) / TPP];
      if (page < p.num_pages) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          e[i] = __builtin_amdgcn_exp2f(fmaf(sc[j][i], p.scale_log2, -msc));
          lsum += e[i];
        }
        const u32x2 pa = {Dt<DT>::pack2(e[0], e[1]), Dt<DT>::pack2(e[2], e[3])};
        const int slot0 = (b * 16) % TPP;
        const uint16_t* vp = vbase + static_cast<int64_t>(page) * page_stride + slot0 + 4 * g;
        const int t0 = b * 16 + 4 * g;
        const bool tail = (b * 16 + 16) > len;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          u32x2 vv = *reinterpret_cast<const u32x2*>(vp + (16 * n + r16) * TPP);
          // Slots past the sequence end may hold anything (NaN bits included):
          // zero them so that 0 * garbage cannot poison the sum.
          if (tail) vv = mask4(vv, t0 < len, t0 + 1 < len, t0 + 2 < len, t0 + 3 < len);
          o[n] = Dt<DT>::mma16x16x16(pa, vv, o[n]);
        }
      }
    }
  }

  // ---- combine the 4 waves --------------------------------------------------
  lsum += shfl_xor(lsum, 16);
  lsum += shfl_xor(lsum, 32);
  if (g == 0) red_l[w][r16] = lsum;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * g + i;
      if (h < hg) smem[(w * hg + h) * HD + 16 * n + r16] = o[n][i];
    }
  }
  __syncthreads();

  for (int idx = threadIdx.x; idx < hg * HD; idx += kNW * kWave) {
    const int h = idx / HD;
    const int d = idx - h * HD;
    float acc = smem[h * HD + d];
    float l = red_l[0][h];
    float mh = red_m[0][h];
#pragma unroll
    for (int ww = 1; ww < kNW; ++ww) {
      acc += smem[(ww * hg + h) * HD + d];
      l += red_l[ww][h];
      mh = fmaxf(mh, red_m[ww][h]);
    }
    const int64_t row = s * p.num_q_heads + qh_base + h;
    if (nparts == 1) {
      p.out[row * HD + d] = Dt<DT>::from_f32(l > 0.f ? acc / l : 0.f);
    } else {
      const int64_t slot = row * p.max_parts + part;
      p.part_o[slot * HD + d] = acc;
      if (d == 0) {
        p.part_ml[slot * 2 + 0] = (mh == -INFINITY) ? -INFINITY : mh * p.scale_log2;
        p.part_ml[slot * 2 + 1] = l;
      }
    }
  }
}

// Log-sum-exp merge of the partitions of one (sequence, query head) per
// wavefront: M = max_c m_c, out = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c.
template <int DT, int HD, int TPP, int BPW>
__global__ __launch_bounds__(kNW * kWave) void decode_merge_kernel(const DecodeParams p) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kNW + wave_id();
  if (row >= p.num_seqs * p.num_q_heads) return;
  const int64_t s = row / p.num_q_heads;
  const int64_t max_tokens = p.page_table_width * TPP;
  const int len = static_cast<int>(min<int64_t>(max<int32_t>(p.seq_lens[s], 0), max_tokens));
  constexpr int kBlocksPart = kNW * BPW;
  const int nparts = (((len + 15) >> 4) + kBlocksPart - 1) / kBlocksPart;
  if (nparts <= 1) return;
  const float* ml = p.part_ml + row * p.max_parts * 2;
  float big_m = -INFINITY;
  for (int c = 0; c < nparts; ++c) big_m = fmaxf(big_m, ml[2 * c]);
  if (big_m == -INFINITY) big_m = 0.f;
  float big_l = 0.f;
  for (int c = 0; c < nparts; ++c) big_l += ml[2 * c + 1] * __builtin_amdgcn_exp2f(ml[2 * c] - big_m);
  const float inv_l = big_l > 0.f ? 1.f / big_l : 0.f;
  const float* po = p.part_o + row * p.max_parts * HD;
  const int lane = lane_id();
  constexpr int kPer = (HD + kWave - 1) / kWave;
  float acc[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) acc[e] = 0.f;
  for (int c = 0; c < nparts; ++c) {
    const float wgt = __builtin_amdgcn_exp2f(ml[2 * c] - big_m);
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int d = lane + e * kWave;
      if (d < HD) acc[e] += wgt * po[c * HD + d];
    }
  }
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int d = lane + e * kWave;
    if (d < HD) p.out[row * HD + d] = Dt<DT>::from_f32(acc[e] * inv_l);
  }
}

template <int DT, int HD, int TPP, int BPW>
hipError_t launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  const int hg_max = p.group < 16 ? p.group : 16;
  const size_t smem = static_cast<size_t>(kNW) * hg_max * HD * sizeof(float);
  const dim3 grid(p.max_parts, p.num_kv_heads * p.head_chunks, static_cast<unsigned>(p.num_seqs));
  hipLaunchKernelGGL((decode_partition_kernel<DT, HD, TPP, BPW>), grid, dim3(kNW * kWave), smem,
                     stream, p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.max_parts <= 1) return err;
  const int64_t rows = p.num_seqs * p.num_q_heads;
  const dim3 mgrid(static_cast<unsigned>((rows + kNW - 1) / kNW));
  hipLaunchKernelGGL((decode_merge_kernel<DT, HD, TPP, BPW>), mgrid, dim3(kNW * kWave), 0, stream,
                     p);
  return hipGetLastError();
}

template <int DT, int HD, int TPP>
hipError_t dispatch_bpw(const DecodeParams& p, int bpw, hipStream_t stream) {
  switch (bpw) {
    case 2: return launch_decode_t<DT, HD, TPP, 2>(p, stream);
    case 4: return launch_decode_t<DT, HD, TPP, 4>(p, stream);
    case 8: return launch_decode_t<DT, HD, TPP, 8>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int DT, int HD>
hipError_t dispatch_tpp(const DecodeParams& p, int tpp, int bpw, hipStream_t stream) {
  switch (tpp) {
    case 16: return dispatch_bpw<DT, HD, 16>(p, bpw, stream);
    case 32: return dispatch_bpw<DT, HD, 32>(p, bpw, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t dispatch_hd(const DecodeParams& p, int hd, int tpp, int bpw, hipStream_t stream) {
  switch (hd) {
    case 32: return dispatch_tpp<DT, 32>(p, tpp, bpw, stream);
    case 64: return dispatch_tpp<DT, 64>(p, tpp, bpw, stream);
    case 80: return dispatch_tpp<DT, 80>(p, tpp, bpw, stream);
    case 96: return dispatch_tpp<DT, 96>(p, tpp, bpw, stream);
    case 128: return dispatch_tpp<DT, 128>(p, tpp, bpw, stream);
    case 256: return dispatch_tpp<DT, 256>(p, tpp, bpw, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_decode(const DecodeParams& p, int dtype, int head_dim, int tokens_per_page,
                         int blocks_per_wave, hipStream_t stream) {
  if (dtype == kBF16) return dispatch_hd<kBF16>(p, head_dim, tokens_per_page, blocks_per_wave, stream);
  return dispatch_hd<kF16>(p, head_dim, tokens_per_page, blocks_per_wave, stream);
}

}  // namespace pal
