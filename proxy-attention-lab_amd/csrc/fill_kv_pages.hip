// fill_kv_pages for gfx950: scatter of new K/V rows into the paged pools,
// optionally fused with the step that produces them (rotary position
// embedding of K, and of Q, plus the cast from the projection's fp32 or
// 16-bit output to the pool dtype, fp8 e4m3 pages quantized with
// per-(page, kv head) scales included).
//
// Reference behaviour: kernels/paged_attention/fill_kv_pages.h.metal:65-116 --
//   seq = q2seq[t], pos = write_pos[t], page = page_table[seq, pos / TPP],
//   slot = pos % TPP,
//   K[page, h, d / x, slot, d % x] = new_k[t, h, d]   (x = 16 / sizeof(element))
//   V[page, h, d, slot]            = new_v[t, h, d]
// a bit-exact copy when source and pool share the 16-bit dtype.
//
// Design (MI355X): HBM-bound byte movement, so the mapping is chosen for
// whole-line writes and short dependency chains.  Workgroup (w, h) owns a
// window of 64 consecutive new tokens (16 for small batches) and kv head h,
// K and V both (twice the bytes in flight per destination lookup).
// Its threads issue all their source loads first; meanwhile the first
// threads resolve every token's destination (page, slot) into LDS.
//  * K: a token's 8-dim chunk is one 16-byte stripe (16-bit pools) or half of
//    one (fp8), and consecutive slots of a page are consecutive stripes, so
//    lane i of a wavefront moves chunk c of token i: a prefill run writes
//    whole lines.
//  * V: row d of a (page, head) block holds the page's slots side by side, so
//    one token's value is a 2-byte (1-byte) piece of a row.  Wherever 8
//    consecutive window tokens fill an 8-aligned run of slots of one page
//    (a prefill chunk), their converted V rows are staged in LDS and a
//    thread gathers element d of the 8 tokens into one 16-byte (8-byte)
//    store of row d; the remaining tokens (decode fills, the ragged ends of
//    runs) are written element by element.
//  * RoPE: position = the token's write position; cos / sin come from the
//    caller's table [rows, rotary_dim] (cos of the rotary_dim / 2
//    frequencies, then their sin).  NeoX style pairs dims (f, f + rot/2);
//    GPT-J style pairs (2f, 2f + 1).  The products are rounded as written
//    (no fused multiply-add), so results are bit-exact against a scalar fp32
//    restatement.
//  * fp8: q = x / scale[page, h], held to [-448, 448] (NaN stays NaN), then
//    rounded to nearest even e4m3.
// Tokens whose destination falls outside the page table or the pool are
// skipped (the reference does not check and would write out of bounds).
#include "pal_device.h"

namespace pal {

// flag word of this translation unit's debug checks (see pal_device.h)
PAL_DEBUG_FLAGS_DEFINE(fill_debug_flags)

namespace {

#ifndef PAL_FILL_THREADS
#define PAL_FILL_THREADS 512  // eight wavefronts: fewer source chunks (registers) per thread
#endif
constexpr int kThreads = PAL_FILL_THREADS;
#ifndef PAL_FILL_LARGE_WIN
#define PAL_FILL_LARGE_WIN 64
#endif
#ifndef PAL_FILL_SMALL_WIN
#define PAL_FILL_SMALL_WIN 16
#endif
constexpr int kSmallWin = PAL_FILL_SMALL_WIN;
constexpr int kLargeWin = PAL_FILL_LARGE_WIN;  // window of prefill-sized batches (16 for small ones)
constexpr int kRowPad = 16;      // LDS row padding (bytes) of the staged K / V rows

// ---- source element access: 8 consecutive values as fp32 -------------------
template <int SRC>
__device__ __forceinline__ void load8(const void* base, int64_t elem, float (&x)[8]) {
  if constexpr (SRC == kF32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + elem);
    const f32x4 b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + elem + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + elem);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = Dt<SRC>::to_f32(static_cast<uint16_t>(w[e] & 0xFFFFu));
      x[2 * e + 1] = Dt<SRC>::to_f32(static_cast<uint16_t>(w[e] >> 16));
    }
  }
}

// ---- destination encodings ---------------------------------------------------
// fp8 e4m3 (OCP "fn" variant): x / scale held to the finite range, round to
// nearest even (v_cvt_pk_fp8_f32).
__device__ __forceinline__ float fp8_prescale(float x, float scale) {
  float q = x / scale;  // correctly rounded division
  q = q > 448.f ? 448.f : q;
  q = q < -448.f ? -448.f : q;  // NaN compares false and stays NaN
  return q;
}
__device__ __forceinline__ uint32_t fp8_pack4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return static_cast<uint32_t>(w);
}

template <int DST>
struct Store8;
template <>
struct Store8<kF16> {
  using T = u32x4;
  static __device__ __forceinline__ T pack(const float (&x)[8], float) {
    return T{Dt<kF16>::pack2(x[0], x[1]), Dt<kF16>::pack2(x[2], x[3]), Dt<kF16>::pack2(x[4], x[5]),
             Dt<kF16>::pack2(x[6], x[7])};
  }
};
template <>
struct Store8<kBF16> {
  using T = u32x4;
  static __device__ __forceinline__ T pack(const float (&x)[8], float) {
    return T{Dt<kBF16>::pack2(x[0], x[1]), Dt<kBF16>::pack2(x[2], x[3]), Dt<kBF16>::pack2(x[4], x[5]),
             Dt<kBF16>::pack2(x[6], x[7])};
  }
};
template <>
struct Store8<kFP8> {
  using T = u32x2;
  static __device__ __forceinline__ T pack(const float (&x)[8], float scale) {
    float q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = fp8_prescale(x[e], scale);
    return T{fp8_pack4(q[0], q[1], q[2], q[3]), fp8_pack4(q[4], q[5], q[6], q[7])};
  }
};

template <int DST>
constexpr int elem_bytes() { return DST == kFP8 ? 1 : 2; }

// Rotates the 8 values of chunk x (dims d0..d0+7) in place.  NeoX: y holds
// their partners (dims d0 + rot/2 ..) and is rotated too; GPT-J: the pairs
// sit inside the chunk.  cs: the position's row of the cos/sin table, f0 the
// chunk's first table index (NeoX d0, GPT-J d0 / 2).  Both styles run one
// unrolled body whose operands are selected by value: with a branch per
// style the compiler merged the two styles' stores behind a run-time address
// and put x and y on the stack.
#pragma clang fp contract(off)
__device__ __forceinline__ void rope_unit(float (&x)[8], float (&y)[8], const float* cs, int f0, int half, bool neox) {
  float xo[8], yo[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int f = f0 + (neox ? e : e >> 1);
    const float c = cs[f];
    const float s = cs[half + f];
    const float t = (neox ? y[e] : x[e ^ 1]) * s;
    xo[e] = x[e] * c + ((neox || (e & 1) == 0) ? -t : t);  // a c - b s, or b c + a s
    yo[e] = y[e] * c + x[e] * s;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = xo[e];
    y[e] = neox ? yo[e] : y[e];
  }
}
// Rotates the 4 values of a 16-byte piece (dims 4j..4j+3 of a head, j the
// piece index) in place.  NeoX: w holds the partner piece's values (j xor
// rot/8); GPT-J: the pairs sit inside the piece.  The products are those of
// rope_unit, rounded alike.
__device__ __forceinline__ void rope_piece(float (&v)[4], const float (&w)[4], const float* cs, int j, int style,
                                           int rot) {
  const int half = rot / 2;
  if (style == 1) {
    const int pr = rot / 8;
    if (j >= 2 * pr) return;  // past rotary_dim
    const bool lo = j < pr;
    const int d = 4 * (lo ? j : j - pr);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c = cs[d + e];
      const float s = cs[half + d + e];
      v[e] = lo ? v[e] * c - w[e] * s : v[e] * c + w[e] * s;
    }
  } else if (style == 2) {
    if (4 * j >= rot) return;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float c = cs[2 * j + q];
      const float s = cs[half + 2 * j + q];
      const float a = v[2 * q], b = v[2 * q + 1];
      v[2 * q] = a * c - b * s;
      v[2 * q + 1] = b * c + a * s;
    }
  }
}
// Rotates a pair of 16-byte pieces of one K row in place: x holds dims
// 4j..4j+3, y dims hd/2 + 4j .. +3.  NeoX (rotary_dim == hd): the two are
// each other's partners; GPT-J: the pairs sit inside each piece.  The
// products are those of rope_unit, rounded alike.
__device__ __forceinline__ void rope_piece_pair(float (&x)[4], float (&y)[4], const float* cs, int j, int style,
                                                int rot, int hd) {
  const int half = rot / 2;
  if (style == 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c = cs[4 * j + e];
      const float s = cs[half + 4 * j + e];
      const float a = x[e], b = y[e];
      x[e] = a * c - b * s;
      y[e] = b * c + a * s;
    }
  } else if (style == 2) {
#pragma unroll
    for (int side = 0; side < 2; ++side) {
      float(&v)[4] = side ? y : x;
      const int d0 = (side ? hd / 2 : 0) + 4 * j;
      if (d0 >= rot) continue;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const float c = cs[d0 / 2 + q];
        const float s = cs[half + d0 / 2 + q];
        const float a = v[2 * q], b = v[2 * q + 1];
        v[2 * q] = a * c - b * s;
        v[2 * q + 1] = b * c + a * s;
      }
    }
  }
}
#pragma clang fp contract(on)

// Stores chunk c (dims 8c..8c+7) of a token at `slot` of the K block that
// starts `hb` bytes into the pool.
template <int DST>
__device__ __forceinline__ void store_k_chunk(const FillParams& p, int64_t hb, int slot, int c,
                                              const typename Store8<DST>::T& v) {
  const int64_t tpp = p.tokens_per_page;
  uint8_t* base = static_cast<uint8_t*>(p.k_pool) + hb;
  if constexpr (DST == kFP8) {  // stripes of 16 dims: chunk c is half of stripe c / 2
    *reinterpret_cast<u32x2*>(base + ((c >> 1) * tpp + slot) * 16 + (c & 1) * 8) = v;
  } else {  // stripes of 8 dims
    *reinterpret_cast<u32x4*>(base + (c * tpp + slot) * 16) = v;
  }
}

// Source rows of 8 values as loaded: raw 16-bit words, or fp32.
template <int SRC>
struct Raw8 {
  u32x4 w;
  // non-temporal: each source row is read once.  Config 4 with its sources
  // cold (three rotated copies): 54.8 -> 48.1 us; the same call repeated on
  // one copy, whose rows the last-level cache could hold: 42.5 -> 48.2 us.
  __device__ __forceinline__ void load(const void* base, int64_t elem) {
    w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + elem));
  }
  __device__ __forceinline__ void to_f32(float (&x)[8]) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = Dt<SRC>::to_f32(static_cast<uint16_t>(w[e] & 0xFFFFu));
      x[2 * e + 1] = Dt<SRC>::to_f32(static_cast<uint16_t>(w[e] >> 16));
    }
  }
};
template <>
struct Raw8<kF32> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const void* base, int64_t elem) {
    a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + elem);
    b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + elem + 4);
  }
  __device__ __forceinline__ void to_f32(float (&x)[8]) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  }
};

// K work unit u of a row: NeoX rotation pairs chunk c with c + rot/16, so
// unit u < rot/16 is that pair; every other unit is one chunk.  Without
// NeoX pairs every unit is one chunk.
// (style: the call's rope style, 0 in the kernels compiled without RoPE)
__device__ __forceinline__ int k_units(const FillParams& p, int style) {
  return style == 1 ? p.head_dim / 8 - p.rotary_dim / 16 : p.head_dim / 8;
}
__device__ __forceinline__ void unit_chunks(const FillParams& p, int style, int u, int& c0, int& c1) {
  if (style == 1) {
    const int pairs = p.rotary_dim / 16;
    if (u < pairs) {
      c0 = u;
      c1 = u + pairs;
    } else {
      c0 = u + pairs;  // chunks at and past rotary_dim
      c1 = -1;
    }
  } else {
    c0 = u;
    c1 = -1;
  }
}

// Rotates the unit's chunk(s) in place (x: chunk c0, y: chunk c1 of a NeoX
// pair) with row `pos` of the table, when rotate.
__device__ __forceinline__ void rotate_unit(const FillParams& p, int style, int c0, int c1, int pos, bool rotate,
                                            float (&x)[8], float (&y)[8]) {
  if (!rotate || style == 0 || 8 * c0 >= p.rotary_dim) return;
  const float* cs = p.cos_sin + static_cast<int64_t>(pos) * p.rotary_dim;
  const bool neox = style == 1;
  if (neox && c1 < 0) return;
  rope_unit(x, y, cs, neox ? 8 * c0 : 4 * c0, p.rotary_dim / 2, neox);
}

// Workgroup (w, y) of the grid: y < Hkv moves K and V of kv head y for the
// window of WIN new tokens w * WIN ..; y >= Hkv (rope with queries only)
// rotates and casts query head y - Hkv of the window.  Each thread first
// issues the loads of all its source chunks, K and V, chunks fastest so that
// a wavefront reads whole lines of the source rows; meanwhile the first
// wavefront resolves the destinations (once for both) and classifies the
// window's tokens: a token inside a full run of 8 slots of one page, or a
// single token.  A single token's K chunks and V values are stored straight
// from registers.  Run tokens' rows go through LDS, and each run is then
// written in whole lines: K stripe q of its 8 slots (8 x 16 contiguous
// bytes) and V row d of its 8 slots, the two runs of one page side by side
// in neighbouring lanes.  ROPE false: the plain fill (no rotation, no
// queries), compiled without the rotation code.
template <int SRC, int DST, int WIN, int MAXC, bool ROPE>
__global__ __launch_bounds__(kThreads) void fill_kv_pages_kernel(const FillParams p) {
  constexpr int kItems = (WIN * MAXC + kThreads - 1) / kThreads;  // source chunks per thread, at most
  constexpr int EB = elem_bytes<DST>();
  static_assert(WIN <= kWave, "the first wavefront classifies the window");
  // dynamic LDS: the run tokens' K rows, then their V rows, [2][WIN][HD * EB + kRowPad] bytes
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
  __shared__ uint32_t page_lds[WIN];  // destination page of each window token
  __shared__ int slot_lds[WIN];       // its slot, or -1: no valid destination
  __shared__ int pos_lds[WIN];
  __shared__ float ks_lds[WIN], vs_lds[WIN];  // fp8 scales of each token's (page, head)
  __shared__ int kind_lds[WIN];       // 0: nothing to write, 1: single token, 2: in a full run
  __shared__ int run_lds[WIN / 8];    // window index of each full run's first token
  __shared__ int n_runs_lds;
  const int hd = p.head_dim;
  const int tpp = p.tokens_per_page;
  const int chunks = hd / 8;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * WIN;
  const int tid = threadIdx.x;
  const int nwin = static_cast<int>(min(static_cast<int64_t>(WIN), p.num_tokens - t0));
  const int style = ROPE ? p.rope_style : 0;
  const int units = k_units(p, style);

  if (ROPE && static_cast<int>(blockIdx.y) >= p.num_kv_heads) {
    // ---- queries: rotate and cast head qh of the window's rows (a row is
    // contiguous in and out, so units run fastest: whole lines per wave)
    const int qh = blockIdx.y - p.num_kv_heads;
    if constexpr (SRC == kF32) {
      // fp32 rows of head dims 32/64/128/256: 16-byte pieces, lane j of a
      // token's hd/4 lanes holding dims 4j..4j+3, so every load and store
      // instruction covers whole lines (8-value units store 16 bytes 32 bytes
      // apart: 1.48x the written bytes), with non-temporal loads and stores
      // (the rows pass once; kept in L2 they pushed out the cos/sin table,
      // which every head re-reads: 1.33x the read bytes)
      const int rot = p.rotary_dim;
      const bool hd_ok = hd == 32 || hd == 64 || hd == 128 || hd == 256;
      const bool rot_ok = style != 1 || (rot >= 8 && rot <= hd && (rot & (rot - 1)) == 0);
      if (hd_ok && rot_ok) {
        constexpr int kPieces = (WIN * 32 + kThreads - 1) / kThreads;  // per thread per round (hd <= 128)
        const int lpt = hd / 4;  // pieces of a row; divides the wavefront
        const int n_items = nwin * lpt;
        const int64_t q_row = static_cast<int64_t>(p.num_q_heads) * hd;
#pragma unroll 1
        for (int base = 0; base < n_items; base += kPieces * kThreads) {  // two rounds at hd 256
          f32x4 xq[kPieces];
          int pos[kPieces];
#pragma unroll
          for (int k = 0; k < kPieces; ++k) {
            const int it = base + tid + k * kThreads;
            xq[k] = f32x4{0.f, 0.f, 0.f, 0.f};
            pos[k] = -1;
            if (it < n_items) {
              const int i = it / lpt;
              xq[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(
                  static_cast<const float*>(p.q_in) + (t0 + i) * q_row + static_cast<int64_t>(qh) * hd + 4 * (it % lpt)));
              pos[k] = p.write_pos[t0 + i];
            }
          }
#pragma unroll
          for (int k = 0; k < kPieces; ++k) {
            const int it = base + tid + k * kThreads;
            float v[4] = {xq[k][0], xq[k][1], xq[k][2], xq[k][3]};
            float w[4] = {0.f, 0.f, 0.f, 0.f};
            if (style == 1) {  // every lane takes part (a token's lanes are valid together)
#pragma unroll
              for (int e = 0; e < 4; ++e) w[e] = __shfl_xor(v[e], rot / 8, kWave);
            }
            if (it < n_items) {
              const int i = it / lpt;
              const int j = it % lpt;
              if (style != 0 && pos[k] >= 0 && pos[k] < p.cos_sin_rows)
                rope_piece(v, w, p.cos_sin + static_cast<int64_t>(pos[k]) * rot, j, style, rot);
              const u32x2 packed = p.q_out_dtype == kBF16
                                       ? u32x2{Dt<kBF16>::pack2(v[0], v[1]), Dt<kBF16>::pack2(v[2], v[3])}
                                       : u32x2{Dt<kF16>::pack2(v[0], v[1]), Dt<kF16>::pack2(v[2], v[3])};
              __builtin_nontemporal_store(packed, reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.q_out) +
                                                                         (t0 + i) * q_row +
                                                                         static_cast<int64_t>(qh) * hd + 4 * j));
            }
          }
        }
        return;
      }
    }
    const int64_t q_row = static_cast<int64_t>(p.num_q_heads) * hd;
    Raw8<SRC> rx[kItems], ry[kItems];
    int pos[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
      const int it = tid + k * kThreads;
      const int i = it / units;
      if (i < nwin) {
        int c0, c1;
        unit_chunks(p, style, it % units, c0, c1);
        const int64_t row = (t0 + i) * q_row + static_cast<int64_t>(qh) * hd;
        rx[k].load(p.q_in, row + 8 * c0);
        if (c1 >= 0) ry[k].load(p.q_in, row + 8 * c1);
        pos[k] = p.write_pos[t0 + i];
      }
    }
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
      const int it = tid + k * kThreads;
      const int i = it / units;
      if (i >= nwin) continue;
      int c0, c1;
      unit_chunks(p, style, it % units, c0, c1);
      float x[8], y[8];
      rx[k].to_f32(x);
      if (c1 >= 0) ry[k].to_f32(y);
      rotate_unit(p, style, c0, c1, pos[k], pos[k] >= 0 && pos[k] < p.cos_sin_rows, x, y);
      uint16_t* qo = static_cast<uint16_t*>(p.q_out) + (t0 + i) * q_row + static_cast<int64_t>(qh) * hd;
      if (p.q_out_dtype == kBF16) {
        *reinterpret_cast<u32x4*>(qo + 8 * c0) = Store8<kBF16>::pack(x, 1.f);
        if (c1 >= 0) *reinterpret_cast<u32x4*>(qo + 8 * c1) = Store8<kBF16>::pack(y, 1.f);
      } else {
        *reinterpret_cast<u32x4*>(qo + 8 * c0) = Store8<kF16>::pack(x, 1.f);
        if (c1 >= 0) *reinterpret_cast<u32x4*>(qo + 8 * c1) = Store8<kF16>::pack(y, 1.f);
      }
    }
    return;
  }

  // K and V of kv head h = y (y < Hkv)
  const int h = blockIdx.y;
  const int64_t k_row = static_cast<int64_t>(p.num_kv_heads) * hd;  // source elements per token
  const int krow_bytes = hd * EB;                                    // one token's K or V row
  const int lrow = krow_bytes + kRowPad;                             // its LDS row stride
  uint8_t* k_lds = dyn_lds;
  uint8_t* v_lds = dyn_lds + WIN * lrow;
  // fp32 rows into 16-bit pools (the RoPE fill's usual case): lane j of a
  // token's hd/8 lanes takes the 16-byte pieces j and j + hd/8, i.e. dims
  // 4j..4j+3 of either half of the row, so each load instruction covers
  // whole lines and reads them non-temporally (8-value units read two 16-byte
  // halves 32 bytes apart per instruction: 1.26 x the read bytes), and a
  // NeoX rotation over the whole head pairs the lane's own two pieces
  constexpr bool kPieceSrc = SRC == kF32 && DST != kFP8;
  const bool piece_path = kPieceSrc && (style != 1 || p.rotary_dim == hd);
  f32x4 pk[kPieceSrc ? kItems : 1][2], pv[kPieceSrc ? kItems : 1][2];
  if constexpr (kPieceSrc) {
    if (piece_path) {
#pragma unroll
      for (int k = 0; k < kItems; ++k) {
        const int it = tid + k * kThreads;
        const int i = it / chunks;  // hd/8 lanes per token
        if (i < nwin) {
          const int64_t row = (t0 + i) * k_row + static_cast<int64_t>(h) * hd + 4 * (it % chunks);
#pragma unroll
          for (int sd = 0; sd < 2; ++sd) {
            pk[k][sd] = __builtin_nontemporal_load(
                reinterpret_cast<const f32x4*>(static_cast<const float*>(p.new_k) + row + sd * (hd / 2)));
            pv[k][sd] = __builtin_nontemporal_load(
                reinterpret_cast<const f32x4*>(static_cast<const float*>(p.new_v) + row + sd * (hd / 2)));
          }
        }
      }
    }
  }
  // ---- otherwise issue every source load of this thread: K units and V
  // chunks of the window's rows (units / chunks fastest, so a wavefront
  // reads whole lines of 16-bit rows)
  Raw8<SRC> kx[kItems], ky[kItems], vx[kItems];
#pragma unroll
  for (int k = 0; k < kItems && !piece_path; ++k) {
    const int it = tid + k * kThreads;
    const int i = it / units;
    if (i < nwin) {
      int c0, c1;
      unit_chunks(p, style, it % units, c0, c1);
      const int64_t row = (t0 + i) * k_row + static_cast<int64_t>(h) * hd;
      kx[k].load(p.new_k, row + 8 * c0);
      if (c1 >= 0) ky[k].load(p.new_k, row + 8 * c1);
    }
    const int iv = it / chunks;
    if (iv < nwin) vx[k].load(p.new_v, (t0 + iv) * k_row + static_cast<int64_t>(h) * hd + 8 * (it % chunks));
  }
  // ---- destinations (two dependent loads: the map, then the page table)
  if (tid < WIN) {
    uint32_t dpage = 0;
    int dslot = -1;
    int pos = 0;
    float ks = 1.f, vs = 1.f;
    if (tid < nwin) {
      const int64_t t = t0 + tid;
      const uint32_t seq = p.q2seq[t];
      pos = p.write_pos[t];
      if (seq < p.num_seqs && pos >= 0 && pos / tpp < p.page_table_width &&
          (style == 0 || pos < p.cos_sin_rows)) {
        const uint32_t page = p.page_table[static_cast<int64_t>(seq) * p.page_table_width + pos / tpp];
        if (page < p.num_pages) {
          dpage = page;
          dslot = pos % tpp;
          if constexpr (DST == kFP8) {
            ks = p.k_scales[static_cast<int64_t>(page) * p.num_kv_heads + h];
            vs = p.v_scales[static_cast<int64_t>(page) * p.num_kv_heads + h];
          }
        }
      }
    }
    PAL_DEBUG_FLAG(tid < nwin && dslot < 0, kDebugFillDest);
    page_lds[tid] = dpage;
    slot_lds[tid] = dslot;
    pos_lds[tid] = pos;
    ks_lds[tid] = ks;
    vs_lds[tid] = vs;
  }
  __syncthreads();
  if (tid < kWave) {
    // A full run: slots 8k..8k+7 of one page (pages of a multiple of 8
    // slots, so the run's pieces of K stripes and V rows are aligned)
    // written by 8 consecutive window tokens.  Token i lies in the run
    // starting at j = i - slot % 8, if any.
    auto is_lead = [&](int j) {
      if (j < 0 || j + 8 > nwin || (tpp % 8) != 0) return false;
      const int s0 = slot_lds[j];
      if (s0 < 0 || s0 % 8 != 0) return false;
      const uint32_t pg0 = page_lds[j];
      for (int e = 1; e < 8; ++e)
        if (slot_lds[j + e] != s0 + e || page_lds[j + e] != pg0) return false;
      return true;
    };
    int kind = 0;
    bool lead = false;
    if (tid < nwin && slot_lds[tid] >= 0) {
      lead = is_lead(tid);
      kind = (lead || is_lead(tid - slot_lds[tid] % 8)) ? 2 : 1;
    }
    if (tid < WIN) kind_lds[tid] = kind;
    const uint64_t leads = __ballot(lead);
    if (lead) run_lds[__popcll(leads & ((1ull << tid) - 1))] = tid;
    if (tid == 0) n_runs_lds = __popcll(leads);
  }
  __syncthreads();

  const int64_t head_block = static_cast<int64_t>(hd) * tpp * EB;  // bytes per (page, kv head) block
  // ---- single tokens to the pool, run tokens into LDS
  if constexpr (kPieceSrc) {
    if (piece_path) {
#pragma unroll
      for (int k = 0; k < kItems; ++k) {
        const int it = tid + k * kThreads;
        const int i = it / chunks;
        const int j = it % chunks;
        if (i >= nwin || slot_lds[i] < 0) continue;
        float x[2][4];
#pragma unroll
        for (int sd = 0; sd < 2; ++sd)
#pragma unroll
          for (int e = 0; e < 4; ++e) x[sd][e] = pk[k][sd][e];
        if (style != 0)
          rope_piece_pair(x[0], x[1], p.cos_sin + static_cast<int64_t>(pos_lds[i]) * p.rotary_dim, j, style,
                          p.rotary_dim, hd);
        const bool single = kind_lds[i] == 1;
        const int64_t hb = (static_cast<int64_t>(page_lds[i]) * p.num_kv_heads + h) * head_block;
#pragma unroll
        for (int sd = 0; sd < 2; ++sd) {
          const int d0 = sd * (hd / 2) + 4 * j;  // first dim of the piece
          const u32x2 kw = {Dt<DST>::pack2(x[sd][0], x[sd][1]), Dt<DST>::pack2(x[sd][2], x[sd][3])};
          const u32x2 vw = {Dt<DST>::pack2(pv[k][sd][0], pv[k][sd][1]), Dt<DST>::pack2(pv[k][sd][2], pv[k][sd][3])};
          if (single) {
            // K: half of stripe d0 / 8; V: one 2-byte value per row
            *reinterpret_cast<u32x2*>(static_cast<uint8_t*>(p.k_pool) + hb +
                                      (static_cast<int64_t>(d0 >> 3) * tpp + slot_lds[i]) * 16 + (d0 & 4) * 2) = kw;
            uint8_t* col = static_cast<uint8_t*>(p.v_pool) + hb + (static_cast<int64_t>(d0) * tpp + slot_lds[i]) * 2;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              *reinterpret_cast<uint16_t*>(col + e * tpp * 2) = static_cast<uint16_t>(vw[e >> 1] >> (16 * (e & 1)));
          } else {  // a run token: its rows into LDS as they are
            *reinterpret_cast<u32x2*>(k_lds + i * lrow + d0 * 2) = kw;
            *reinterpret_cast<u32x2*>(v_lds + i * lrow + d0 * 2) = vw;
          }
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kItems && !piece_path; ++k) {
    const int it = tid + k * kThreads;
    {  // K unit
      const int i = it / units;
      if (i < nwin && slot_lds[i] >= 0) {
        int c0, c1;
        unit_chunks(p, style, it % units, c0, c1);
        typename Store8<DST>::T a, b;
        bool copied = false;
        if constexpr (SRC == DST) {
          if (style == 0) {  // the reference's fill: a bit copy (NaN payloads included)
            a = kx[k].w;
            copied = true;
          }
        }
        if (!copied) {
          float x[8], y[8];
          kx[k].to_f32(x);
          if (c1 >= 0) ky[k].to_f32(y);
          rotate_unit(p, style, c0, c1, pos_lds[i], true, x, y);
          a = Store8<DST>::pack(x, ks_lds[i]);
          if (c1 >= 0) b = Store8<DST>::pack(y, ks_lds[i]);
        }
        if (kind_lds[i] == 1) {
          const int64_t hb = (static_cast<int64_t>(page_lds[i]) * p.num_kv_heads + h) * head_block;
          store_k_chunk<DST>(p, hb, slot_lds[i], c0, a);
          if (c1 >= 0) store_k_chunk<DST>(p, hb, slot_lds[i], c1, b);
        } else {
          *reinterpret_cast<typename Store8<DST>::T*>(k_lds + i * lrow + c0 * 8 * EB) = a;
          if (c1 >= 0) *reinterpret_cast<typename Store8<DST>::T*>(k_lds + i * lrow + c1 * 8 * EB) = b;
        }
      }
    }
    {  // V chunk
      const int i = it / chunks;
      const int c = it % chunks;
      if (i < nwin && slot_lds[i] >= 0) {
        // the chunk's 8 values as pool elements (16-bit, or fp8 bytes in the low byte)
        uint32_t e16[8];
        if constexpr (SRC == DST) {  // bit copy
#pragma unroll
          for (int e = 0; e < 8; ++e) e16[e] = (vx[k].w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        } else {
          float x[8];
          vx[k].to_f32(x);
          if constexpr (DST == kFP8) {
            const u32x2 q = Store8<kFP8>::pack(x, vs_lds[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) e16[e] = (q[e >> 2] >> (8 * (e & 3))) & 0xFFu;
          } else {
            const u32x4 q = Store8<DST>::pack(x, 1.f);
#pragma unroll
            for (int e = 0; e < 8; ++e) e16[e] = (q[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          }
        }
        if (kind_lds[i] == 1) {
          const int64_t hb = (static_cast<int64_t>(page_lds[i]) * p.num_kv_heads + h) * head_block;
          uint8_t* col = static_cast<uint8_t*>(p.v_pool) + hb + (static_cast<int64_t>(8 * c) * tpp + slot_lds[i]) * EB;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if constexpr (DST == kFP8) {
              col[e * tpp] = static_cast<uint8_t>(e16[e]);
            } else {
              *reinterpret_cast<uint16_t*>(col + e * tpp * 2) = static_cast<uint16_t>(e16[e]);
            }
          }
        } else {  // a run token: its chunk into LDS as it is
          if constexpr (DST == kFP8) {
            *reinterpret_cast<u32x2*>(v_lds + i * lrow + c * 8) =
                u32x2{e16[0] | (e16[1] << 8) | (e16[2] << 16) | (e16[3] << 24),
                      e16[4] | (e16[5] << 8) | (e16[6] << 16) | (e16[7] << 24)};
          } else {
            *reinterpret_cast<u32x4*>(v_lds + i * lrow + c * 16) =
                u32x4{e16[0] | (e16[1] << 16), e16[2] | (e16[3] << 16), e16[4] | (e16[5] << 16), e16[6] | (e16[7] << 16)};
          }
        }
      }
    }
  }
  __syncthreads();

  const int n_runs = n_runs_lds;
  if (n_runs == 0) return;
  // ---- K of the runs: item = (stripe q, run r, slot j), slots fastest: 8
  // lanes write the run's 128 contiguous bytes of stripe q (a stripe is 16
  // bytes: 8 dims of 16-bit, 16 of fp8), and runs r, r+1 (often the two
  // halves of one page) follow each other.
  const int pieces = krow_bytes / 16;  // 16-byte pieces of a token's K row
  for (int it = tid; it < pieces * n_runs * 8; it += kThreads) {
    const int j = it % 8;
    const int r = (it / 8) % n_runs;
    const int q = it / (8 * n_runs);
    const int i = run_lds[r] + j;
    const int64_t hb = (static_cast<int64_t>(page_lds[i]) * p.num_kv_heads + h) * head_block;
    // piece q is stripe q (16-bit: 8 dims, fp8: 16 dims) of the token
    *reinterpret_cast<u32x4*>(static_cast<uint8_t*>(p.k_pool) + hb + (static_cast<int64_t>(q) * tpp + slot_lds[i]) * 16) =
        *reinterpret_cast<const u32x4*>(k_lds + i * lrow + q * 16);
  }
  // ---- V of the runs: item = (row d, run r), runs fastest in pairs, so
  // lanes 2d, 2d+1 write row d of two runs (a page's two halves side by
  // side) and consecutive rows follow: whole lines per wavefront
  for (int it = tid; it < hd * n_runs; it += kThreads) {
    const int r = it % n_runs;
    const int d = it / n_runs;
    const int i = run_lds[r];
    const int64_t hb = (static_cast<int64_t>(page_lds[i]) * p.num_kv_heads + h) * head_block;
    uint8_t* row = static_cast<uint8_t*>(p.v_pool) + hb + (static_cast<int64_t>(d) * tpp + slot_lds[i]) * EB;
    // element d of the run's 8 tokens (rows i .. i+7 in LDS)
    const uint8_t* src = v_lds + i * lrow + d * EB;
    if constexpr (DST == kFP8) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo |= static_cast<uint32_t>(src[e * lrow]) << (8 * e);
        hi |= static_cast<uint32_t>(src[(4 + e) * lrow]) << (8 * e);
      }
      *reinterpret_cast<u32x2*>(row) = u32x2{lo, hi};
    } else {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(src + 2 * e * lrow)) |
               (static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(src + (2 * e + 1) * lrow)) << 16);
      *reinterpret_cast<u32x4*>(row) = w;
    }
  }
}

// Small batches (a decode step's new tokens): one thread per (token, kv
// head, 8-dim chunk) copies the chunk's K piece and its 8 V values straight
// into the pools -- no windows, runs through LDS or barriers; at these sizes
// coalescing V rows buys nothing and the kernel is its chain of dependent
// loads.  16-bit pools written from rows of the same dtype (a bit copy).
constexpr int kTokensThreads = 256;
constexpr int64_t kSmallFillTokens = 256;  // batches up to this many tokens take it
__global__ __launch_bounds__(kTokensThreads) void fill_tokens_kernel(const FillParams p) {
  const int chunks = p.head_dim / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kTokensThreads + threadIdx.x;
  if (i >= p.num_tokens * p.num_kv_heads * chunks) return;
  const int c = static_cast<int>(i % chunks);
  const int64_t th = i / chunks;
  const int h = static_cast<int>(th % p.num_kv_heads);
  const int64_t t = th / p.num_kv_heads;
  const int64_t row = (t * p.num_kv_heads + h) * p.head_dim + 8 * c;
  const u32x4 kw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.new_k) + row));
  const u32x4 vw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.new_v) + row));
  const uint32_t seq = p.q2seq[t];
  const int pos = p.write_pos[t];
  const int tpp = p.tokens_per_page;
  bool ok = seq < p.num_seqs && pos >= 0 && pos / tpp < p.page_table_width;
  uint32_t page = 0;
  if (ok) {
    page = p.page_table[static_cast<int64_t>(seq) * p.page_table_width + pos / tpp];
    ok = page < p.num_pages;
  }
  PAL_DEBUG_FLAG(!ok, kDebugFillDest);
  if (!ok) return;
  const int slot = pos % tpp;
  const int64_t blk = static_cast<int64_t>(page) * p.num_kv_heads + h;  // the (page, kv head) block
  *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.k_pool) + ((blk * chunks + c) * tpp + slot) * 8) = kw;
  uint16_t* vp = static_cast<uint16_t*>(p.v_pool) + (blk * p.head_dim + 8 * c) * tpp + slot;
#pragma unroll
  for (int e = 0; e < 8; ++e) vp[e * tpp] = static_cast<uint16_t>(vw[e >> 1] >> (16 * (e & 1)));
}

template <int SRC, int DST, int MAXC, bool ROPE>
hipError_t launch_win(const FillParams& p, hipStream_t stream) {
  if constexpr (!ROPE && SRC == DST && DST != kFP8) {
    if (p.num_tokens <= kSmallFillTokens) {
      const int64_t n = p.num_tokens * p.num_kv_heads * (p.head_dim / 8);
      hipLaunchKernelGGL(fill_tokens_kernel, dim3(static_cast<unsigned>((n + kTokensThreads - 1) / kTokensThreads)),
                         dim3(kTokensThreads), 0, stream, p);
      return hipGetLastError();
    }
  }
  // small batches (decode fills): windows of 16 tokens, so a 64-token fill
  // still spreads over 4 x 2 Hkv workgroups; prefill batches: 32
  const int win = p.num_tokens >= 2048 ? kLargeWin : kSmallWin;
  const int64_t windows = (p.num_tokens + win - 1) / win;
  const unsigned gy = p.num_kv_heads + (p.q_in ? p.num_q_heads : 0);
  const size_t lds = 2 * static_cast<size_t>(win) * (p.head_dim * elem_bytes<DST>() + kRowPad);  // K and V rows
  if (win == kLargeWin)
    hipLaunchKernelGGL((fill_kv_pages_kernel<SRC, DST, kLargeWin, MAXC, ROPE>), dim3(static_cast<unsigned>(windows), gy),
                       dim3(kThreads), lds, stream, p);
  else
    hipLaunchKernelGGL((fill_kv_pages_kernel<SRC, DST, kSmallWin, MAXC, ROPE>), dim3(static_cast<unsigned>(windows), gy),
                       dim3(kThreads), lds, stream, p);
  return hipGetLastError();
}

template <int SRC, int DST>
hipError_t launch_t(const FillParams& p, hipStream_t stream) {
  // per-thread item registers sized for the head dim: up to 128 or up to 256
  const bool rope = p.rope_style != 0 || p.q_in != nullptr;
  if (p.head_dim <= 128)
    return rope ? launch_win<SRC, DST, 16, true>(p, stream) : launch_win<SRC, DST, 16, false>(p, stream);
  return rope ? launch_win<SRC, DST, kMaxFillHeadDim / 8, true>(p, stream)
              : launch_win<SRC, DST, kMaxFillHeadDim / 8, false>(p, stream);
}

template <int SRC>
hipError_t launch_dst(const FillParams& p, hipStream_t stream) {
  switch (p.kv_dtype) {
    case kF16: return launch_t<SRC, kF16>(p, stream);
    case kBF16: return launch_t<SRC, kBF16>(p, stream);
    case kFP8: return launch_t<SRC, kFP8>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_fill_kv_pages(const FillParams& p, hipStream_t stream) {
  if (p.num_tokens <= 0) return hipSuccess;
  if (p.head_dim > kMaxFillHeadDim) return hipErrorInvalidValue;
  switch (p.src_dtype) {
    case kF16: return launch_dst<kF16>(p, stream);
    case kBF16: return launch_dst<kBF16>(p, stream);
    case kF32: return launch_dst<kF32>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pal
