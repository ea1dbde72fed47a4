// Device-side helpers shared by the gfx950 kernels: 16-bit float traits,
// MFMA wrappers and wave64 reductions.
//
// Raw fp16/bf16 data is carried as 16-bit patterns inside 32-bit vector
// registers (u32x2 / u32x4) and bit-cast to the operand types the MFMA
// builtins want, so one kernel body serves both dtypes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pal_hip_internal.h"

namespace pal {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Debug checks (builds with -DPAL_DEBUG_CHECKS only): a kernel that meets an
// input it tolerates but that the caller most likely did not mean (a page id
// past the pool, a length past the page table, a fill destination out of
// range) sets a bit in its translation unit's flag word instead of silently
// reading zeros or skipping; pal_debug_flags() reads and clears the words.
// Nothing traps.  Release builds compile the checks away.
// ---------------------------------------------------------------------------
constexpr uint32_t kDebugPageId = 1u;     // a page id >= num_pages where a token was to be read
constexpr uint32_t kDebugLength = 2u;     // a length or position past page_table_width * TPP
constexpr uint32_t kDebugFillDest = 4u;   // a fill token with no valid destination (skipped)

#ifdef PAL_DEBUG_CHECKS
#define PAL_DEBUG_FLAGS_DEFINE(fn)                                                       \
  namespace {                                                                            \
  __device__ uint32_t g_debug_flags;                                                     \
  }                                                                                      \
  hipError_t fn(uint32_t* out, bool reset) {                                             \
    hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(g_debug_flags), sizeof(uint32_t)); \
    if (e != hipSuccess || !reset) return e;                                             \
    const uint32_t zero = 0;                                                             \
    return hipMemcpyToSymbol(HIP_SYMBOL(g_debug_flags), &zero, sizeof(uint32_t));        \
  }
#define PAL_DEBUG_FLAG(cond, bit)                      \
  do {                                                 \
    if (cond) atomicOr(&g_debug_flags, (bit));         \
  } while (0)
#else
#define PAL_DEBUG_FLAGS_DEFINE(fn)             \
  hipError_t fn(uint32_t* out, bool) {         \
    *out = 0;                                  \
    return hipSuccess;                         \
  }
#define PAL_DEBUG_FLAG(cond, bit) \
  do {                            \
  } while (0)
#endif

// ---------------------------------------------------------------------------
// dtype traits: scalar conversion, packing and the MFMA shapes used here.
//   mma16x16x32: A[16 x 32] * B[32 x 16] (8 elements per lane per operand)
//   mma16x16x16: A[16 x 16] * B[16 x 16] (4 elements per lane per operand)
//   mma32x32x16: A[32 x 16] * B[16 x 32] (8 elements per lane per operand)
// ---------------------------------------------------------------------------
template <int DT>
struct Dt;

template <>
struct Dt<kBF16> {
  static __device__ __forceinline__ float to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
  }
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  // one v_cvt_pk_bf16_f32 (round to nearest even)
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
  }
  static __device__ __forceinline__ f32x4 mma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // acc + lo + hi of a packed pair (one v_dot2c_f32_bf16 against (1, 1))
  static __device__ __forceinline__ float sum2(uint32_t packed, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, packed), __builtin_bit_cast(bf16x2, 0x3F803F80u),
                                           acc, false);
  }
  // two fp8 e4m3 values (bytes 0-1, or 2-3 when hi) of w as a packed pair;
  // exact (every e4m3 value is a bf16 value): one v_cvt_scalef32_pk_bf16_fp8
  // with scale 1
  static __device__ __forceinline__ uint32_t fp8x2(uint32_t w, bool hi) {
    const bf16x2 v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, true)
                        : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, false);
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <>
struct Dt<kF16> {
  static __device__ __forceinline__ float to_f32(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
  }
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  // one v_cvt_pk_f16_f32 (round to nearest even)
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), f16x2));
  }
  static __device__ __forceinline__ f32x4 mma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // acc + lo + hi of a packed pair (one v_dot2c_f32_f16 against (1, 1))
  static __device__ __forceinline__ float sum2(uint32_t packed, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, packed), __builtin_bit_cast(f16x2, 0x3C003C00u), acc, false);
  }
  // two fp8 e4m3 values as a packed pair; exact (e4m3's range and 3-bit
  // mantissa fit fp16, subnormals included): one v_cvt_scalef32_pk_f16_fp8
  // with scale 1
  static __device__ __forceinline__ uint32_t fp8x2(uint32_t w, bool hi) {
    const f16x2 v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, true)
                       : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, false);
    return __builtin_bit_cast(uint32_t, v);
  }
};

// Eight fp8 e4m3 values (w: bytes 0..7) as packed 16-bit values of dtype DT,
// exactly (every finite e4m3 value, subnormals included, is a bf16 and an
// fp16 value).
template <int DT>
__device__ __forceinline__ u32x4 fp8x8_exact(u32x2 w) {
  return u32x4{Dt<DT>::fp8x2(w.x, false), Dt<DT>::fp8x2(w.x, true), Dt<DT>::fp8x2(w.y, false),
               Dt<DT>::fp8x2(w.y, true)};
}

// ---------------------------------------------------------------------------
// fp8 e4m3 operands of the gfx950 scaled MFMA: D[16 x 16] += A[16 x 128]
// B[128 x 16] with 32 codes per lane per operand.  Lane 16 g + i holds 32
// k-slots of row i of A and the same 32 k-slots of column i of B (the two
// operands distribute k alike, checked on the GPU against a host product),
// so any assignment of dims to (lane group, byte) that A and B share gives
// the inner product.  Output: lane l holds D[4 (l / 16) + e][l % 16], e < 4,
// as in mma16x16x32.  sb is the E8M0 scale of B's column l % 16 (2^(sb -
// 127)); A is unscaled.
// ---------------------------------------------------------------------------
typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mma_fp8_16x16x128(i32x8 a, i32x8 b, f32x4 c, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, sb);
}

// A query head as fp8 terms for mma_fp8_16x16x128.  With x = q 2^sh (sh per
// head: the head's largest |q| scales into [128, 256)), the terms are hi =
// e4m3(x), lo = e4m3(16 (x - hi)) and, for fp16 queries, lo2 = e4m3(16 (16
// (x - hi) - lo)), each rounded to nearest even; term t carries the scale
// 2^-(sh + 4 t).  Two terms are exact for bf16 (8 significant bits: hi keeps
// 4, the remainder is k 2^(e - 7) with |k| <= 8) and three leave fp16 within
// 2^-12 of each value, for every element above 2^-13 of the head's largest
// (smaller ones are within 2^-21 of the largest).
//
// q4[kk]: the lane's 8 query values of k-step kk (16-bit, packed in pairs);
// operand m takes the values of k-steps 4m .. 4m+3 as its bytes 0..31 (zeros
// past KK).  The largest magnitude is taken over the 4 lane groups of the head.
template <int DT, int KK>
struct QueryFp8 {
  static constexpr int kOps = (KK + 3) / 4;      // MFMAs per 128 dims
  static constexpr int kTerms = DT == kBF16 ? 2 : 3;
  i32x8 w[kTerms][kOps];
  int s_hi;  // E8M0 scale of term 0; term t uses s_hi - 4 t
};

template <int DT, int KK>
__device__ __forceinline__ void query_to_fp8(const u32x4 (&q4)[KK], QueryFp8<DT, KK>& out) {
  constexpr int kOps = QueryFp8<DT, KK>::kOps;
  constexpr int kTerms = QueryFp8<DT, KK>::kTerms;
  // largest magnitude: for bf16 and fp16 alike the magnitude order of
  // non-NaN values is the integer order of their low 15 bits
  uint32_t mb = 0;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t w = q4[kk][c];
      mb = max(mb, max(w & 0x7FFFu, (w >> 16) & 0x7FFFu));
    }
  }
  mb = max(mb, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mb), 16, 64)));
  mb = max(mb, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mb), 32, 64)));
  // floor(log2 of the largest); zero and subnormal heads take the clamp
  const int e = DT == kBF16 ? static_cast<int>(mb >> 7) - 127 : static_cast<int>(mb >> 10) - 15;
  int sh = 7 - e;
  // E8M0 scales 127 - sh - 4 t stay in [0, 254] and 2^sh is a normal float;
  // -126 covers every finite bf16 and fp16 head (their largest exponent is
  // 127), 119 only heads below 2^-112, whose scores vanish anyway
  sh = sh < -126 ? -126 : (sh > 119 ? 119 : sh);
  const float mul = __uint_as_float(static_cast<uint32_t>(sh + 127) << 23);
  out.s_hi = 127 - sh;
#pragma unroll
  for (int m = 0; m < kOps; ++m) {
#pragma unroll
    for (int wd = 0; wd < 8; ++wd) {  // word wd: values 4 wd .. 4 wd + 3 of operand m
      const int kk = 4 * m + wd / 2;
      float x[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (kk < KK) {
          const uint32_t w = q4[kk][2 * (wd & 1) + t / 2];
          x[t] = Dt<DT>::to_f32(static_cast<uint16_t>((t & 1) ? (w >> 16) : (w & 0xFFFFu))) * mul;
        } else {
          x[t] = 0.f;
        }
      }
#pragma unroll
      for (int term = 0; term < kTerms; ++term) {
        int code = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
        code = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], code, true);
        out.w[term][m][wd] = code;
        if (term + 1 < kTerms) {
          const f32x2 b01 = __builtin_amdgcn_cvt_pk_f32_fp8(code, false);
          const f32x2 b23 = __builtin_amdgcn_cvt_pk_f32_fp8(code, true);
          x[0] = (x[0] - b01[0]) * 16.f;  // exact: the remainder of a rounding
          x[1] = (x[1] - b01[1]) * 16.f;
          x[2] = (x[2] - b23[0]) * 16.f;
          x[3] = (x[3] - b23[1]) * 16.f;
        }
      }
    }
  }
}

// Eight fp8 e4m3 values (w: bytes 0..7) times scale s, as packed 16-bit
// values of dtype DT (round to nearest even).
template <int DT>
__device__ __forceinline__ u32x4 fp8x8_scaled(u32x2 w, float s) {
  u32x4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t word = q < 2 ? w.x : w.y;
    const f32x2 f = (q & 1) ? __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(word), true)
                            : __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(word), false);
    r[q] = Dt<DT>::pack2(f[0] * s, f[1] * s);
  }
  return r;
}

// s_waitcnt immediates (gfx9 encoding): vmcnt <= n only, and lgkmcnt(0) only.
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kLgkmZero = 15 | (3 << 14) | (7 << 4);

// Direct-to-LDS copy (global_load_lds_dwordx4): lane l copies the 16 bytes
// at base + off to LDS byte address lds + 16 l; base and lds wave-uniform.
// Issued as inline assembly so that the compiler does not track an LDS write
// in flight: it would otherwise wait for every such copy (vmcnt(0)) before
// later LDS reads it cannot prove disjoint.  Callers wait with counted
// s_waitcnt.  The compiler's hazard pass does not look inside the asm, so
// the asm carries the wait states itself: s_nop 4 gives the five that a
// vector memory instruction needs after a VALU write of an SGPR it reads (the
// compiler may materialise the base with v_readlane / v_readfirstlane right
// before the asm), which also covers the one after the M0 write.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));  // low half of a generic LDS address
}
__device__ __forceinline__ void copy_to_lds16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// Transposing LDS read (ds_read_b64_tr_b16).  In each group of 16 lanes,
// lane 4r + c points at 4 consecutive 16-bit elements, columns 4c .. 4c+3 of
// row r of a 4 x 16 block; lane j receives column j, rows 0..3 (element i in
// bits 16i .. 16i+15).  The address must be 8-byte aligned.
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4* lds_s16x4;
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(p));
  return __builtin_bit_cast(u32x2, r);
}

// Scheduling fence: the compiler's instruction scheduler moves nothing
// across this point (data dependences are unaffected; waits are inserted
// as usual).
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }
// Keeps the compiler from moving memory accesses across this point (the
// direct-to-LDS copies and counted waits are invisible to its dependence
// tracking).
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// ---------------------------------------------------------------------------
// wave64 helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// max / sum of v and its value in lane l ^ 32 (v_permlane32_swap: no LDS trip).
// The max is one plain v_max_f32: the scores it compares are finite or
// -inf, so the NaN quieting fmaxf would add is not needed.
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(__uint_as_float(r[0])), "v"(__uint_as_float(r[1])));
  return m;
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The same with lane l ^ 16 (v_permlane16_swap: the two results hold v of
// lanes l and l ^ 16).
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(__uint_as_float(r[0])), "v"(__uint_as_float(r[1])));
  return m;
}
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 4 x 4 transpose of 32-bit words across the four 16-lane groups: lane
// 16 g + i holds words 0..3 of "row" g (of its column i) and receives word g
// of rows 0..3.  v_permlane32_swap exchanges the upper 32 lanes of its first
// operand with the lower 32 of its second, v_permlane16_swap the odd 16-lane
// rows of its first operand with the even rows of its second (each returns
// both operands).  After the two 32-lane swaps groups 0, 1 hold words 0, 1
// of rows g (x02[0], x13[0]) and g + 2 (x02[1], x13[1]), groups 2, 3 words
// 2, 3 of rows g - 2 and g; the 16-lane swaps then leave word g of rows 0, 1
// in y and of rows 2, 3 in z.
__device__ __forceinline__ u32x4 transpose_lane_groups4(u32x4 w) {
  const auto x02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
  const auto x13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  const auto y = __builtin_amdgcn_permlane16_swap(x02[0], x13[0], false, false);
  const auto z = __builtin_amdgcn_permlane16_swap(x02[1], x13[1], false, false);
  return u32x4{y[0], y[1], z[0], z[1]};
}

// Index of this thread's wavefront, forced into a scalar register so that
// addresses derived from it stay uniform (scalar loads of page-table entries).
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// Zero the 16-bit elements i (0..3) of a packed 4-element vector whose
// keep-bit is clear.
__device__ __forceinline__ u32x2 mask4(u32x2 v, bool k0, bool k1, bool k2, bool k3) {
  u32x2 r;
  r.x = (k0 ? 0x0000FFFFu : 0u) | (k1 ? 0xFFFF0000u : 0u);
  r.y = (k2 ? 0x0000FFFFu : 0u) | (k3 ? 0xFFFF0000u : 0u);
  r.x &= v.x;
  r.y &= v.y;
  return r;
}

// Block-wide inclusive scan of int64 values over kThreads threads.
template <int kThreads>
__device__ int64_t block_inclusive_scan(int64_t v, int64_t* wave_sums) {
  const int lane = lane_id();
  const int wv = static_cast<int>(threadIdx.x) >> 6;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int64_t o = __shfl_up(v, off, kWave);
    if (lane >= off) v += o;
  }
  if (lane == kWave - 1) wave_sums[wv] = v;
  __syncthreads();
  int64_t add = 0;
  for (int i = 0; i < wv; ++i) add += wave_sums[i];
  __syncthreads();
  return v + add;
}

}  // namespace pal
