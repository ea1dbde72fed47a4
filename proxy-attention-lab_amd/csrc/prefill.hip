// Paged causal attention for query tiles on gfx950 MFMA: the prefill kernel
// (the reference's uniform-prompt signature) and the prefill half of the
// fused mixed batch.  The tile code and its design notes are in
// prefill_tile.h.
//
// Reference behaviour: kernels/paged_attention/prefill/paged_attention_prefill.h.metal
// (history + causal prompt keys :147-234, :251-360; scores scaled after the
// dot product :178, :302; output rows (token, head) :379-381).
#include "pal_device.h"

namespace pal {

// flag word of this translation unit's debug checks (see pal_device.h)
PAL_DEBUG_FLAGS_DEFINE(prefill_debug_flags)

}  // namespace pal

#include "prefill_tile.h"

namespace pal {

namespace {

// One workgroup of tiles per block (the work mapping is in prefill_block).
// Head dims up to 128 are held to half of the register file (two wavefronts
// per SIMD); head dim 256 needs more than that and runs one per SIMD.
template <int DT, int HD, int TPP, bool KV8>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_tile_kernel(const PrefillParams p) {
  __shared__ PrefillLds<HD, KV8> lds;
  prefill_block<DT, HD, TPP, KV8>(p, blockIdx.x, lds);
}
template <int DT, int HD, int TPP, bool KV8>
__global__ __launch_bounds__(kPfThreads) void prefill_tile_kernel_wide(const PrefillParams p) {
  __shared__ PrefillLds<HD, KV8> lds;
  prefill_block<DT, HD, TPP, KV8>(p, blockIdx.x, lds);
}

template <int DT, int HD, int TPP, bool KV8>
hipError_t launch_prefill_t(const PrefillParams& p, hipStream_t stream) {
  const int64_t blocks = static_cast<int64_t>(p.num_units) * p.num_kv_heads * p.head_chunks;
  if constexpr (HD <= 128)
    hipLaunchKernelGGL((prefill_tile_kernel<DT, HD, TPP, KV8>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kPfThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_tile_kernel_wide<DT, HD, TPP, KV8>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kPfThreads), 0, stream, p);
  return hipGetLastError();
}

// Page sizes 16 and 32 have their own kernels; other multiples of 8 (16-bit
// pools, uniform-prompt mode) run the kernel built for a run-time page size.
template <int DT, int HD, bool KV8>
hipError_t prefill_tpp(const PrefillParams& p, int tpp, hipStream_t stream) {
  switch (tpp) {
    case 16: return launch_prefill_t<DT, HD, 16, KV8>(p, stream);
    case 32: return launch_prefill_t<DT, HD, 32, KV8>(p, stream);
    default:
      if constexpr (!KV8) {
        if (tpp > 0 && tpp % 8 == 0 && p.prompt_len > 0) return launch_prefill_t<DT, HD, 0, false>(p, stream);
      }
      return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t prefill_hd(const PrefillParams& p, int hd, int tpp, hipStream_t stream) {
  if (p.k_scales) {  // fp8 pools: head dims of whole 16-dim stripes
    switch (hd) {
      case 64: return prefill_tpp<DT, 64, true>(p, tpp, stream);
      case 128: return prefill_tpp<DT, 128, true>(p, tpp, stream);
      case 256: return prefill_tpp<DT, 256, true>(p, tpp, stream);
      default: return hipErrorInvalidValue;
    }
  }
  switch (hd) {
    case 32: return prefill_tpp<DT, 32, false>(p, tpp, stream);
    case 64: return prefill_tpp<DT, 64, false>(p, tpp, stream);
    case 96: return prefill_tpp<DT, 96, false>(p, tpp, stream);
    case 128: return prefill_tpp<DT, 128, false>(p, tpp, stream);
    case 256: return prefill_tpp<DT, 256, false>(p, tpp, stream);
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
