// Work-list builder of the fused mixed-batch op, run on the device so the
// host never reads the row metadata.
//
// The fused op has no reference counterpart (the reference benchmark only
// builds query_to_seq_map / query_token_offset, batch_latency_vs_num_sequences.cpp:124-131).
// Rows are grouped into runs of consecutive rows naming the same sequence:
//  * a run of one row is a decode item (streamed by the decode kernel, which
//    splits long contexts over many wavefronts);
//  * a longer run is cut into prefill tiles of up to tokens_per_tile rows
//    (MFMA tiles that share each K/V step across the tile's rows).
// One workgroup of 1024 threads walks the rows in chunks with block scans.
#include "pal_device.h"
#include "pal_hip_internal.h"

namespace pal {

namespace {

constexpr int kPlanRowsPerChunk = 1024;

__global__ __launch_bounds__(kPlanRowsPerChunk) void fused_plan_kernel(const FusedPlanParams p) {
  __shared__ int64_t sums_a[kPlanRowsPerChunk / kWave];
  __shared__ int64_t sums_b[kPlanRowsPerChunk / kWave];
  __shared__ int64_t chunk_tot[3];
  const int tid = threadIdx.x;
  const int64_t n = p.num_rows;
  const int qt = p.tokens_per_tile;
  int64_t items = 0, tiles = 0, run_start = 0;
  for (int64_t base = 0; base < n; base += kPlanRowsPerChunk) {
    const int64_t r = base + tid;
    const bool valid = r < n;
    bool single = false, tile_start = false;
    int64_t start_here = -1;
    uint32_t sq = 0;
    if (valid) {
      sq = p.q2seq[r];
      const bool starts = r == 0 || p.q2seq[r - 1] != sq;
      const bool ends = r + 1 == n || p.q2seq[r + 1] != sq;
      single = starts && ends;
      start_here = starts ? r : -1;
    }
    // run start of row r: the last start at or before r (max-scan); runs
    // open in an earlier chunk carry in through run_start
    int64_t rs = start_here;
    {
      const int lane = lane_id();
      const int wv = tid >> 6;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int64_t o = __shfl_up(rs, off, kWave);
        if (lane >= off && o > rs) rs = o;
      }
      if (lane == kWave - 1) sums_a[wv] = rs;
      __syncthreads();
      for (int i = 0; i < wv; ++i) rs = sums_a[i] > rs ? sums_a[i] : rs;
      __syncthreads();
      if (rs < 0) rs = run_start;
    }
    if (valid && !single) tile_start = ((r - rs) % qt) == 0;
    const int64_t di = block_inclusive_scan<kPlanRowsPerChunk>(single ? 1 : 0, sums_a);
    const int64_t ti = block_inclusive_scan<kPlanRowsPerChunk>(tile_start ? 1 : 0, sums_b);
    if (single) p.item_rows[items + di - 1] = static_cast<int32_t>(r);
    if (tile_start) {
      int cnt = 1;
      while (cnt < qt && r + cnt < n && p.q2seq[r + cnt] == sq) ++cnt;
      int32_t* t = p.tiles + 3 * (tiles + ti - 1);
      t[0] = static_cast<int32_t>(r);
      t[1] = cnt;
      t[2] = static_cast<int32_t>(sq);
    }
    if (tid == kPlanRowsPerChunk - 1) {
      chunk_tot[0] = di;
      chunk_tot[1] = ti;
      chunk_tot[2] = rs;
    }
    __syncthreads();
    items += chunk_tot[0];
    tiles += chunk_tot[1];
    run_start = chunk_tot[2];
    __syncthreads();
  }
  if (tid == 0) {
    p.counts[0] = static_cast<int32_t>(items);
    p.counts[1] = static_cast<int32_t>(tiles);
  }
}

}  // namespace

hipError_t launch_fused_plan(const FusedPlanParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(fused_plan_kernel, dim3(1), dim3(kPlanRowsPerChunk), 0, stream, p);
  return hipGetLastError();
}

}  // namespace pal
