// Tile plan of the persistent gathers: every workgroup reads the row
// metadata written by the norm kernel, counts each gathered row's tiles and
// scans the counts in LDS.  All workgroups compute the same prefix, so none
// waits on another, and each then walks a contiguous range of the W tiles.
#pragma once

#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {

template <int kThreads, uint32_t kRows = kPlanRowsMax>
struct TilePlan {
  uint32_t prefix[kRows + 1];  // prefix[r] = first tile of row r
  uint32_t begin[kRows];       // list start in the state lists
  uint32_t count[kRows];       // gathered candidates (0 = not gathered)
  uint32_t kind[kRows];
  uint32_t wave_total[kThreads / kWave];
};

__device__ __forceinline__ bool row_gathered(const RowMeta& m, bool lookup) {
  return ((m.kind & kRowRestricted) && !(m.kind & kRowDense)) ||
         (lookup && (m.kind & kRowUnrestricted));
}

// Fills the plan (all threads call; ends with a barrier) and returns W.
// meta_of(r) gives row r's metadata.
template <int kThreads, uint32_t kRows, typename MetaOf>
__device__ uint32_t plan_tiles_by(MetaOf meta_of, uint32_t rows, uint32_t tile, bool lookup,
                                  TilePlan<kThreads, kRows>& p) {
  const uint32_t tid = threadIdx.x;
  for (uint32_t r = tid; r < rows; r += kThreads) {
    const RowMeta m = meta_of(r);
    const bool use = row_gathered(m, lookup);
    p.begin[r] = m.list_begin;
    p.count[r] = use ? m.count : 0u;
    p.kind[r] = m.kind;
    p.prefix[r + 1] = use ? (m.count + tile - 1) / tile : 0u;
  }
  __syncthreads();
  // in-place inclusive scan of prefix[1..rows]: thread segments + block scan
  const uint32_t seg = (rows + kThreads - 1) / kThreads;
  const uint32_t s0 = tid * seg < rows ? tid * seg : rows;
  const uint32_t s1 = s0 + seg < rows ? s0 + seg : rows;
  uint32_t local = 0u;
  for (uint32_t i = s0; i < s1; ++i) local += p.prefix[i + 1];
  uint32_t incl = local;
  const uint32_t lane = tid % kWave;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d);
    if (static_cast<int>(lane) >= d) incl += o;
  }
  if (lane == kWave - 1) p.wave_total[tid / kWave] = incl;
  __syncthreads();
  uint32_t run = incl - local;
  for (uint32_t w = 0; w < tid / kWave; ++w) run += p.wave_total[w];
  for (uint32_t i = s0; i < s1; ++i) {
    run += p.prefix[i + 1];
    p.prefix[i + 1] = run;
  }
  if (tid == 0) p.prefix[0] = 0u;
  __syncthreads();
  return p.prefix[rows];
}

// The plan from the metadata the norm kernel wrote.
template <int kThreads>
__device__ uint32_t plan_tiles(const RowMeta* row_meta, uint32_t rows, uint32_t tile,
                               bool lookup, TilePlan<kThreads>& p) {
  return plan_tiles_by<kThreads, kPlanRowsMax>([row_meta](uint32_t r) { return row_meta[r]; },
                                               rows, tile, lookup, p);
}

// The row holding tile w: largest r with prefix[r] <= w < prefix[r + 1].
template <int kThreads, uint32_t kRows>
__device__ uint32_t plan_row_of(const TilePlan<kThreads, kRows>& p, uint32_t rows, uint32_t w) {
  uint32_t lo = 0u, hi = rows;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) / 2;
    if (p.prefix[mid + 1] <= w) lo = mid + 1; else hi = mid;
  }
  return lo;
}

}  // namespace mf
