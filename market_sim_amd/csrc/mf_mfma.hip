// gfx950 MFMA kernels: the head of the unrestricted rows
// (vocab_head_*_kernel): every token's score against the rows' FP16 hi/lo
// split, reduced in a windowed-argmax epilogue to tile records (no logits
// written).  The FP16 hi + lo pair of an FP32 value (two MFMAs per step)
// makes the fast score accurate to ~2^-22 relative before the
// reference-order rescore.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"
#include "mf_head.hpp"

namespace mf {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kMTile = 32;

// Reductions over the 8 consecutive lanes that share one row.
__device__ __forceinline__ float group8_max(float v) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, m, 8));
  return v;
}
__device__ __forceinline__ uint32_t group8_and(uint32_t v) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) v &= __shfl_xor(v, m, 8);
  return v;
}

// Narrow rows: H = 32 kSteps, the panel tile in LDS, the whole K range of
// the wave's kBlocks token blocks in registers.
template <int kWaves, int kBlocks, int kSteps>
__global__ __launch_bounds__(kWaves * 64) void vocab_head_lds_kernel(FallbackArgs f) {
  static_assert(kWaves * kBlocks == static_cast<int>(kHeadTileBlocks), "tile of 12 blocks");
  constexpr uint32_t H = 32u * kSteps;
  constexpr uint32_t kRowHalves = H + kPanelPad;
  constexpr uint32_t kTileHalves = static_cast<uint32_t>(panel_tile_bytes(H) / 2u);
  constexpr uint32_t kBursts = static_cast<uint32_t>(panel_tile_bytes(H) / 1024u);
  static_assert(panel_tile_bytes(H) % 1024u == 0, "whole bursts");
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t src_row[kMTile];
  __shared__ float src_norm[kMTile];
  __shared__ float src_slack[kMTile];
  HeadEpi& epi = *reinterpret_cast<HeadEpi*>(dyn);
  uint16_t* stage = reinterpret_cast<uint16_t*>(dyn + sizeof(HeadEpi));
  const uint32_t m0 = blockIdx.y * kMTile;
  const uint32_t tiles = (f.V + kHeadTileTokens - 1) / kHeadTileTokens;
  const uint32_t t_begin = blockIdx.x * f.tiles_per_group;
  const uint32_t t_end = t_begin + f.tiles_per_group < tiles ? t_begin + f.tiles_per_group : tiles;
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t wave = threadIdx.x / 64;
  const uint32_t col = lane % 16;
  const uint32_t kb = lane / 16;
  // the panel tile into LDS: wave w takes bursts w, w + kWaves, ...
  const uint16_t* panel = f.panel + static_cast<uint64_t>(blockIdx.y) * kTileHalves;
  for (uint32_t c = wave; c < kBursts; c += kWaves) {
    burst_to_lds(panel + c * 512u + lane * 8u, stage + c * 512u);
  }
  half8_t bt[kBlocks][kSteps];
  auto load_tile = [&](uint32_t t) {
#pragma unroll
    for (int tb = 0; tb < kBlocks; ++tb) {
      const uint32_t token = t * kHeadTileTokens + (wave * kBlocks + tb) * 16u + col;
      const uint16_t* p = f.emb + static_cast<uint64_t>(token < f.V ? token : 0u) * H + kb * 8u;
#pragma unroll
      for (int s = 0; s < kSteps; ++s) bt[tb][s] = *reinterpret_cast<const half8_t*>(p + s * 32);
    }
  };
  load_tile(t_begin);
  head_slots(f, m0, src_row, src_norm, src_slack);
  wait_vector_memory();
  __syncthreads();
  const uint16_t* a_lane = stage + col * kRowHalves + kb * 8u;
  constexpr uint32_t kRbStride = 16u * kRowHalves;
  for (uint32_t tile = t_begin; tile < t_end; ++tile) {
    if (tile != t_begin) load_tile(tile);
    HeadAcc<kBlocks> h;
#pragma unroll
    for (int tb = 0; tb < kBlocks; ++tb) {
      h.gram[tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) h.acc[rb][tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // A fragments one step ahead: the LDS reads of step s + 1 are in flight
    // during the MFMAs of step s
    half8_t a_cur[4];
    half8_t a_nxt[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      a_cur[rb] = *reinterpret_cast<const half8_t*>(a_lane + rb * kRbStride);
    }
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      if (s + 1 < kSteps) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          a_nxt[rb] = *reinterpret_cast<const half8_t*>(a_lane + rb * kRbStride + (s + 1) * 32);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tb = 0; tb < kBlocks; ++tb) {
        h.gram[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bt[tb][s], bt[tb][s], h.gram[tb], 0, 0, 0);
      }
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
        for (int tb = 0; tb < kBlocks; ++tb) {
          h.acc[rb][tb] =
              __builtin_amdgcn_mfma_f32_16x16x32_f16(a_cur[rb], bt[tb][s], h.acc[rb][tb], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) a_cur[rb] = a_nxt[rb];
    }
    head_records<kWaves, kBlocks>(f, h, epi, src_row, src_norm, src_slack, m0, tile, tiles);
  }
}

// Wide rows: units of KC steps of table rows and A (from the panel in L2),
// two units in flight; the steady-state loop has no branch around a load,
// and sched_barrier(0) keeps each unit's loads issued before the previous
// unit's MFMAs (the scheduler would otherwise sink them past the MFMAs and
// every unit would wait a full round trip).

template <int KC>
struct ABUnit {
  half8_t b[kWideBlocks][KC];
  half8_t a[4][KC];
};

template <int KC>
__device__ __forceinline__ void unit_load(const uint16_t* const (&bptr)[kWideBlocks],
                                          const uint16_t* const (&aptr)[4], uint32_t f0,
                                          ABUnit<KC>& u) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
#pragma unroll
    for (int tb = 0; tb < kWideBlocks; ++tb) {
      u.b[tb][s] = *reinterpret_cast<const half8_t*>(bptr[tb] + f0 + s * 32);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      u.a[rb][s] = *reinterpret_cast<const half8_t*>(aptr[rb] + f0 + s * 32);
    }
  }
}

__device__ __forceinline__ half8_t masked(const half8_t& v, uint32_t mask) {
  uint4 q = __builtin_bit_cast(uint4, v);
  q.x &= mask;
  q.y &= mask;
  q.z &= mask;
  q.w &= mask;
  return __builtin_bit_cast(half8_t, q);
}

// slots without a row are masked to zero (their panel rows are not written)
template <int KC>
__device__ __forceinline__ void unit_mma(const ABUnit<KC>& u, const uint32_t (&amask)[4],
                                         HeadAcc<kWideBlocks>& h) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
#pragma unroll
    for (int tb = 0; tb < kWideBlocks; ++tb) {
      h.gram[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(u.b[tb][s], u.b[tb][s], h.gram[tb], 0, 0, 0);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const half8_t a = masked(u.a[rb][s], amask[rb]);
#pragma unroll
      for (int tb = 0; tb < kWideBlocks; ++tb) {
        h.acc[rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, u.b[tb][s], h.acc[rb][tb], 0, 0, 0);
      }
    }
  }
}

template <int KC>
__global__ __launch_bounds__(kWideWaves * 64) void vocab_head_wide_kernel(FallbackArgs f) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t src_row[kMTile];
  __shared__ float src_norm[kMTile];
  __shared__ float src_slack[kMTile];
  HeadEpi& epi = *reinterpret_cast<HeadEpi*>(dyn);
  const uint32_t m0 = blockIdx.y * kMTile;
  const uint32_t tiles = (f.V + kHeadTileTokens - 1) / kHeadTileTokens;
  const uint32_t t_begin = blockIdx.x * f.tiles_per_group;
  const uint32_t t_end = t_begin + f.tiles_per_group < tiles ? t_begin + f.tiles_per_group : tiles;
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t wave = threadIdx.x / 64;
  const uint32_t H = f.H;
  const uint32_t col = lane % 16;
  const uint32_t kb = lane / 16;
  const uint32_t row_halves = H + kPanelPad;
  const uint16_t* panel = f.panel + static_cast<uint64_t>(blockIdx.y) * (panel_tile_bytes(H) / 2u);
  const uint32_t units = H / (32 * KC);
  constexpr uint32_t kUnitF = 32 * KC;
  head_slots(f, m0, src_row, src_norm, src_slack);
  __syncthreads();
  const uint16_t* aptr[4];
  uint32_t amask[4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    aptr[rb] = panel + (16u * rb + col) * row_halves + kb * 8u;
    amask[rb] = src_row[rb * 8 + col / 2] != kInvalidToken ? 0xFFFFFFFFu : 0u;
  }
  const uint16_t* bptr[kWideBlocks];
  for (uint32_t tile = t_begin; tile < t_end; ++tile) {
#pragma unroll
    for (int tb = 0; tb < kWideBlocks; ++tb) {
      const uint32_t token = tile * kHeadTileTokens + (wave * kWideBlocks + tb) * 16u + col;
      bptr[tb] = f.emb + static_cast<uint64_t>(token < f.V ? token : 0u) * H + kb * 8u;
    }
    HeadAcc<kWideBlocks> h;
#pragma unroll
    for (int tb = 0; tb < kWideBlocks; ++tb) {
      h.gram[tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) h.acc[rb][tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    ABUnit<KC> u0, u1;
    unit_load<KC>(bptr, aptr, 0, u0);
    uint32_t q = 0;
    for (; q + 2 < units; q += 2) {
      unit_load<KC>(bptr, aptr, (q + 1) * kUnitF, u1);
      __builtin_amdgcn_sched_barrier(0);
      unit_mma<KC>(u0, amask, h);
      __builtin_amdgcn_sched_barrier(0);
      unit_load<KC>(bptr, aptr, (q + 2) * kUnitF, u0);
      __builtin_amdgcn_sched_barrier(0);
      unit_mma<KC>(u1, amask, h);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (q + 1 < units) {
      unit_load<KC>(bptr, aptr, (q + 1) * kUnitF, u1);
      __builtin_amdgcn_sched_barrier(0);
      unit_mma<KC>(u0, amask, h);
      unit_mma<KC>(u1, amask, h);
    } else {
      unit_mma<KC>(u0, amask, h);
    }
    head_records<kWideWaves, kWideBlocks>(f, h, epi, src_row, src_norm, src_slack, m0, tile,
                                          tiles);
  }
}

} // namespace

uint32_t fallback_tiles(uint32_t vocab) {
  return (vocab + kHeadTileTokens - 1) / kHeadTileTokens;
}

// Narrow-row variant per H = 32 kSteps (H % 64 == 0, panel tile <= 76 KiB).
template <int kSteps>
static void launch_head_lds(const FallbackArgs& f, dim3 grid, hipStream_t stream) {
  constexpr int kWaves = kHeadLdsWaves;
  constexpr int kBlocks = static_cast<int>(kHeadTileBlocks) / kWaves;
  const uint32_t lds = static_cast<uint32_t>(sizeof(HeadEpi) + panel_tile_bytes(32u * kSteps));
  hipLaunchKernelGGL((vocab_head_lds_kernel<kWaves, kBlocks, kSteps>), grid, dim3(kWaves * 64), lds,
                     stream, f);
}

hipError_t launch_fallback(const FallbackArgs& args, hipStream_t stream) {
  if (args.m == 0) return hipSuccess;
  if (args.H % 64 != 0 || args.panel == nullptr) return hipErrorInvalidValue;
  // runs of tiles per workgroup: as many workgroups as compute units (or
  // tiles), every run the same length
  const uint32_t tiles = fallback_tiles(args.V);
  const uint32_t groups = args.groups > 0 ? args.groups : 256u;
  FallbackArgs f = args;
  f.tiles_per_group = (tiles + groups - 1) / groups;
  const dim3 grid((tiles + f.tiles_per_group - 1) / f.tiles_per_group, panel_tiles(args.m));
  const uint32_t steps = args.H / 32;  // even
  if (panel_tile_bytes(args.H) <= kPanelLdsMaxBytes) {
    switch (steps) {
      case 2: launch_head_lds<2>(f, grid, stream); break;
      case 4: launch_head_lds<4>(f, grid, stream); break;
      case 6: launch_head_lds<6>(f, grid, stream); break;
      case 8: launch_head_lds<8>(f, grid, stream); break;
      case 10: launch_head_lds<10>(f, grid, stream); break;
      case 12: launch_head_lds<12>(f, grid, stream); break;
      case 14: launch_head_lds<14>(f, grid, stream); break;
      case 16: launch_head_lds<16>(f, grid, stream); break;
      case 18: launch_head_lds<18>(f, grid, stream); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    const uint32_t lds = static_cast<uint32_t>(sizeof(HeadEpi));
    const dim3 block(kWideWaves * 64);
    // units of two steps: wider units spill (A and B of a unit share the
    // registers)
    hipLaunchKernelGGL((vocab_head_wide_kernel<2>), grid, block, lds, stream, f);
  }
  return hipGetLastError();
}

} // namespace mf
