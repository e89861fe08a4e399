// gfx950 MFMA kernels: dense products against the whole FP16 table.
//
// (1) The head of the unrestricted rows (vocab_head_*_kernel): every token's
//     score against the rows' FP16 hi/lo split, reduced in a windowed-argmax
//     epilogue to tile records (no logits written).
// (2) linear_f16 (projection_kernel): FP16 logits, the reference's
//     cublasGemmEx call.  Tiling: a 256-thread workgroup owns 32 A rows x 128
//     tokens; each wave computes one 32x32 block with
//     v_mfma_f32_32x32x16_f16.  K runs in chunks of 64 features; per chunk
//     the workgroup stages the 128 x 64 FP16 slice of E and the 32 x 64 A
//     slice in LDS (double-buffered, rows padded to 144 bytes so b128 reads
//     are bank-conflict free), with four chunks' global loads in flight.
//
// FP32 hidden values enter as the FP16 pair hi = rne(y), lo = rne(y - hi)
// (two MFMAs per step), so the fast score is accurate to ~2^-22 relative
// before the reference-order rescore.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"
#include "mf_head.hpp"

namespace mf {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTileTokens = 128;
constexpr int kMTile = 32;
constexpr int kKC = 64;          // features per chunk
constexpr int kRowHalves = 72;   // padded LDS row: 64 + 8 halves = 144 B

struct ProjShared {
  union {
    struct {
      _Float16 b[2][kTileTokens][kRowHalves];   // 36,864 B
      _Float16 a[2][2][kMTile][kRowHalves];     // [buf][hi|lo] 18,432 B
    } k;
    struct {
      float g[kMTile][kTileTokens];
      float b[kMTile][kTileTokens];
    } epi;                                      // 32,768 B
  };
};

enum class ASrc { kF32Split, kF16Pair, kF16 };

struct AView {
  const float* y;           // kF32Split
  const uint16_t* hi;       // kF16Pair, kF16
  const uint16_t* lo;       // kF16Pair
  const uint32_t* row_index;
  uint32_t m;
  uint32_t rows;
  uint32_t H;
};

// Source row of A row m (row_index applied; 0xFFFFFFFF reads as zeros).
__device__ __forceinline__ uint32_t a_source_row(const AView& A, uint32_t m) {
  if (m >= A.m) return 0xFFFFFFFFu;
  return A.row_index != nullptr ? A.row_index[m] : m;
}

// Per-thread registers holding one chunk in flight: 4 B pieces (16 B each)
// and the A piece (hi and lo, 16 B each).
struct ChunkRegs {
  uint4 b[4];
  uint4 ahi;
  uint4 alo;
};

template <ASrc kA>
__device__ __forceinline__ void load_chunk(const AView& A, const uint16_t* emb, uint32_t V,
                                           uint32_t tok0, uint32_t row, uint32_t c,
                                           ChunkRegs& r) {
  const uint32_t t = threadIdx.x;
  const uint32_t part = t % 8;
  const uint32_t f = c * kKC + part * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t token = tok0 + t / 8 + 32 * j;
    r.b[j] = token < V ? *reinterpret_cast<const uint4*>(emb + static_cast<uint64_t>(token) * A.H + f)
                       : uint4{0u, 0u, 0u, 0u};
  }
  // A: 32 rows x 8 pieces = 256 pieces, one per thread (row resolved by
  // the caller once per kernel)
  r.ahi = uint4{0u, 0u, 0u, 0u};
  r.alo = uint4{0u, 0u, 0u, 0u};
  if (row < A.rows) {
    const uint64_t o = static_cast<uint64_t>(row) * A.H + f;
    if constexpr (kA == ASrc::kF32Split) {
      const float4* src = reinterpret_cast<const float4*>(A.y + o);
      const float4 v0 = src[0];
      const float4 v1 = src[1];
      const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
      half8_t hi, lo;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const _Float16 h = static_cast<_Float16>(v[k]);
        hi[k] = h;
        lo[k] = static_cast<_Float16>(v[k] - static_cast<float>(h));
      }
      r.ahi = __builtin_bit_cast(uint4, hi);
      r.alo = __builtin_bit_cast(uint4, lo);
    } else {
      r.ahi = *reinterpret_cast<const uint4*>(A.hi + o);
      if constexpr (kA == ASrc::kF16Pair) r.alo = *reinterpret_cast<const uint4*>(A.lo + o);
    }
  }
}

__device__ __forceinline__ void store_chunk(ProjShared& sh, int buf, const ChunkRegs& r) {
  const uint32_t t = threadIdx.x;
  const uint32_t part = t % 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    *reinterpret_cast<uint4*>(&sh.k.b[buf][t / 8 + 32 * j][part * 8]) = r.b[j];
  }
  *reinterpret_cast<uint4*>(&sh.k.a[buf][0][t / 8][part * 8]) = r.ahi;
  *reinterpret_cast<uint4*>(&sh.k.a[buf][1][t / 8][part * 8]) = r.alo;
}

// MFMAs of one staged chunk (LDS buffer buf): the hi and lo halves of A
// accumulate separately (two independent MFMA chains) and are added once at
// the end.
template <ASrc kA>
__device__ __forceinline__ void mma_chunk(const ProjShared& sh, int buf, floatx16& acc_hi,
                                          floatx16& acc_lo, float& tok_sq) {
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const int g = lane / 32;
  const int i = lane % 32;
#pragma unroll
  for (int s = 0; s < kKC / 16; ++s) {
    const half8_t b = *reinterpret_cast<const half8_t*>(&sh.k.b[buf][wave * 32 + i][s * 16 + g * 8]);
    const half8_t ahi = *reinterpret_cast<const half8_t*>(&sh.k.a[buf][0][i][s * 16 + g * 8]);
    acc_hi = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi, b, acc_hi, 0, 0, 0);
    if constexpr (kA != ASrc::kF16) {
      const half8_t alo = *reinterpret_cast<const half8_t*>(&sh.k.a[buf][1][i][s * 16 + g * 8]);
      acc_lo = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo, b, acc_lo, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float e = static_cast<float>(b[k]);
      tok_sq = __builtin_fmaf(e, e, tok_sq);
    }
  }
}

// Step c of the pipeline (chunk k travels through register set k % 4): the
// load of chunk c + 4 into the set chunk c left, the MFMAs of chunk c, then
// chunk c + 1 into the other LDS buffer.  Four chunks are in flight from
// HBM while one is multiplied.
template <ASrc kA>
__device__ __forceinline__ void pipeline_step(const AView& A, const uint16_t* emb, uint32_t V,
                                              uint32_t tok0, uint32_t arow, uint32_t c,
                                              uint32_t chunks, ChunkRegs& free_set,
                                              const ChunkRegs& next_set, ProjShared& sh,
                                              floatx16& acc_hi, floatx16& acc_lo,
                                              float& tok_sq) {
  if (c >= chunks) return;
  if (c + 4 < chunks) load_chunk<kA>(A, emb, V, tok0, arow, c + 4, free_set);
  mma_chunk<kA>(sh, c & 1, acc_hi, acc_lo, tok_sq);
  if (c + 1 < chunks) store_chunk(sh, (c + 1) & 1, next_set);
  __syncthreads();
}

// The wave's 32 x 32 block (rows m0.., tokens tok0 + 32 * wave ..).  Returns
// the accumulator and the lane's sum of squares of its B values; combined
// across the two lane groups that is ||e_token||^2 of token lane % 32.
template <ASrc kA>
__device__ floatx16 project_block(const AView& A, const uint16_t* emb, uint32_t V,
                                  uint32_t m0, uint32_t tok0, ProjShared& sh, float& tok_sq) {
  floatx16 acc_hi, acc_lo;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    acc_hi[v] = 0.0f;
    acc_lo[v] = 0.0f;
  }
  tok_sq = 0.0f;
  const uint32_t chunks = A.H / kKC;
  const uint32_t arow = a_source_row(A, m0 + threadIdx.x / 8);
  ChunkRegs r0, r1, r2, r3;
  load_chunk<kA>(A, emb, V, tok0, arow, 0, r0);
  if (chunks > 1) load_chunk<kA>(A, emb, V, tok0, arow, 1, r1);
  if (chunks > 2) load_chunk<kA>(A, emb, V, tok0, arow, 2, r2);
  if (chunks > 3) load_chunk<kA>(A, emb, V, tok0, arow, 3, r3);
  store_chunk(sh, 0, r0);
  __syncthreads();
  for (uint32_t c = 0; c < chunks; c += 4) {
    pipeline_step<kA>(A, emb, V, tok0, arow, c, chunks, r0, r1, sh, acc_hi, acc_lo, tok_sq);
    pipeline_step<kA>(A, emb, V, tok0, arow, c + 1, chunks, r1, r2, sh, acc_hi, acc_lo, tok_sq);
    pipeline_step<kA>(A, emb, V, tok0, arow, c + 2, chunks, r2, r3, sh, acc_hi, acc_lo, tok_sq);
    pipeline_step<kA>(A, emb, V, tok0, arow, c + 3, chunks, r3, r0, sh, acc_hi, acc_lo, tok_sq);
  }
  tok_sq += __shfl_xor(tok_sq, 32);
  if constexpr (kA == ASrc::kF16) return acc_hi;
  return acc_hi + acc_lo;
}

// Accumulator element v of lane l holds D[row][col] with col = l % 32 and
// row = 8 * (v / 4) + 4 * (l / 32) + v % 4 (the 32x32 MFMA output layout).
__device__ __forceinline__ int acc_row(int v, int lane) {
  return 8 * (v / 4) + 4 * (lane / 32) + (v % 4);
}

template <ASrc kA>
__global__ __launch_bounds__(kThreads) void projection_kernel(ProjArgs p) {
  __shared__ ProjShared sh;
  const uint32_t m0 = blockIdx.y * kMTile;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const uint32_t tok0 = blockIdx.x * kTileTokens;
  const uint32_t token = tok0 + wave * 32 + (lane % 32);
  const AView A{p.y, p.a16, p.a16_lo, p.row_index, p.m, p.rows, p.H};
  float tok_sq;
  const floatx16 acc = project_block<kA>(A, p.emb, p.V, m0, tok0, sh, tok_sq);
  if (token >= p.V) return;
  if (p.tok_norm != nullptr && blockIdx.y == 0 && lane < 32) {
    p.tok_norm[token] = __fsqrt_rn(tok_sq) * (1.0f + 0x1p-7f);
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const uint32_t row = m0 + acc_row(v, lane);
    if (row < p.m) {
      const uint64_t o = static_cast<uint64_t>(row) * p.V + token;
      if (p.out_f32 != nullptr) p.out_f32[o] = acc[v];
      if (p.out_f16 != nullptr) p.out_f16[o] = float_to_half_rne(acc[v]);
    }
  }
}

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

hipError_t launch_projection(const ProjArgs& args, hipStream_t stream) {
  if (args.H % kKC != 0) return hipErrorInvalidValue;
  const dim3 grid((args.V + kTileTokens - 1) / kTileTokens, (args.m + kMTile - 1) / kMTile);
  if (args.a16 != nullptr && args.a16_lo != nullptr) {
    hipLaunchKernelGGL((projection_kernel<ASrc::kF16Pair>), grid, dim3(kThreads), 0, stream, args);
  } else if (args.a16 != nullptr) {
    hipLaunchKernelGGL((projection_kernel<ASrc::kF16>), grid, dim3(kThreads), 0, stream, args);
  } else {
    hipLaunchKernelGGL((projection_kernel<ASrc::kF32Split>), grid, dim3(kThreads), 0, stream, args);
  }
  return hipGetLastError();
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
