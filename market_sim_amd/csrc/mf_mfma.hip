// gfx950 MFMA kernels: the dense full-vocabulary projection Y * E^T.
//
// Used for (1) the fallback head of unrestricted rows (windowed-argmax
// epilogue writing tile records; no logits written), (2) the
// full-output-projection comparator (FP32 scores), and (3) linear_f16 (FP16
// logits, the reference's cublasGemmEx call).
//
// Tiling: a 256-thread workgroup owns 32 A rows (hidden vectors) x 128
// tokens; each wave computes one 32x32 block with v_mfma_f32_32x32x16_f16.
// K runs in chunks of 64 features.  Per chunk the workgroup stages the
// 128 x 64 FP16 slice of E and the 32 x 64 A slice in LDS (double-buffered,
// rows padded to 144 bytes so b128 reads are bank-conflict free): eight
// consecutive lanes load one token's 128 contiguous bytes, so every HBM line
// is fetched once, and four chunks' global loads are in flight (in
// registers) while the staged chunk's MFMAs run.
//
// FP32 hidden values enter as the FP16 pair hi = rne(y), lo = rne(y - hi)
// (two MFMAs per step into two accumulators, added at the end), so the fast
// score is accurate to ~2^-22 relative before the reference-order rescore.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
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
  const AView A{p.y, p.a16, nullptr, p.row_index, p.m, p.rows, p.H};
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

// ---- MFMA head of the unrestricted rows -----------------------------------
//
// A workgroup owns the 32 rows of an M-tile and a contiguous run of 192-token
// tiles (one window record per row and tile); the runs are sized so that
// every compute unit gets the same number of tiles.  Each wave owns 48
// tokens of a tile, three 16-token blocks of v_mfma_f32_16x16x32_f16, and
// all 32 rows as four 16-row blocks: A rows 2j and 2j + 1 of block rb are
// the hi and lo halves of row 8 rb + j.  In the 16x16x32 layout lane l holds
// 8 consecutive features of column / A row l % 16 at k-block l / 16, so the
// four lanes of a token read 64 contiguous bytes per step.  The table rows
// go straight from memory into the MFMA registers, two units of KC steps in
// flight; A comes from an LDS stage of the M-tile's FP16 split (while it
// fits two 32-row stages... one per workgroup) or, for wide rows, from L2.
// A second MFMA of each token block with itself gives the squared token
// norms (Gram diagonal) for the error bound.

typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kHeadBlocks = 3;                                   // per wave
constexpr uint32_t kHeadTileTokens = (kThreads / 64) * 16 * kHeadBlocks;  // 192
constexpr uint32_t kAStagePad = 8;  // halves; spreads the 16 row-parts of a read over banks
__host__ __device__ constexpr uint32_t a_stage_bytes(uint32_t H) {
  return kMTile * 2u * (H + kAStagePad) * 2u;
}
constexpr uint32_t kAStageMaxBytes = 76u * 1024u;

// Per-wave partial results of the tile's window records.
struct HeadEpi {
  float lo[kThreads / 64][kMTile];
  uint32_t fin[kThreads / 64][kMTile];
  uint32_t cnt[kThreads / 64][kMTile];
};

// Units of KC steps: table rows only (A from LDS) or table rows and A (A
// from L2).  All loads are straight-line: a load under a branch makes the
// compiler wait for every load in flight before the next MFMA.
template <int KC>
struct BUnit {
  half8_t b[kHeadBlocks][KC];
};
template <int KC>
struct ABUnit {
  half8_t b[kHeadBlocks][KC];
  half8_t a[4][KC];
};

template <int KC>
__device__ __forceinline__ void unit_load(const uint16_t* const (&bptr)[kHeadBlocks],
                                          uint32_t f0, BUnit<KC>& u) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
#pragma unroll
    for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
      u.b[tb][s] = *reinterpret_cast<const half8_t*>(bptr[tb] + f0 + s * 32);
    }
  }
}
template <int KC>
__device__ __forceinline__ void unit_load(const uint16_t* const (&bptr)[kHeadBlocks],
                                          const uint16_t* const (&aptr)[4], uint32_t f0,
                                          ABUnit<KC>& u) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
#pragma unroll
    for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
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

struct HeadAcc {
  floatx4 acc[4][kHeadBlocks];
  floatx4 gram[kHeadBlocks];
};

// MFMAs of one unit.  A from the LDS stage: a_lane points at the lane's
// row-part of block 0 (rows outside the M-tile are zero in the stage).
template <int KC>
__device__ __forceinline__ void unit_mma(const BUnit<KC>& u, const uint16_t* a_lane,
                                         uint32_t rb_stride, uint32_t f0, HeadAcc& h) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
#pragma unroll
    for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
      h.gram[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(u.b[tb][s], u.b[tb][s], h.gram[tb], 0, 0, 0);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const half8_t a = *reinterpret_cast<const half8_t*>(a_lane + rb * rb_stride + f0 + s * 32);
#pragma unroll
      for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
        h.acc[rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, u.b[tb][s], h.acc[rb][tb], 0, 0, 0);
      }
    }
  }
}
// A from L2, rows outside the M-tile masked
template <int KC>
__device__ __forceinline__ void unit_mma(const ABUnit<KC>& u, const uint32_t (&amask)[4],
                                         HeadAcc& h) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
#pragma unroll
    for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
      h.gram[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(u.b[tb][s], u.b[tb][s], h.gram[tb], 0, 0, 0);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const half8_t a = masked(u.a[rb][s], amask[rb]);
#pragma unroll
      for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
        h.acc[rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, u.b[tb][s], h.acc[rb][tb], 0, 0, 0);
      }
    }
  }
}

// kALds: A from the LDS stage; otherwise from L2 (wide rows).  KC steps per
// unit, two units in flight; the steady-state loop has no branch around a
// load, and sched_barrier(0) keeps each unit's loads issued before the
// previous unit's MFMAs (the scheduler would otherwise sink them past the
// MFMAs and every unit would wait a full round trip).
template <bool kALds, int KC, bool kScores>
__global__ __launch_bounds__(kThreads) void vocab_head_kernel(FallbackArgs f) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t src_row[kMTile];
  __shared__ float src_norm[kMTile];
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
  const AView A{nullptr, f.y_hi, f.y_lo, f.row_index, f.m, f.rows, H};
  const uint32_t row_halves = H + kAStagePad;
  uint16_t* stage = reinterpret_cast<uint16_t*>(dyn + sizeof(HeadEpi));
  const uint32_t units = H / (32 * KC);
  constexpr uint32_t kUnitF = 32 * KC;
  // table-row pointers of tile t for this lane
  auto tile_rows = [&](uint32_t t, const uint16_t* (&bptr)[kHeadBlocks]) {
#pragma unroll
    for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
      const uint32_t token = t * kHeadTileTokens + wave * (16 * kHeadBlocks) + tb * 16 + col;
      bptr[tb] = f.emb + static_cast<uint64_t>(token < f.V ? token : 0u) * H + kb * 8;
    }
  };
  const uint16_t* bptr[kHeadBlocks];
  tile_rows(t_begin, bptr);
  // the first unit of the first tile is in flight during the row lookups
  // and the A staging
  BUnit<KC> b0;
  if constexpr (kALds) unit_load<KC>(bptr, 0, b0);
  if (threadIdx.x < kMTile) {
    const uint32_t row = a_source_row(A, m0 + threadIdx.x);
    const bool ok = row < f.rows;
    src_row[threadIdx.x] = ok ? row : 0xFFFFFFFFu;
    src_norm[threadIdx.x] = ok ? f.row_norm[row] : 0.0f;
    if (blockIdx.x == 0 && ok && f.fb_map != nullptr) f.fb_map[row] = m0 + threadIdx.x;
  }
  __syncthreads();
  if constexpr (kALds) {
    // the M-tile's FP16 split, [row][hi|lo][H + pad], zero rows beyond it;
    // kStageBatch loads per thread are in flight before their stores (a
    // copy loop that stores each load before the next would pay one round
    // trip per iteration)
    constexpr uint32_t kStageBatch = 6;
    const uint32_t per = H / 8;
    const uint32_t n = 64u * per;
    for (uint32_t base = threadIdx.x; base < n; base += kThreads * kStageBatch) {
      uint4 v[kStageBatch];
#pragma unroll
      for (uint32_t u = 0; u < kStageBatch; ++u) {
        const uint32_t q = base + u * kThreads;
        const uint32_t p = q / per;
        const uint32_t row = q < n ? src_row[p / 2] : 0xFFFFFFFFu;
        v[u] = row != 0xFFFFFFFFu
                   ? *reinterpret_cast<const uint4*>(((p & 1u) ? f.y_lo : f.y_hi) +
                                                    static_cast<uint64_t>(row) * H + (q % per) * 8)
                   : uint4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (uint32_t u = 0; u < kStageBatch; ++u) {
        const uint32_t q = base + u * kThreads;
        if (q < n) *reinterpret_cast<uint4*>(stage + (q / per) * row_halves + (q % per) * 8) = v[u];
      }
    }
    __syncthreads();
  }
  const uint16_t* a_lane = stage + col * row_halves + kb * 8;  // LDS variant
  const uint32_t rb_stride = 16u * row_halves;
  const uint16_t* aptr[4];                                     // L2 variant
  uint32_t amask[4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const uint32_t row = src_row[rb * 8 + col / 2];
    const bool ok = row != 0xFFFFFFFFu;
    aptr[rb] = ((col & 1u) ? f.y_lo : f.y_hi) + static_cast<uint64_t>(ok ? row : 0u) * H + kb * 8;
    amask[rb] = ok ? 0xFFFFFFFFu : 0u;
  }

  for (uint32_t tile = t_begin; tile < t_end; ++tile) {
    if (tile != t_begin) tile_rows(tile, bptr);
    HeadAcc h;
#pragma unroll
    for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
      h.gram[tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) h.acc[rb][tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if constexpr (kALds) {
      BUnit<KC> u0, u1;
      if (tile == t_begin) {
        u0 = b0;
      } else {
        unit_load<KC>(bptr, 0, u0);
      }
      uint32_t q = 0;
      for (; q + 2 < units; q += 2) {
        unit_load<KC>(bptr, (q + 1) * kUnitF, u1);
        __builtin_amdgcn_sched_barrier(0);
        unit_mma<KC>(u0, a_lane, rb_stride, q * kUnitF, h);
        __builtin_amdgcn_sched_barrier(0);
        unit_load<KC>(bptr, (q + 2) * kUnitF, u0);
        __builtin_amdgcn_sched_barrier(0);
        unit_mma<KC>(u1, a_lane, rb_stride, (q + 1) * kUnitF, h);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (q + 1 < units) {  // the last two units
        unit_load<KC>(bptr, (q + 1) * kUnitF, u1);
        __builtin_amdgcn_sched_barrier(0);
        unit_mma<KC>(u0, a_lane, rb_stride, q * kUnitF, h);
        unit_mma<KC>(u1, a_lane, rb_stride, (q + 1) * kUnitF, h);
      } else {
        unit_mma<KC>(u0, a_lane, rb_stride, q * kUnitF, h);
      }
    } else {
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
    }

    if constexpr (kScores) {
      // the comparator: every score of the tile, and the token norms
      const uint32_t tok0 = tile * kHeadTileTokens;
#pragma unroll
      for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
        const uint32_t token = tok0 + wave * (16 * kHeadBlocks) + tb * 16 + col;
        const uint32_t e = col % 4u;
        const float d = e == 0u ? h.gram[tb][0]
                                : (e == 1u ? h.gram[tb][1] : (e == 2u ? h.gram[tb][2] : h.gram[tb][3]));
        const float tsq = __shfl(d, static_cast<int>(col + 16u * (col / 4u)));
        if (token >= f.V) continue;
        if (blockIdx.y == 0 && kb == 0u && f.tok_norm != nullptr) {
          f.tok_norm[token] = __fsqrt_rn(tsq) * (1.0f + 0x1p-7f);
        }
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const uint32_t i = rb * 8 + 2 * kb + jj;
            if (m0 + i < f.m) {
              f.scores[static_cast<uint64_t>(m0 + i) * f.V + token] =
                  h.acc[rb][tb][2 * jj] + h.acc[rb][tb][2 * jj + 1];
            }
          }
        }
      }
      continue;
    }
    // The tile's window records, reduced in registers.  Lane l holds
    // D[4 (l / 16) + i][l % 16] of each block: rows 2j, 2j + 1 (hi, lo of
    // row 8 rb + j) for j = 2 kb and 2 kb + 1, so the scores of row
    // 8 rb + 2 kb + jj (jj = 0, 1) are h.acc[rb][tb][2 jj] + [2 jj + 1] for
    // the wave's tokens wave * 48 + 16 tb + col.  The Gram diagonal of
    // column c sits in lane c + 16 (c / 4), element c % 4.
    const uint32_t tok0 = tile * kHeadTileTokens;
    const uint32_t nt = f.V - tok0 < kHeadTileTokens ? f.V - tok0 : kHeadTileTokens;
    float g[4][2][kHeadBlocks];
    float b[4][2][kHeadBlocks];
    bool valid[kHeadBlocks];
#pragma unroll
    for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
      const uint32_t e = col % 4u;
      const float d = e == 0u ? h.gram[tb][0]
                              : (e == 1u ? h.gram[tb][1] : (e == 2u ? h.gram[tb][2] : h.gram[tb][3]));
      const float tsq = __shfl(d, static_cast<int>(col + 16u * (col / 4u)));
      const float tok_norm = __fsqrt_rn(tsq) * (1.0f + 0x1p-7f);
      valid[tb] = wave * (16 * kHeadBlocks) + tb * 16 + col < nt;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const uint32_t i = rb * 8 + 2 * kb + jj;
          g[rb][jj][tb] = h.acc[rb][tb][2 * jj] + h.acc[rb][tb][2 * jj + 1];
          b[rb][jj][tb] =
              __builtin_fmaf(tok_norm, __builtin_fmaf(f.coef, src_norm[i], f.coef2), f.slack);
        }
      }
    }
    // per row: the best lower bound g - b and finiteness, over the lane's
    // tokens, then over the 16 lanes of the row, then over the 4 waves
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        float lo = -__builtin_huge_valf();
        uint32_t fin = 1u;
#pragma unroll
        for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
          if (!valid[tb]) continue;
          const float gv = g[rb][jj][tb];
          const float bv = b[rb][jj][tb];
          fin &= (__builtin_isfinite(gv) && __builtin_isfinite(bv) && bv < 0x1p100f) ? 1u : 0u;
          lo = __builtin_fmaxf(lo, gv - bv);
        }
#pragma unroll
        for (int m = 8; m > 0; m >>= 1) {
          lo = __builtin_fmaxf(lo, __shfl_xor(lo, m, 16));
          fin &= __shfl_xor(fin, m, 16);
        }
        if (col == 0u) {
          epi.lo[wave][rb * 8 + 2 * kb + jj] = lo;
          epi.fin[wave][rb * 8 + 2 * kb + jj] = fin;
        }
      }
    }
    __syncthreads();
    // members (g + b >= L) per row: count per wave, rank across waves
    float L[4][2];
    uint32_t rowfin[4][2];
    uint32_t below[4][2][kHeadBlocks];  // members of this row before (tb, col) in the wave
    uint32_t mine[4][2];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const uint32_t i = rb * 8 + 2 * kb + jj;
        float l = epi.lo[0][i];
        uint32_t fn = epi.fin[0][i];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
          l = __builtin_fmaxf(l, epi.lo[w][i]);
          fn &= epi.fin[w][i];
        }
        L[rb][jj] = l;
        rowfin[rb][jj] = fn;
        uint32_t run = 0u;
#pragma unroll
        for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
          const bool member = valid[tb] && g[rb][jj][tb] + b[rb][jj][tb] >= l;
          const uint64_t mask = __ballot(member);
          const uint32_t group = static_cast<uint32_t>(mask >> (16u * kb)) & 0xFFFFu;
          below[rb][jj][tb] = run + static_cast<uint32_t>(__popc(group & ((1u << col) - 1u)));
          run += static_cast<uint32_t>(__popc(group));
        }
        mine[rb][jj] = run;
        if (col == 0u) epi.cnt[wave][i] = run;
      }
    }
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const uint32_t i = rb * 8 + 2 * kb + jj;
        if (src_row[i] == 0xFFFFFFFFu) continue;
        uint32_t base = 0u;
        uint32_t total = 0u;
#pragma unroll
        for (uint32_t w = 0; w < 4; ++w) {
          const uint32_t c = epi.cnt[w][i];
          base += w < wave ? c : 0u;
          total += c;
        }
        const bool ordinary = rowfin[rb][jj] && total <= static_cast<uint32_t>(kTileMembers);
        TileRecord* rec = f.records + static_cast<uint64_t>(m0 + i) * tiles + tile;
        if (ordinary) {
#pragma unroll
          for (uint32_t tb = 0; tb < kHeadBlocks; ++tb) {
            const float gv = g[rb][jj][tb];
            const float bv = b[rb][jj][tb];
            if (valid[tb] && gv + bv >= L[rb][jj]) {
              const uint32_t token = tok0 + wave * (16 * kHeadBlocks) + tb * 16 + col;
              rec->m[base + below[rb][jj][tb]] = TileMember{token, token, gv - bv, gv + bv};
            }
          }
        }
        if (wave == 0 && col == 0u) {
          rec->best_lower = L[rb][jj];
          rec->flags = ordinary ? 0u : kTileRescoreAll;
          rec->min_token = tok0;
          rec->min_pos = tok0;
          rec->begin = tok0;
          rec->count = nt;
          rec->n_members = ordinary ? total : 0u;
        }
      }
    }
    (void)mine;
    __syncthreads();  // the next tile rewrites the scores
  }
}

} // namespace

uint32_t fallback_tiles(uint32_t vocab) {
  return (vocab + kHeadTileTokens - 1) / kHeadTileTokens;
}

hipError_t launch_projection(const ProjArgs& args, hipStream_t stream) {
  if (args.H % kKC != 0) return hipErrorInvalidValue;
  const dim3 grid((args.V + kTileTokens - 1) / kTileTokens, (args.m + kMTile - 1) / kMTile);
  if (args.a16 != nullptr) {
    hipLaunchKernelGGL((projection_kernel<ASrc::kF16>), grid, dim3(kThreads), 0, stream, args);
  } else {
    hipLaunchKernelGGL((projection_kernel<ASrc::kF32Split>), grid, dim3(kThreads), 0, stream, args);
  }
  return hipGetLastError();
}

template <bool kALds, int KC, bool kScores>
static void launch_head(const FallbackArgs& f, dim3 grid, uint32_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((vocab_head_kernel<kALds, KC, kScores>), grid, dim3(kThreads), lds, stream, f);
}

template <bool kScores>
static hipError_t launch_vocab(const FallbackArgs& args, hipStream_t stream) {
  if (args.m == 0) return hipSuccess;
  if (args.H % 64 != 0) return hipErrorInvalidValue;
  // runs of tiles per workgroup: as many workgroups as compute units (or
  // tiles), every run the same length
  const uint32_t tiles = fallback_tiles(args.V);
  const uint32_t groups = args.groups > 0 ? args.groups : 256u;
  FallbackArgs f = args;
  f.tiles_per_group = (tiles + groups - 1) / groups;
  const dim3 grid((tiles + f.tiles_per_group - 1) / f.tiles_per_group,
                  (args.m + kMTile - 1) / kMTile);
  const uint32_t steps = args.H / 32;  // even
  const uint32_t stage = a_stage_bytes(args.H);
  if (stage <= kAStageMaxBytes) {
    const uint32_t lds = static_cast<uint32_t>(sizeof(HeadEpi)) + stage;
    if (steps % 6 == 0) {
      launch_head<true, 6, kScores>(f, grid, lds, stream);
    } else if (steps % 4 == 0) {
      launch_head<true, 4, kScores>(f, grid, lds, stream);
    } else {
      launch_head<true, 2, kScores>(f, grid, lds, stream);
    }
  } else {
    launch_head<false, 2, kScores>(f, grid, static_cast<uint32_t>(sizeof(HeadEpi)), stream);
  }
  return hipGetLastError();
}

hipError_t launch_fallback(const FallbackArgs& args, hipStream_t stream) {
  return launch_vocab<false>(args, stream);
}

hipError_t launch_vocab_scores(const FallbackArgs& args, hipStream_t stream) {
  if (args.scores == nullptr) return hipErrorInvalidValue;
  return launch_vocab<true>(args, stream);
}

} // namespace mf
