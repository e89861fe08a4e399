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

// Window records of one 128-token tile for the (up to) 32 rows of an
// M-tile, from scores and bounds staged in LDS: per row, eight lanes cover
// 16 tokens each.  Called by all 256 threads after a barrier.
__device__ void write_fallback_records(const FallbackArgs& f, const float (*g_tile)[kTileTokens],
                                       const float (*b_tile)[kTileTokens],
                                       const uint32_t* src_row, uint32_t m0, uint32_t tile,
                                       uint32_t tiles) {
  const uint32_t tok0 = tile * kTileTokens;
  // per row (8 lanes, 16 tokens each): the tile's window record
  const uint32_t i = threadIdx.x / 8;
  const uint32_t sub = threadIdx.x % 8;
  const uint32_t nt = f.V - tok0 < kTileTokens ? f.V - tok0 : kTileTokens;
  uint32_t fin = 1u;
  float lo = -__builtin_huge_valf();
  for (uint32_t c = sub; c < nt; c += 8) {
    const float g = g_tile[i][c];
    const float b = b_tile[i][c];
    fin &= (__builtin_isfinite(g) && __builtin_isfinite(b) && b < 0x1p100f) ? 1u : 0u;
    lo = __builtin_fmaxf(lo, g - b);
  }
  fin = group8_and(fin);
  const float L = group8_max(lo);
  uint32_t cnt = 0u;
  for (uint32_t c = sub; c < nt; c += 8) cnt += (g_tile[i][c] + b_tile[i][c] >= L) ? 1u : 0u;
  // exclusive prefix of the member counts across the row's 8 lanes
  uint32_t incl = cnt;
#pragma unroll
  for (int d = 1; d < 8; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d, 8);
    if (static_cast<int>(sub) >= d) incl += o;
  }
  const uint32_t total = __shfl(incl, 7, 8);
  const bool row_ok = src_row[i] != 0xFFFFFFFFu;
  if (!row_ok) return;
  TileRecord* rec = f.records + static_cast<uint64_t>(m0 + i) * tiles + tile;
  const bool ordinary = fin && total <= static_cast<uint32_t>(kTileMembers);
  if (ordinary) {
    uint32_t rank = incl - cnt;
    for (uint32_t c = sub; c < nt; c += 8) {
      const float g = g_tile[i][c];
      const float b = b_tile[i][c];
      if (g + b >= L) {
        rec->m[rank] = TileMember{tok0 + c, tok0 + c, g - b, g + b};
        ++rank;
      }
    }
  }
  if (sub == 0) {
    rec->best_lower = L;
    rec->flags = ordinary ? 0u : kTileRescoreAll;
    rec->min_token = tok0;
    rec->min_pos = tok0;
    rec->begin = tok0;
    rec->count = nt;
    rec->n_members = ordinary ? total : 0u;
  }
}

__global__ __launch_bounds__(kThreads) void fallback_kernel(FallbackArgs f) {
  __shared__ ProjShared sh;
  __shared__ uint32_t src_row[kMTile];  // source row of A row i (>= rows: none)
  __shared__ float src_norm[kMTile];    // its ||y|| bound
  const uint32_t tile = blockIdx.x;
  const uint32_t m0 = blockIdx.y * kMTile;
  const uint32_t tiles = gridDim.x;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const uint32_t tok0 = tile * kTileTokens;
  const AView A{nullptr, f.y_hi, f.y_lo, f.row_index, f.m, f.rows, f.H};
  // resolved before the main loop (its first barrier publishes them), so
  // the epilogue waits on no global load
  if (threadIdx.x < kMTile) {
    const uint32_t row = a_source_row(A, m0 + threadIdx.x);
    const bool ok = row < f.rows;
    src_row[threadIdx.x] = ok ? row : 0xFFFFFFFFu;
    src_norm[threadIdx.x] = ok ? f.row_norm[row] : 0.0f;
    if (tile == 0 && ok) f.fb_map[row] = m0 + threadIdx.x;
  }
  float tok_sq;
  const floatx16 acc = project_block<ASrc::kF16Pair>(A, f.emb, f.V, m0, tok0, sh, tok_sq);

  // scores and bounds into LDS (the staging area is free after the loop)
  const float tok_norm = __fsqrt_rn(tok_sq) * (1.0f + 0x1p-7f);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int i = acc_row(v, lane);
    const float yn = src_norm[i];
    sh.epi.g[i][wave * 32 + (lane % 32)] = acc[v];
    sh.epi.b[i][wave * 32 + (lane % 32)] =
        __builtin_fmaf(tok_norm, __builtin_fmaf(f.coef, yn, f.coef2), f.slack);
  }
  __syncthreads();

  write_fallback_records(f, sh.epi.g, sh.epi.b, src_row, m0, tile, tiles);
}


// ---- register-direct MFMA head ---------------------------------------------
//
// The same tiles and records as fallback_kernel, with the operands loaded
// straight from memory into the registers of v_mfma_f32_16x16x32_f16 (no
// LDS staging, no barrier until the epilogue).  Each wave owns 32 tokens
// (two 16-token blocks) of the workgroup's 128 and all 32 rows of the M-tile
// as four 16-row blocks: A rows 2j and 2j + 1 of block rb are the hi and lo
// halves of row 8 rb + j.  In the 16x16x32 layout lane l holds 8 consecutive
// features of column / A row l % 16 at k-block l / 16, so the four lanes of
// a token read 64 contiguous bytes per step.  A (the FP16 split of at most
// 32 hidden rows) is read from L2; a second MFMA of each token block with
// itself gives the squared token norms (Gram diagonal).

typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr int kDirectKC = 2;  // MFMA steps (32 features each) per unit

struct DirectUnit {
  half8_t b[2][kDirectKC];
  half8_t a[4][kDirectKC];
};

// Straight-line loads (no predication, no branches): rows outside the M-tile
// read a valid row and are zeroed by a mask applied just before the MFMA, so
// the compiler can count the loads in flight and wait only for the unit about
// to be multiplied.
__device__ __forceinline__ void direct_load(const uint16_t* const (&bptr)[2],
                                            const uint16_t* const (&aptr)[4], uint32_t f0,
                                            DirectUnit& u) {
#pragma unroll
  for (int s = 0; s < kDirectKC; ++s) {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
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

__device__ __forceinline__ void direct_mma(const DirectUnit& u, const uint32_t (&amask)[4],
                                           floatx4 (&acc)[4][2], floatx4 (&gram)[2]) {
#pragma unroll
  for (int s = 0; s < kDirectKC; ++s) {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      gram[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(u.b[tb][s], u.b[tb][s], gram[tb], 0, 0, 0);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const half8_t a = masked(u.a[rb][s], amask[rb]);
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        acc[rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, u.b[tb][s], acc[rb][tb], 0, 0, 0);
      }
    }
  }
}

// A staged in LDS: rows i of the M-tile as [i][hi|lo][H + 8] halves (the
// 16-byte pad spreads the 16 row-parts of one MFMA read over distinct banks);
// rows outside the M-tile are zero.  Used while it fits two workgroups per
// CU; the scores of the epilogue reuse the same LDS.
constexpr uint32_t kAStagePad = 8;
__host__ __device__ constexpr uint32_t a_stage_bytes(uint32_t H) {
  return kMTile * 2u * (H + kAStagePad) * 2u;
}
constexpr uint32_t kAStageMaxBytes = 76u * 1024u;

template <int KC>
struct BUnit {
  half8_t b[2][KC];
};

template <int KC>
__device__ __forceinline__ void b_load(const uint16_t* const (&bptr)[2], uint32_t f0,
                                       BUnit<KC>& u) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      u.b[tb][s] = *reinterpret_cast<const half8_t*>(bptr[tb] + f0 + s * 32);
    }
  }
}

template <int KC>
__device__ __forceinline__ void lds_a_mma(const BUnit<KC>& u, const uint16_t* a_lane, uint32_t f0,
                                          uint32_t rb_stride, floatx4 (&acc)[4][2],
                                          floatx4 (&gram)[2]) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      gram[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(u.b[tb][s], u.b[tb][s], gram[tb], 0, 0, 0);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const half8_t a = *reinterpret_cast<const half8_t*>(a_lane + rb * rb_stride + f0 + s * 32);
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        acc[rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, u.b[tb][s], acc[rb][tb], 0, 0, 0);
      }
    }
  }
}

// kALds: A from the LDS stage (one VMEM instruction per token block and
// step remains); otherwise A from L2 with B in the same units.  KC steps per
// unit with the LDS stage: two units, 2 x KC x 2 KiB of table rows, are in
// flight per wave (all of a 576-feature row at KC = 9).
template <bool kALds, int KC>
__global__ __launch_bounds__(kThreads) void fallback_direct_kernel(FallbackArgs f) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t src_row[kMTile];
  __shared__ float src_norm[kMTile];
  float(*sh_g)[kTileTokens] = reinterpret_cast<float(*)[kTileTokens]>(dyn);
  float(*sh_b)[kTileTokens] = reinterpret_cast<float(*)[kTileTokens]>(dyn + kMTile * kTileTokens * 4);
  const uint32_t tile = blockIdx.x;
  const uint32_t m0 = blockIdx.y * kMTile;
  const uint32_t tiles = gridDim.x;
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t wave = threadIdx.x / 64;
  const uint32_t tok0 = tile * kTileTokens;
  const uint32_t H = f.H;
  const uint32_t col = lane % 16;
  const uint32_t kb = lane / 16;
  const AView A{nullptr, f.y_hi, f.y_lo, f.row_index, f.m, f.rows, H};
  const uint16_t* bptr[2];
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    const uint32_t token = tok0 + wave * 32 + tb * 16 + col;
    bptr[tb] = f.emb + static_cast<uint64_t>(token < f.V ? token : 0u) * H + kb * 8;
  }
  if (threadIdx.x < kMTile) {
    const uint32_t row = a_source_row(A, m0 + threadIdx.x);
    const bool ok = row < f.rows;
    src_row[threadIdx.x] = ok ? row : 0xFFFFFFFFu;
    src_norm[threadIdx.x] = ok ? f.row_norm[row] : 0.0f;
    if (tile == 0 && ok) f.fb_map[row] = m0 + threadIdx.x;
  }

  floatx4 acc[4][2];
  floatx4 gram[2];
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    gram[tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) acc[rb][tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // units of KC steps, two in flight (H % 64 == 0).  The steady-state loop
  // has no branch around a load (a load under a branch makes the compiler
  // wait for every load in flight), and sched_barrier(0) keeps each unit's
  // loads issued before the previous unit's MFMAs (the scheduler would
  // otherwise sink them past the MFMAs and every unit would wait a full
  // round trip).
  if constexpr (kALds) {
    const uint32_t units = H / (32 * KC);
    constexpr uint32_t kUnitF = 32 * KC;
    uint16_t* stage = reinterpret_cast<uint16_t*>(dyn);
    const uint32_t row_halves = H + kAStagePad;
    BUnit<KC> u0, u1;
    b_load(bptr, 0, u0);  // in flight during the staging
    __syncthreads();      // src_row
    // stage A: 64 row-parts x H halves, 16 bytes per copy
    const uint32_t per = H / 8;
    for (uint32_t q = threadIdx.x; q < 64u * per; q += kThreads) {
      const uint32_t p = q / per;
      const uint32_t c = q % per;
      const uint32_t row = src_row[p / 2];
      uint4 v = uint4{0u, 0u, 0u, 0u};
      if (row != 0xFFFFFFFFu) {
        v = *reinterpret_cast<const uint4*>(((p & 1u) ? f.y_lo : f.y_hi) +
                                           static_cast<uint64_t>(row) * H + c * 8);
      }
      *reinterpret_cast<uint4*>(stage + p * row_halves + c * 8) = v;
    }
    __syncthreads();
    // lane's A row-part in block rb: row 8 rb + col / 2, part col & 1
    const uint16_t* a_lane = stage + col * row_halves + kb * 8;
    const uint32_t rb_stride = 16u * row_halves;
    uint32_t q = 0;
    for (; q + 2 < units; q += 2) {
      b_load(bptr, (q + 1) * kUnitF, u1);
      __builtin_amdgcn_sched_barrier(0);
      lds_a_mma(u0, a_lane, q * kUnitF, rb_stride, acc, gram);
      __builtin_amdgcn_sched_barrier(0);
      b_load(bptr, (q + 2) * kUnitF, u0);
      __builtin_amdgcn_sched_barrier(0);
      lds_a_mma(u1, a_lane, (q + 1) * kUnitF, rb_stride, acc, gram);
      __builtin_amdgcn_sched_barrier(0);
    }
    // the last one or two units
    if (q + 1 < units) {
      b_load(bptr, (q + 1) * kUnitF, u1);
      __builtin_amdgcn_sched_barrier(0);
      lds_a_mma(u0, a_lane, q * kUnitF, rb_stride, acc, gram);
      lds_a_mma(u1, a_lane, (q + 1) * kUnitF, rb_stride, acc, gram);
    } else {
      lds_a_mma(u0, a_lane, q * kUnitF, rb_stride, acc, gram);
    }
    __syncthreads();  // every wave is done with the stage before the scores reuse it
  } else {
    const uint32_t units = H / (32 * kDirectKC);
    const uint32_t last = units - 1;
    constexpr uint32_t kUnitF = 32 * kDirectKC;
    const uint16_t* aptr[4];
    uint32_t amask[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint32_t row = a_source_row(A, m0 + rb * 8 + col / 2);
      const bool ok = row < f.rows;
      aptr[rb] = ((col & 1u) ? f.y_lo : f.y_hi) + static_cast<uint64_t>(ok ? row : 0u) * H + kb * 8;
      amask[rb] = ok ? 0xFFFFFFFFu : 0u;
    }
    DirectUnit u0, u1;
    direct_load(bptr, aptr, 0, u0);
    uint32_t q = 0;
    for (; q + 1 < units; q += 2) {
      direct_load(bptr, aptr, (q + 1) * kUnitF, u1);
      __builtin_amdgcn_sched_barrier(0);
      direct_mma(u0, amask, acc, gram);
      __builtin_amdgcn_sched_barrier(0);
      direct_load(bptr, aptr, (q + 2 < last ? q + 2 : last) * kUnitF, u0);
      __builtin_amdgcn_sched_barrier(0);
      direct_mma(u1, amask, acc, gram);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (q < units) direct_mma(u0, amask, acc, gram);  // odd unit count: the last unit
    __syncthreads();  // src_row / src_norm
  }

  // scores and bounds into LDS.  Lane l holds D[4 (l / 16) + i][l % 16]:
  // rows 2j, 2j + 1 (hi, lo of row 8 rb + j) for j = 2 kb and 2 kb + 1; the
  // Gram diagonal of column c sits in lane c + 16 (c / 4), element c % 4.
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    const uint32_t e = col % 4u;
    const float d = e == 0u ? gram[tb][0]
                            : (e == 1u ? gram[tb][1] : (e == 2u ? gram[tb][2] : gram[tb][3]));
    const float tsq = __shfl(d, static_cast<int>(col + 16u * (col / 4u)));
    const float tok_norm = __fsqrt_rn(tsq) * (1.0f + 0x1p-7f);
    const uint32_t c = wave * 32 + tb * 16 + col;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint32_t i0 = rb * 8 + 2 * kb;
      const float g0 = acc[rb][tb][0] + acc[rb][tb][1];
      const float g1 = acc[rb][tb][2] + acc[rb][tb][3];
      sh_g[i0][c] = g0;
      sh_g[i0 + 1][c] = g1;
      sh_b[i0][c] = __builtin_fmaf(tok_norm, __builtin_fmaf(f.coef, src_norm[i0], f.coef2), f.slack);
      sh_b[i0 + 1][c] =
          __builtin_fmaf(tok_norm, __builtin_fmaf(f.coef, src_norm[i0 + 1], f.coef2), f.slack);
    }
  }
  __syncthreads();
  write_fallback_records(f, sh_g, sh_b, src_row, m0, tile, tiles);
}

} // namespace

uint32_t fallback_tiles(uint32_t vocab) {
  return (vocab + kTileTokens - 1) / kTileTokens;
}

hipError_t launch_projection(const ProjArgs& args, hipStream_t stream) {
  if (args.H % kKC != 0) return hipErrorInvalidValue;
  const dim3 grid(fallback_tiles(args.V), (args.m + kMTile - 1) / kMTile);
  if (args.a16 != nullptr) {
    hipLaunchKernelGGL((projection_kernel<ASrc::kF16>), grid, dim3(kThreads), 0, stream, args);
  } else {
    hipLaunchKernelGGL((projection_kernel<ASrc::kF32Split>), grid, dim3(kThreads), 0, stream, args);
  }
  return hipGetLastError();
}

hipError_t launch_fallback(const FallbackArgs& args, hipStream_t stream) {
  if (args.m == 0) return hipSuccess;
  if (args.H % kKC != 0) return hipErrorInvalidValue;
  const dim3 grid(fallback_tiles(args.V), (args.m + kMTile - 1) / kMTile);
  constexpr uint32_t kEpiBytes = 2u * kMTile * kTileTokens * 4u;
  const uint32_t stage = a_stage_bytes(args.H);
  const uint32_t steps = args.H / 32;  // even (H % 64 == 0)
  if (stage <= kAStageMaxBytes) {
    const uint32_t lds = stage > kEpiBytes ? stage : kEpiBytes;
    if (steps % 9 == 0) {
      hipLaunchKernelGGL((fallback_direct_kernel<true, 9>), grid, dim3(kThreads), lds, stream, args);
    } else if (steps % 8 == 0) {
      hipLaunchKernelGGL((fallback_direct_kernel<true, 8>), grid, dim3(kThreads), lds, stream, args);
    } else if (steps % 6 == 0) {
      hipLaunchKernelGGL((fallback_direct_kernel<true, 6>), grid, dim3(kThreads), lds, stream, args);
    } else if (steps % 4 == 0) {
      hipLaunchKernelGGL((fallback_direct_kernel<true, 4>), grid, dim3(kThreads), lds, stream, args);
    } else {
      hipLaunchKernelGGL((fallback_direct_kernel<true, 2>), grid, dim3(kThreads), lds, stream, args);
    }
  } else {
    hipLaunchKernelGGL((fallback_direct_kernel<false, kDirectKC>), grid, dim3(kThreads),
                       kEpiBytes, stream, args);
  }
  return hipGetLastError();
}

} // namespace mf
