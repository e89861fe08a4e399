// The MFMA head's tile pieces shared by the head kernels (mf_mfma.hip) and
// the table pass (mf_pass.hip): slot metadata of a panel tile, the per-tile
// accumulators and the windowed-argmax epilogue that turns a tile's scores
// into window records.
#pragma once

#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// ---- MFMA head of the unrestricted rows -----------------------------------
//
// A workgroup owns the 32 slots of one panel tile (an M-tile) and a run of
// 192-token tiles (one window record per row and tile); the runs are sized
// so that every compute unit gets the same number of tiles.  The tile's 12
// blocks of 16 tokens are split over the waves, kBlocks per wave; each block
// is one v_mfma_f32_16x16x32_f16 column block against the 32 slots as four
// 16-row A blocks: A rows 2j and 2j + 1 of block rb are the hi and lo halves
// of slot 8 rb + j.  In the 16x16x32 layout lane l holds 8 consecutive
// features of column / A row l % 16 at k-block l / 16, so the four lanes of
// a token read 64 contiguous bytes per step, and table rows go straight from
// memory into the MFMA registers.  A second MFMA of each token block with
// itself gives the squared token norms (Gram diagonal) for the error bound.
//
// Two variants:
//   narrow rows (panel tile in LDS, H <= 576): at entry the workgroup copies
//     its panel tile into LDS with 1 KiB global-to-LDS bursts and every wave
//     issues the loads of its whole K range; one wait, one barrier, then the
//     MFMAs.  Each tile costs one memory round trip.
//   wide rows: A and B from memory (A from L2) in units of KC steps, two
//     units in flight.

typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kHeadTileBlocks = kHeadTileTokens / 16;
// narrow-row variant: waves per workgroup (tile blocks per wave = 12 / waves)
constexpr int kHeadLdsWaves = 4;
// wide-row variant: 4 waves x 3 blocks
constexpr int kWideWaves = 4;
constexpr int kWideBlocks = 3;

// The tile's scores [slot][token] and token norm bounds, staged in LDS for
// the epilogue (rows padded so the four slot rows one write instruction
// touches fall on different banks).
constexpr uint32_t kEpiStride = kHeadTileTokens + 8;
constexpr int kEpiWaves = 4;  // both variants run four waves
struct HeadEpi {
  float g[kPanelRows][kEpiStride];
  float tn[kEpiWaves];             // per-wave token-norm maxima
  uint32_t count[kEpiWaves][64];   // per-lane member counts
};

template <int kBlocks>
struct HeadAcc {
  floatx4 acc[4][kBlocks];
  floatx4 gram[kBlocks];
};

// Slot metadata of the workgroup's panel tile: source row (kInvalidToken
// for slots past m or without a row) and norm bound; block column 0 also
// records row -> slot for the finalize kernel.  Straight-line loads.
__device__ __forceinline__ void head_slots(const FallbackArgs& f, uint32_t m0,
                                           uint32_t* src_row, float* src_norm,
                                           float* src_slack) {
  if (threadIdx.x < kPanelRows) {
    const uint32_t i = m0 + threadIdx.x;
    const uint32_t at = i < f.m ? i : f.m - 1u;
    const uint32_t row = f.slot_row[at];
    const float norm = f.slot_norm[at];
    const float slack = f.slot_slack[at];
    const uint32_t r = i < f.m ? row : kInvalidToken;
    src_row[threadIdx.x] = r;
    src_norm[threadIdx.x] = r != kInvalidToken ? norm : 0.0f;
    src_slack[threadIdx.x] = r != kInvalidToken ? slack : 0.0f;
    if (blockIdx.x == 0 && r != kInvalidToken && f.fb_map != nullptr) f.fb_map[r] = i;
  }
}

// head_slots in two halves, for a caller that issues the loads early and
// stores the slots once they have landed: a thread's slot (threads below
// kPanelRows), loaded from clamped positions without a branch.  With no
// slots (m == 0) the loads read entry 0 of `dummy`, a valid array of at
// least one word the caller names.
struct HeadSlotLoad {
  uint32_t row;
  float norm;
  float slack;
};
__device__ __forceinline__ HeadSlotLoad head_slot_load(const FallbackArgs& f, uint32_t m0,
                                                       const float* dummy) {
  const uint32_t t = threadIdx.x < kPanelRows ? threadIdx.x : 0u;
  const uint32_t i = m0 + t;
  const uint32_t at = f.m == 0u ? 0u : (i < f.m ? i : f.m - 1u);
  const uint32_t* rows = f.m > 0u ? f.slot_row : reinterpret_cast<const uint32_t*>(dummy);
  const float* norms = f.m > 0u ? f.slot_norm : dummy;
  const float* slacks = f.m > 0u ? f.slot_slack : dummy;
  return HeadSlotLoad{rows[at], norms[at], slacks[at]};
}
__device__ __forceinline__ void head_slot_store(const FallbackArgs& f, uint32_t m0,
                                                const HeadSlotLoad& v, uint32_t* src_row,
                                                float* src_norm, float* src_slack) {
  if (threadIdx.x < kPanelRows) {
    const uint32_t i = m0 + threadIdx.x;
    const uint32_t r = i < f.m ? v.row : kInvalidToken;
    src_row[threadIdx.x] = r;
    src_norm[threadIdx.x] = r != kInvalidToken ? v.norm : 0.0f;
    src_slack[threadIdx.x] = r != kInvalidToken ? v.slack : 0.0f;
    if (blockIdx.x == 0 && r != kInvalidToken && f.fb_map != nullptr) f.fb_map[r] = i;
  }
}

// 8-lane max (lanes 8 s .. 8 s + 7): quad_perm xor 1 and xor 2, then the
// mirror inside the half row.  v_max_f32 with the DPP operand directly (the
// compiler's form adds a canonicalizing max per step); s_nop 1 is the
// VALU-write to DPP-read wait.
__device__ __forceinline__ float lane8_max(float v) {
  asm("s_nop 1\n\tv_max_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf"
      : "+v"(v));
  asm("s_nop 1\n\tv_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf"
      : "+v"(v));
  asm("s_nop 1\n\tv_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf"
      : "+v"(v));
  return v;
}

// The tile's window records.  Lane l holds D[4 (l / 16) + i][l % 16] of
// each block: A rows 2j, 2j + 1 (hi, lo of slot 8 rb + j) for j = 2 kb and
// 2 kb + 1, so the score of slot 8 rb + 2 kb + jj (jj = 0, 1) and token
// (wave kBlocks + tb) 16 + col of the tile is acc[rb][tb][2 jj] +
// acc[rb][tb][2 jj + 1]; the Gram diagonal of column c sits in lane
// c + 16 (c / 4), element c % 4.
//
// One bound per slot and tile: b = tn_max (coef ||z|| + coef2) + slack with
// tn_max the largest token-norm bound of the tile, which is at least every
// token's own bound.  Then the best lower bound is L = fl(max g - b) (the
// rounding is monotone) and a token is a member when fl(g + b) >= L.  The
// scores go through LDS; then lanes 8 s .. 8 s + 7 of wave w take slot
// 8 w + s, 24 consecutive tokens each, so the eight slots of a wave share
// every instruction; members come out in ascending token order.  Ends with
// a barrier (LDS is reused by the next tile).
//
// kHiOnly: A rows are the slots' FP16 hi alone, A row j of block rb being
// slot 16 rb + j (blocks rb = 0, 1), so the score of slot 16 rb + 4 kb + i
// is acc[rb][tb][i].
template <int kWaves, int kBlocks, bool kHiOnly = false>
__device__ __forceinline__ void head_records(const FallbackArgs& f, const HeadAcc<kBlocks>& h,
                                             HeadEpi& epi, const uint32_t* src_row,
                                             const float* src_norm, const float* src_slack,
                                             uint32_t m0, uint32_t tile,
                                             uint32_t tiles) {
  static_assert(kWaves == kEpiWaves && kPanelRows == 8 * kWaves, "eight slots per wave");
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t wave = threadIdx.x / 64;
  const uint32_t col = lane % 16;
  const uint32_t kb = lane / 16;
  const uint32_t wtok = wave * (16u * kBlocks);
  const uint32_t tok0 = tile * kHeadTileTokens;
  const uint32_t nt = f.V - tok0 < kHeadTileTokens ? f.V - tok0 : kHeadTileTokens;
  float tn_local = 0.0f;
#pragma unroll
  for (int tb = 0; tb < kBlocks; ++tb) {
    const uint32_t t = wtok + tb * 16u + col;
    const uint32_t e = col % 4u;
    const float d = e == 0u ? h.gram[tb][0]
                            : (e == 1u ? h.gram[tb][1] : (e == 2u ? h.gram[tb][2] : h.gram[tb][3]));
    // lanes of the Gram diagonal, tokens of the vocabulary
    if (col / 4u == kb && t < nt) tn_local = __builtin_fmaxf(tn_local, __fsqrt_rn(d) * (1.0f + 0x1p-7f));
    if constexpr (kHiOnly) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) epi.g[rb * 16 + 4 * kb + i][t] = h.acc[rb][tb][i];
      }
    } else {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          epi.g[rb * 8 + 2 * kb + jj][t] = h.acc[rb][tb][2 * jj] + h.acc[rb][tb][2 * jj + 1];
        }
      }
    }
  }
  // a NaN norm (a non-finite table row) propagates: the bound then fails the
  // finiteness test and the tile is rescored in full
  const bool any_nan = __ballot(tn_local != tn_local) != 0ull;
  const float tn_wave = wave_max(tn_local);
  if (lane == 0) epi.tn[wave] = any_nan ? __builtin_nanf("") : tn_wave;
  __syncthreads();
  float tn_max = epi.tn[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    const float v = epi.tn[w];
    tn_max = (tn_max != tn_max || v != v) ? __builtin_nanf("") : __builtin_fmaxf(tn_max, v);
  }

  constexpr int kSeg = kHeadTileTokens / 8;  // tokens per lane
  const uint32_t sl = lane / 8;              // slot of the wave
  const uint32_t j8 = lane % 8;
  const uint32_t i = wave * 8u + sl;
  const uint32_t t0 = j8 * kSeg;
  float gv[kSeg];
  const float4* src = reinterpret_cast<const float4*>(&epi.g[i][t0]);
#pragma unroll
  for (int q = 0; q < kSeg / 4; ++q) {
    const float4 v = src[q];
    gv[4 * q] = v.x;
    gv[4 * q + 1] = v.y;
    gv[4 * q + 2] = v.z;
    gv[4 * q + 3] = v.w;
  }
  // tokens past the vocabulary (last tile only) read as -inf / 0
  if (nt < kHeadTileTokens) {
#pragma unroll
    for (int k = 0; k < kSeg; ++k) {
      if (t0 + k >= nt) gv[k] = -__builtin_huge_valf();
    }
  }
  float gm = gv[0];
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < kSeg; ++k) {
    gm = __builtin_fmaxf(gm, gv[k]);
    sum += (t0 + k < nt) ? gv[k] : 0.0f;
  }
  // every score of the lane finite (a sum that overflows counts as not
  // finite: the tile is then rescored in full, which is exact too)
  const uint64_t fin_lanes = __ballot(__builtin_isfinite(sum));
  const bool slot_finite = ((fin_lanes >> (8u * sl)) & 0xFFull) == 0xFFull;
  const float G = lane8_max(gm);
  const float bs = __builtin_fmaf(tn_max, __builtin_fmaf(f.coef, src_norm[i], f.coef2), src_slack[i]);
  const float L = G - bs;
  uint32_t members = 0u;  // bit k: token t0 + k
#pragma unroll
  for (int k = 0; k < kSeg; ++k) members |= (gv[k] + bs >= L) ? (1u << k) : 0u;
  const uint32_t n = static_cast<uint32_t>(__popc(members));
  epi.count[wave][lane] = n;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint4 c0 = *reinterpret_cast<const uint4*>(&epi.count[wave][8u * sl]);
  const uint4 c1 = *reinterpret_cast<const uint4*>(&epi.count[wave][8u * sl + 4u]);
  const uint32_t cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  uint32_t before = 0u;
  uint32_t total = 0u;
#pragma unroll
  for (uint32_t q = 0; q < 8; ++q) {
    before += q < j8 ? cs[q] : 0u;
    total += cs[q];
  }
  if (src_row[i] != kInvalidToken) {
    const bool ordinary = slot_finite && bs < 0x1p100f && total <= static_cast<uint32_t>(kTileMembers);
    TileRecord* rec = f.records + static_cast<uint64_t>(m0 + i) * tiles + tile;
    if (ordinary) {
      // the lane's members in ascending order, their scores read back
      uint32_t r = before;
      while (members != 0u) {
        const uint32_t k = static_cast<uint32_t>(__builtin_ctz(members));
        members &= members - 1u;
        const float gk = epi.g[i][t0 + k];
        const uint32_t token = tok0 + t0 + k;
        rec->m[r] = TileMember{token, token, gk - bs, gk + bs};
        ++r;
      }
    }
    if (j8 == 0u) {
      const bool finite = slot_finite && bs < 0x1p100f;
      rec->best_lower = L;
      rec->flags = ordinary ? 0u : (finite ? kTileRescoreAll | kTileCrowded : kTileRescoreAll);
      rec->upper_max = G + bs;
      rec->min_token = tok0;
      rec->min_pos = tok0;
      rec->begin = tok0;
      rec->count = nt;
      rec->n_members = ordinary ? total : 0u;
    }
  }
  __syncthreads();
}

}  // namespace
}  // namespace mf
