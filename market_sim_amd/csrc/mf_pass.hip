// The table pass: the restricted and unrestricted stages of
// mf_decode_tail_f16 in one launch that reads every table row once, when the
// state lists are ascending (MF_TAIL_SORTED_LISTS).
//
// A workgroup owns a run of 192-token tiles of the vocabulary.  Per tile its
// four waves load the tile's 12 blocks of 16 table rows into MFMA B
// registers, three blocks per wave, the whole K range in flight, and use them
// for both kinds of rows:
//
//   restricted rows    every candidate id of a row that falls in the tile:
//                      the norm kernel's range index gives, per row, the span
//                      of its ascending list inside the tile, so the tile's
//                      candidates are found without a search.  The FP16 hi of
//                      z (x * w, the normalized row up to its positive factor)
//                      of every row with candidates in the tile is staged in
//                      LDS with global-to-LDS copies issued before the table
//                      rows, so it has landed when they have.  Candidates are
//                      bucketed by 16-token block; 16 at a time go through
//                      v_mfma_f32_16x16x32_f16 with A = the candidates' rows
//                      (one A row per candidate, from LDS) and B = the
//                      block's table rows, and candidate i's score is
//                      D[i][its column].  Each (row, tile) with candidates
//                      gets one window record (best lower bound, <= 4
//                      members, or "rescore all"), the format the finalize
//                      kernel merges.
//   unrestricted rows  the head's dense product against the FP16 hi of their
//                      z (the norm kernel's panel, hi rows staged in LDS),
//                      one window record per row and tile (mf_head.hpp).
//
// Scores use hi = rne_f16(z) alone: |z - hi| <= 2^-11 |z| (+ 2^-25 below the
// FP16 normal range), which the bound carries (mf_abi.cpp pass_bound_coefs).
// The Gram diagonal of each block (an MFMA of the block with itself) gives
// the token norms of the bounds.  Rows with more candidates in a tile than
// the LDS holds are taken in batches of whole rows.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_head.hpp"
#include "mf_launch.hpp"
#include "mf_plan.hpp"

namespace mf {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kBlocks = 3;  // token blocks per wave
static_assert(kWaves * kBlocks == static_cast<int>(kHeadTileBlocks), "tile of 12 blocks");
static_assert(kPassRowsMax == static_cast<uint32_t>(kThreads), "one plan row per thread");
// Candidates scored per batch (whole rows; a row has at most 192 in a tile).
constexpr uint32_t kPairBatch = 512;
// Bucket entries: every block's bucket padded to whole groups of 16.
constexpr uint32_t kBucketSlots = kPairBatch + kHeadTileBlocks * 16u;
constexpr uint16_t kNoPair = 0xFFFFu;
// Dynamic LDS of the workgroup (one per compute unit), and the slack after
// the staging area that a wave's last 1 KiB copy may run into.
constexpr uint32_t kLdsBudget = 160u * 1024u - 1024u;
constexpr uint32_t kCopySlack = 1024u;

// One candidate in its block's bucket: where its row is staged, which
// candidate of the batch it is, its column in the block and its row's bound
// terms, so that scoring a group of 16 needs one LDS read per lane.
struct alignas(16) PairEntry {
  uint32_t a_off;  // byte offset of the staged row in the staging area
  uint32_t kc;     // candidate index (bits 0..15, kNoPair: empty) | column << 16 | row << 20
  float f1;        // coef * ||z|| + coef2 of the row
  float f2;        // the row's absolute error term
};
static_assert(kPassRowsMax <= 4096u, "row index in 12 bits");

// Float bits with the float order as unsigned integers (for LDS atomicMax).
__device__ __forceinline__ uint32_t order_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_order_bits(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

struct PassShared {
  TilePlan<kThreads, kPassRowsMax> plan;  // per row: list index of its first id in the tile
  uint32_t lo[kPassRowsMax];              // list position of that id
  uint32_t rec[kPassRowsMax];             // record index of (row, tile)
  uint32_t rprefix[kPassRowsMax + 1];     // rows with candidates before row r
  uint32_t slot_row[kPassRowsMax];        // staged slot -> row (batch)
  float rf1[kPassRowsMax];                // coef * ||z|| + coef2, absolute error term
  float rf2[kPassRowsMax];
  uint32_t ptok[kPairBatch];              // candidate k of the batch: id, row, g + b
  uint16_t prow[kPairBatch];
  float pupper[kPairBatch];               // (+inf: not scored)
  uint32_t row_lower[kPassRowsMax];       // per row: max of g - b, order-preserving bits
  uint32_t row_upper[kPassRowsMax];       // per row: max of g + b, order-preserving bits
  uint32_t row_all[kPassRowsMax];         // per row: a candidate needs the exact rescore
  uint32_t row_members[kPassRowsMax];     // per row: candidates with g + b >= the row's lower bound
  PairEntry bent[kBucketSlots];
  uint32_t bcount[kHeadTileBlocks];
  uint32_t bfill[kHeadTileBlocks];
  uint32_t bstart[kHeadTileBlocks + 1];   // padded bucket starts (multiples of 16)
  uint32_t wave_sum[kWaves];
  float tn[kHeadTileTokens];              // token norm bounds of the tile
};

// LDS image of one FP16 row of z (or of a panel slot's hi row): H halves and
// a 16-byte pad, the panel's own row format; the 1168-byte stride at
// H = 576 puts the 16 rows of one A read on distinct banks.
__host__ __device__ constexpr uint32_t slot_bytes(uint32_t H) { return 2u * (H + kPanelPad); }

// Layout: [PassShared][staging area].  The staging area holds the rows of
// z while candidates are scored, then the hi rows of a panel tile followed
// by the head's epilogue scratch (HeadEpi).  The panel part is rounded up to
// whole 1 KiB copies so that its last copy stays inside it.
__host__ __device__ constexpr uint32_t panel_part(uint32_t H) {
  return (kPanelRows * slot_bytes(H) + 1023u) / 1024u * 1024u;
}
__host__ __device__ constexpr uint32_t stage_slots(uint32_t H) {
  const uint32_t room = kLdsBudget - static_cast<uint32_t>(sizeof(PassShared)) - kCopySlack;
  const uint32_t n = room / slot_bytes(H);
  return n < kPassRowsMax ? n : kPassRowsMax;
}
__host__ __device__ constexpr uint32_t pass_lds_bytes(uint32_t H) {
  const uint32_t rows = stage_slots(H) * slot_bytes(H);
  const uint32_t head = panel_part(H) + static_cast<uint32_t>(sizeof(HeadEpi));
  return static_cast<uint32_t>(sizeof(PassShared)) + (rows > head ? rows : head) + kCopySlack;
}
static_assert(stage_slots(576) >= 96 && pass_lds_bytes(576) <= kLdsBudget,
              "the pass fits one workgroup per CU at H = 576");

// Largest r1 in [r0, rows] with v[r1] - v[r0] <= limit (v nondecreasing).
__device__ __forceinline__ uint32_t last_within(const uint32_t* v, uint32_t rows, uint32_t r0,
                                                uint32_t limit) {
  uint32_t lo = r0, hi = rows;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) / 2;
    if (v[mid] - v[r0] <= limit) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Copies `n` FP16 rows of H halves into LDS slots (slot_bytes(H) each),
// wave w taking the 1 KiB copies w, w + 4, ...: piece q of the area is 16
// bytes of slot q / per at offset q % per; src(i) is slot i's row.  The pad
// piece and the lanes past the last piece read piece 0 of a staged row.
template <uint32_t H, typename Src>
__device__ __forceinline__ void stage_rows(unsigned char* area, uint32_t n, Src src) {
  constexpr uint32_t per = slot_bytes(H) / 16u;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t pieces = n * per;
  for (uint32_t c = wave; c * kWave < pieces; c += kWaves) {
    const uint32_t q = c * kWave + lane;
    const uint32_t i = q < pieces ? q / per : 0u;
    const uint32_t pp = q < pieces ? q % per : 0u;
    burst_to_lds(src(i) + (pp < per - 1u ? pp : 0u) * 8u, area + c * kWave * 16u);
  }
}

// One group of 16 candidates: its bucket entries (lane l < 16 holds
// candidate l's) and A rows from the staged slots.
template <int kSteps>
struct Group {
  PairEntry e;
  half8_t a[kSteps];
};

template <int kSteps>
__global__ __launch_bounds__(kThreads) void pass_kernel(PassArgs p) {
  constexpr uint32_t H = 32u * kSteps;
  constexpr uint32_t kSlot = slot_bytes(H);
  constexpr uint32_t kTileHalves = static_cast<uint32_t>(panel_tile_bytes(H) / 2u);
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t src_row[kPanelRows];
  __shared__ float src_norm[kPanelRows];
  __shared__ float src_slack[kPanelRows];
  const FallbackArgs& f = p.head;
  const uint32_t panels = f.m > 0 ? panel_tiles(f.m) : 0u;
  PassShared& ps = *reinterpret_cast<PassShared*>(dyn);
  unsigned char* stage = dyn + sizeof(PassShared);
  // after the candidates: a panel tile's hi rows, then the head's epilogue
  unsigned char* panel = stage;
  HeadEpi& epi = *reinterpret_cast<HeadEpi*>(stage + panel_part(H));
  const uint32_t slots = stage_slots(H);
  const uint32_t tiles = p.ranges;
  const uint32_t t_begin = blockIdx.x * f.tiles_per_group;
  const uint32_t t_end = t_begin + f.tiles_per_group < tiles ? t_begin + f.tiles_per_group : tiles;
  const uint32_t rows = p.rows;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  const uint32_t col = lane % 16;
  const uint32_t kb = lane / 16;

  half8_t bt[kBlocks][kSteps];
  auto load_tile = [&](uint32_t t) {
#pragma unroll
    for (int tb = 0; tb < kBlocks; ++tb) {
      const uint32_t token = t * kHeadTileTokens + (wave * kBlocks + tb) * 16u + col;
      const uint16_t* src = f.emb + static_cast<uint64_t>(token < f.V ? token : 0u) * H + kb * 8u;
#pragma unroll
      for (int s = 0; s < kSteps; ++s) bt[tb][s] = *reinterpret_cast<const half8_t*>(src + s * 32);
    }
  };
  // the hi rows of panel tile pt (slot j's hi row leads its [hi | lo] pair)
  auto stage_panel = [&](uint32_t pt) {
    const uint16_t* base = f.panel + static_cast<uint64_t>(pt) * kTileHalves;
    stage_rows<H>(panel, kPanelRows, [&](uint32_t j) { return base + j * 2u * (H + kPanelPad); });
  };

  for (uint32_t tile = t_begin; tile < t_end; ++tile) {
    const uint32_t t0 = tile * kHeadTileTokens;
    // (1) the tile's candidates: per row (one per thread) the span [lo, hi)
    // of its list (range index of the norm kernel, range-major).
    const uint32_t ri = tid < rows ? tid : 0u;
    const RowMeta m = p.row_meta[ri];
    const uint32_t rt = p.row_tiles[ri];
    const uint4 ix = p.range_index[static_cast<uint64_t>(tile) * rows + ri];
    const uint32_t lo_r = ix.x;
    const uint32_t hi_r = ix.y;
    const uint32_t rec_r = ix.z;
    const float norm_r = p.row_norm[ri];
    const float slack_r = p.row_slack[ri];
    {
      const bool use = tid < rows && (m.kind & kRowRestricted) && !(rt & kRangesUnused) &&
                       hi_r > lo_r && hi_r <= m.count && rec_r < p.max_recs;
      const uint32_t n = use ? hi_r - lo_r : 0u;
      const uint32_t has = n > 0u ? 1u : 0u;
      if (tid < rows) {
        ps.plan.begin[tid] = m.list_begin + lo_r;
        ps.plan.count[tid] = n;
        ps.lo[tid] = lo_r;
        ps.rec[tid] = rec_r;
        ps.rf1[tid] = __builtin_fmaf(p.coef, norm_r, p.coef2);
        ps.rf2[tid] = slack_r;
      }
      // exclusive scans over the rows: candidates and rows with candidates
      uint32_t in_n = n;
      uint32_t in_h = has;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t on = static_cast<uint32_t>(__shfl_up(static_cast<int>(in_n), d));
        const uint32_t oh = static_cast<uint32_t>(__shfl_up(static_cast<int>(in_h), d));
        if (static_cast<int>(lane) >= d) {
          in_n += on;
          in_h += oh;
        }
      }
      if (lane == kWave - 1) {
        ps.plan.wave_total[wave] = in_n;
        ps.wave_sum[wave] = in_h;
      }
      __syncthreads();
      uint32_t bn = in_n - n;
      uint32_t bh = in_h - has;
      for (uint32_t w = 0; w < wave; ++w) {
        bn += ps.plan.wave_total[w];
        bh += ps.wave_sum[w];
      }
      if (tid <= rows) {  // tid == rows: the totals
        ps.plan.prefix[tid] = bn;
        ps.rprefix[tid] = bh;
      }
      if (tid == kThreads - 1 && rows == kPassRowsMax) {
        ps.plan.prefix[rows] = bn + n;
        ps.rprefix[rows] = bh + has;
      }
      __syncthreads();
    }

    // (2) per batch of whole rows: stage, ids, buckets, scores, records.
    // The first batch's staging and ids are issued before the table rows.
    uint32_t r0 = 0u;
    bool first = true;
    while (first || r0 < rows) {
      const uint32_t r1a = last_within(ps.plan.prefix, rows, r0, kPairBatch);
      const uint32_t r1b = last_within(ps.rprefix, rows, r0, slots);
      const uint32_t r1 = r1a < r1b ? r1a : r1b;
      const uint32_t k0 = ps.plan.prefix[r0];
      const uint32_t nb = ps.plan.prefix[r1] - k0;
      const uint32_t s0 = ps.rprefix[r0];
      const uint32_t nz = ps.rprefix[r1] - s0;
      if (tid < kHeadTileBlocks) {
        ps.bcount[tid] = 0u;
        ps.bfill[tid] = 0u;
      }
      if (tid >= r0 && tid < r1 && ps.plan.count[tid] > 0u) ps.slot_row[ps.rprefix[tid] - s0] = tid;
      if (tid < rows) {
        ps.row_lower[tid] = order_bits(-__builtin_huge_valf());
        ps.row_upper[tid] = order_bits(-__builtin_huge_valf());
        ps.row_all[tid] = 0u;
        ps.row_members[tid] = 0u;
      }
      __syncthreads();  // slot rows, cleared counters
      uint32_t tok[2] = {0u, 0u};
      uint32_t row[2] = {0u, 0u};
      if (nb > 0u) {
        // lanes past the batch load candidate k0 again (a valid list
        // position) instead of branching around their loads
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint32_t k = k0 + tid + u * kThreads;
          const uint32_t kk = k < k0 + nb ? k : k0;
          row[u] = plan_row_of(ps.plan, rows, kk);
          tok[u] = p.tokens[ps.plan.begin[row[u]] + (kk - ps.plan.prefix[row[u]])];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      stage_rows<H>(stage, nz, [&](uint32_t i) { return p.z_hi + static_cast<uint64_t>(ps.slot_row[i]) * H; });
      __builtin_amdgcn_sched_barrier(0);
      if (first) load_tile(tile);
      __builtin_amdgcn_sched_barrier(0);
      if (first && panels == 1u && tile == t_begin) head_slots(f, 0u, src_row, src_norm, src_slack);
      __builtin_amdgcn_sched_barrier(0);
      uint32_t blk[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t k = k0 + tid + u * kThreads;
        const uint32_t c = tok[u] - t0;
        blk[u] = (k < k0 + nb && c < kHeadTileTokens) ? c / 16u : kHeadTileBlocks;
        if (k < k0 + nb) {
          ps.ptok[k - k0] = tok[u];
          ps.prow[k - k0] = static_cast<uint16_t>(row[u]);
          ps.pupper[k - k0] = __builtin_huge_valf();
          if (blk[u] < kHeadTileBlocks) {
            atomicAdd(&ps.bcount[blk[u]], 1u);
          } else {
            ps.row_all[row[u]] = 1u;  // an id outside the tile: rescore the record in full
          }
        }
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t run = 0u;
        for (uint32_t b = 0; b < kHeadTileBlocks; ++b) {
          ps.bstart[b] = run;
          run += (ps.bcount[b] + 15u) & ~15u;
        }
        ps.bstart[kHeadTileBlocks] = run;
      }
      for (uint32_t e = tid; e < kBucketSlots; e += kThreads) {
        ps.bent[e] = PairEntry{0u, static_cast<uint32_t>(kNoPair), 0.0f, 0.0f};
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (blk[u] < kHeadTileBlocks) {
          const uint32_t at = ps.bstart[blk[u]] + atomicAdd(&ps.bfill[blk[u]], 1u);
          const uint32_t r = row[u];
          ps.bent[at] = PairEntry{(ps.rprefix[r] - s0) * kSlot,
                                  (tid + u * kThreads) | (((tok[u] - t0) % 16u) << 16) | (r << 20),
                                  ps.rf1[r], ps.rf2[r]};
        }
      }
      wait_vector_memory();  // table rows (first batch), staged rows
      floatx4 gram[kBlocks];
      if (first) {
        // Gram diagonal: token norm bounds of the tile
#pragma unroll
        for (int tb = 0; tb < kBlocks; ++tb) {
          gram[tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int s = 0; s < kSteps; ++s) {
            gram[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bt[tb][s], bt[tb][s], gram[tb], 0, 0, 0);
          }
          const uint32_t e = col % 4u;
          const float d = e == 0u ? gram[tb][0]
                                  : (e == 1u ? gram[tb][1] : (e == 2u ? gram[tb][2] : gram[tb][3]));
          if (col / 4u == kb) ps.tn[(wave * kBlocks + tb) * 16u + col] = __fsqrt_rn(d) * (1.0f + 0x1p-7f);
        }
      }
      __syncthreads();  // buckets, staged rows and token norms visible

      // (3) this wave's groups: its three blocks' buckets, 16 candidates
      // per group, two accumulators per group (even and odd steps)
      const uint32_t qb = __builtin_amdgcn_readfirstlane(ps.bstart[wave * kBlocks] / 16u);
      const uint32_t q1 = __builtin_amdgcn_readfirstlane(ps.bstart[wave * kBlocks + 1] / 16u) - qb;
      const uint32_t q2 = __builtin_amdgcn_readfirstlane(ps.bstart[wave * kBlocks + 2] / 16u) - qb;
      const uint32_t nq = __builtin_amdgcn_readfirstlane(ps.bstart[wave * kBlocks + 3] / 16u) - qb;
      auto load_group = [&](uint32_t q, Group<kSteps>& g) {
        g.e = ps.bent[(qb + (q < nq ? q : 0u)) * 16u + col];
        const unsigned char* src = stage + g.e.a_off + kb * 16u;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) g.a[s] = *reinterpret_cast<const half8_t*>(src + s * 64);
      };
      auto score_group = [&](uint32_t q, const Group<kSteps>& g) {
        floatx4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
        floatx4 acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
        auto chain = [&](const half8_t(&b)[kSteps]) {
#pragma unroll
          for (int s = 0; s < kSteps; s += 2) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(g.a[s], b[s], acc0, 0, 0, 0);
            if (s + 1 < kSteps) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(g.a[s + 1], b[s + 1], acc1, 0, 0, 0);
          }
        };
        if (q < q1) chain(bt[0]); else if (q < q2) chain(bt[1]); else chain(bt[2]);
        const floatx4 acc = acc0 + acc1;
        // candidate i = lane (lanes 0..15): D[i][c] sits in lane
        // 16 (i / 4) + c, element i % 4
        const uint32_t k = g.e.kc & 0xFFFFu;
        const uint32_t c = (g.e.kc >> 16) & 15u;
        const uint32_t r = g.e.kc >> 20;
        const bool mine = lane < 16u && k != kNoPair;
        const int src = lane < 16u ? static_cast<int>(16u * (lane / 4u) + c) : static_cast<int>(lane);
        const float v0 = __shfl(acc[0], src);
        const float v1 = __shfl(acc[1], src);
        const float v2 = __shfl(acc[2], src);
        const float v3 = __shfl(acc[3], src);
        const uint32_t blk = q < q1 ? 0u : (q < q2 ? 1u : 2u);
        const float tnv = ps.tn[(wave * kBlocks + blk) * 16u + c];
        if (mine) {
          const uint32_t e = lane % 4u;
          const float gs = e == 0u ? v0 : (e == 1u ? v1 : (e == 2u ? v2 : v3));
          const float b = __builtin_fmaf(tnv, g.e.f1, g.e.f2);
          const bool ok = __builtin_isfinite(gs) && __builtin_isfinite(b) && b < 0x1p100f;
          if (ok) {
            atomicMax(&ps.row_lower[r], order_bits(gs - b));
            atomicMax(&ps.row_upper[r], order_bits(gs + b));
            ps.pupper[k] = gs + b;
          } else {
            ps.row_all[r] = 1u;
          }
        }
      };
      // one group at a time: its LDS reads complete in order, so each MFMA
      // waits only for its own operand (a second group in flight costs
      // register spills)
      for (uint32_t q = 0; q < nq; ++q) {
        Group<kSteps> g;
        load_group(q, g);
        score_group(q, g);
      }
      __syncthreads();  // every candidate scored; the staging area is free
      // the first panel tile's hi rows land while the records are written
      if (first && panels > 0u) stage_panel(0u);

      // (4) one window record per (row, tile).  The best lower bound came
      // from the scoring; each candidate then checks itself against its
      // row's (members in any order: the finalize only collects them), and
      // one thread per row writes the header.  The list is ascending, so a
      // row's lowest id here is its first.
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t kk = tid + u * kThreads;
        if (kk < nb) {
          const uint32_t r = ps.prow[kk];
          const float up = ps.pupper[kk];
          if (ps.row_all[r] == 0u && up >= from_order_bits(ps.row_lower[r])) {
            const uint32_t i = atomicAdd(&ps.row_members[r], 1u);
            if (i < static_cast<uint32_t>(kTileMembers)) {
              const uint32_t j = k0 + kk - ps.plan.prefix[r];
              TileRecord* rec = p.records + static_cast<uint64_t>(r) * p.max_recs + ps.rec[r];
              // g - b of a member is only used against the row's window
              rec->m[i] = TileMember{ps.ptok[kk], ps.lo[r] + j, -__builtin_huge_valf(), up};
            }
          }
        }
      }
      __syncthreads();
      for (uint32_t r = r0 + tid; r < r1; r += kThreads) {
        const uint32_t n = ps.plan.count[r];
        if (n == 0u) continue;
        const uint32_t members = ps.row_members[r];
        const bool ordinary = ps.row_all[r] == 0u && members <= static_cast<uint32_t>(kTileMembers);
        TileRecord* rec = p.records + static_cast<uint64_t>(r) * p.max_recs + ps.rec[r];
        const uint32_t lo = ps.lo[r];
        rec->best_lower = from_order_bits(ps.row_lower[r]);
        rec->flags = ordinary ? 0u
                              : (ps.row_all[r] == 0u ? kTileRescoreAll | kTileCrowded : kTileRescoreAll);
        rec->upper_max = from_order_bits(ps.row_upper[r]);
        rec->min_token = ps.ptok[ps.plan.prefix[r] - k0];
        rec->min_pos = lo;
        rec->begin = lo;
        rec->count = n;
        rec->n_members = ordinary ? members : 0u;
      }

      // (5) the unrestricted rows (first batch): the head against the panel
      // tiles' hi rows
      if (first) {
        for (uint32_t pt = 0; pt < panels; ++pt) {
          if (pt > 0u) {
            __syncthreads();  // the previous panel tile's readers are done
            stage_panel(pt);
          }
          if (panels > 1u) head_slots(f, pt * kPanelRows, src_row, src_norm, src_slack);
          wait_vector_memory();
          __syncthreads();
          HeadAcc<kBlocks> h;
#pragma unroll
          for (int tb = 0; tb < kBlocks; ++tb) {
            h.gram[tb] = gram[tb];
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) h.acc[rb][tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
          }
          const unsigned char* a_lane = panel + col * kSlot + kb * 16u;
#pragma unroll
          for (int s = 0; s < kSteps; ++s) {
            half8_t a[2];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) a[rb] = *reinterpret_cast<const half8_t*>(a_lane + rb * 16u * kSlot + s * 64);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
              for (int tb = 0; tb < kBlocks; ++tb) {
                h.acc[rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rb], bt[tb][s], h.acc[rb][tb], 0, 0, 0);
              }
            }
          }
          head_records<kWaves, kBlocks, true>(f, h, epi, src_row, src_norm, src_slack,
                                              pt * kPanelRows, tile, tiles);
        }
      }
      __syncthreads();  // the batch's LDS is free again
      first = false;
      r0 = r1;
      if (nb == 0u) break;
    }
  }
}

template <int kSteps>
void launch_steps(const PassArgs& a, uint32_t groups, hipStream_t stream) {
  const uint32_t lds = pass_lds_bytes(32u * kSteps);
  hipLaunchKernelGGL((pass_kernel<kSteps>), dim3(groups), dim3(kThreads), lds, stream, a);
}

}  // namespace

hipError_t launch_pass(const PassArgs& args, hipStream_t stream) {
  if (args.head.H % 64u != 0 || args.rows == 0 || args.rows > kPassRowsMax ||
      args.ranges != fallback_tiles(args.head.V) ||
      (args.head.m > 0 && args.head.panel == nullptr) ||
      panel_tile_bytes(args.head.H) > kPanelLdsMaxBytes) {
    return hipErrorInvalidValue;
  }
  // runs of tiles per workgroup: as many workgroups as compute units (or
  // tiles), every run the same length
  const uint32_t tiles = args.ranges;
  const uint32_t cus = args.head.groups > 0 ? args.head.groups : 256u;
  PassArgs a = args;
  a.head.tiles_per_group = (tiles + cus - 1) / cus;
  const uint32_t groups = (tiles + a.head.tiles_per_group - 1) / a.head.tiles_per_group;
  switch (args.head.H / 32u) {
    case 2: launch_steps<2>(a, groups, stream); break;
    case 4: launch_steps<4>(a, groups, stream); break;
    case 6: launch_steps<6>(a, groups, stream); break;
    case 8: launch_steps<8>(a, groups, stream); break;
    case 10: launch_steps<10>(a, groups, stream); break;
    case 12: launch_steps<12>(a, groups, stream); break;
    case 14: launch_steps<14>(a, groups, stream); break;
    case 16: launch_steps<16>(a, groups, stream); break;
    case 18: launch_steps<18>(a, groups, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mf
