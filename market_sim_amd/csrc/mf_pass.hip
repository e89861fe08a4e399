// The table pass: the restricted and unrestricted stages of
// mf_decode_tail_f16 in one launch that reads every table row once, when the
// state lists are ascending (MF_TAIL_SORTED_LISTS).
//
// A workgroup owns a run of 192-token tiles of the vocabulary.  Per tile its
// four waves hold the tile's 12 blocks of 16 table rows in MFMA B registers,
// three blocks per wave, and use them for both kinds of rows:
//
//   restricted rows    every candidate id of a row that falls in the tile:
//                      the norm kernel's range index gives, per row, the span
//                      of its ascending list inside the tile, so the tile's
//                      candidates are found without a search.  The FP16 hi of
//                      z (x * w, the normalized row up to its positive factor)
//                      of every row with candidates in the tile is staged in
//                      LDS.  Candidates are bucketed by 16-token block; 16 at a
//                      time go through v_mfma_f32_16x16x32_f16 with A = the
//                      candidates' rows (one A row per candidate, from LDS)
//                      and B = the block's table rows, and candidate i's score
//                      is D[i][its column].  Each (row, tile) with candidates
//                      gets one window record (best lower bound, <= 4
//                      members, or "rescore all"), the format the finalize
//                      kernel merges.
//   unrestricted rows  the head's dense product against the FP16 hi of their
//                      z (the norm kernel's panel, hi rows staged in LDS), one
//                      window record per row and tile (mf_head.hpp).
//
// Timeline of a tile.  The compute unit's vector memory pipeline is the
// bottleneck: loads complete in issue order, and a wave issuing more than
// the pipeline holds stalls until earlier loads drain, so the order of the
// loads is the schedule:
//   1. the plan's per-row values, then the first half of the tile's first
//      block of table rows (it streams while the plan is scanned);
//   2. (plan landed) scans over the rows; each candidate's row; the
//      block's second half; the rows of z to stage (copies straight into
//      LDS) and the candidate ids;
//   3. (all landed) the second block's first half; buckets; its second
//      half; block 0's token norms and candidates; the third block is
//      issued; block 1's, then block 2's candidates, each as its rows land;
//   4. the head's A rows are staged in LDS while the candidates' records
//      are written; the head runs against the three blocks still in
//      registers and writes its records.
// A block's candidates run as a software pipeline (A rows of the next group
// read from LDS while the MFMAs of this one run); candidate scoring is
// bound by LDS bandwidth (one 1152-byte A row per candidate).
// Scores use hi = rne_f16(z) alone: |z - hi| <= 2^-11 |z| (+ 2^-25 below the
// FP16 normal range), which the bound carries (mf_abi.cpp pass_bound_coefs).
// The Gram diagonal of each block (an MFMA of the block with itself) gives
// the token norms of the bounds.  Rows with more candidates in a tile than
// the LDS holds are taken in batches of whole rows; later batches run after
// the first with every block in registers.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "mf_device.hpp"
#include "mf_head.hpp"
#include "mf_launch.hpp"

#ifdef MF_PASS_TIMELINE
static __device__ unsigned long long mf_timeline[1024 * 4 * 32];
extern "C" int mf_debug_pass_timeline(void* dst, unsigned long bytes) {
  return static_cast<int>(hipMemcpyFromSymbol(dst, HIP_SYMBOL(mf_timeline), bytes, 0,
                                              hipMemcpyDeviceToHost));
}
#endif

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
// Bucket entry: staged slot (bits 0-7), candidate index in the batch (8-17,
// kNoPair: an empty entry), column in the block (18-21), row (22-29).
constexpr uint32_t kNoPair = 0x3FFu;
static_assert(kPassRowsMax <= 256u && kPairBatch <= kNoPair, "bucket entry fields");
__device__ __forceinline__ uint32_t pair_pack(uint32_t slot, uint32_t k, uint32_t c, uint32_t r) {
  return slot | (k << 8) | (c << 18) | (r << 22);
}
// A staged slot's class: slot % 8.  With the slot stride of the panel's
// rows (2 mod 4 bank groups of 16 bytes), the A reads of one K offset by the
// lanes of columns 0-3 and 12-15 of a group meet no bank conflict when their
// slots have distinct classes, and the same for columns 4-11 (the lanes one
// ds_read_b128 cycle serves); the buckets deal each block's candidates so
// that those two halves of a group hold distinct classes wherever the counts
// allow.
constexpr uint32_t kSlotClasses = 8;
// column of entry i (0..7) of half h of a group: h = 0 takes columns 0-3,
// 12-15, h = 1 columns 4-11
__device__ __forceinline__ uint32_t half_col(uint32_t h, uint32_t i) {
  return h == 0u ? (i < 4u ? i : i + 8u) : 4u + i;
}
// Per-row flags of a batch: bit 31 = the record is rescored in full; the low
// bits count the members.
constexpr uint32_t kRowAll = 0x80000000u;
// Dynamic LDS of the workgroup (one per compute unit), and the slack after
// the staging area that a wave's last 1 KiB copy may run into.
constexpr uint32_t kLdsBudget = 160u * 1024u - 1024u;
constexpr uint32_t kCopySlack = 1024u;
// s_waitcnt immediate for vmcnt(0) alone (gfx9 encoding: vmcnt in bits 3:0
// and 15:14, expcnt 6:4, lgkmcnt 11:8; the other counters at their maxima).
constexpr int kWaitVmcnt0 = 0x0F70;

// Float bits with the float order as unsigned integers (for LDS atomicMax).
__device__ __forceinline__ uint32_t order_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_order_bits(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// 16-byte aligned size: the staging area after it is read in 16-byte pieces
// (a misaligned ds_read_b128 is split and several times slower).
struct alignas(16) PassShared {
  uint32_t begin[kPassRowsMax];         // list index of the row's first id in the tile
  uint32_t count[kPassRowsMax];         // its ids in the tile
  uint32_t prefix[kPassRowsMax + 1];    // candidates before row r
  uint32_t rprefix[kPassRowsMax + 1];   // rows with candidates before row r
  uint32_t lo[kPassRowsMax];            // list position of the row's first id in the tile
  uint32_t rec[kPassRowsMax];           // record index of (row, tile)
  uint32_t slot_off[kPassRowsMax];      // staged slot -> byte offset of its row of z (batch)
  float rf1[kPassRowsMax];              // coef * ||z|| + coef2 of the row
  float rf2[kPassRowsMax];              // its absolute error term
  uint32_t row_lower[kPassRowsMax];     // per row: max of g - b, order-preserving bits
  uint32_t row_upper[kPassRowsMax];     // per row: max of g + b, order-preserving bits
  uint32_t row_flags[kPassRowsMax];     // kRowAll | members
  uint32_t ptok[kPairBatch];            // candidate k of the batch: id, g + b, row
  float pupper[kPairBatch];             // (+inf: not scored)
  float pscore[kPairBatch];             // candidate k's fast score
  uint16_t prow[kPairBatch];
  alignas(16) uint32_t bent[kBucketSlots];  // read 16 bytes at a time
  uint32_t bcount[kHeadTileBlocks * kSlotClasses];  // candidates per (block, slot class)
  uint32_t bfill[kHeadTileBlocks * kSlotClasses];   // rank of the class's next candidate
  uint32_t bstart[kHeadTileBlocks + 1];  // padded bucket starts (multiples of 16)
  uint32_t wave_n[kWaves];
  uint32_t wave_h[kWaves];
  float tn[kHeadTileTokens];            // token norm bounds of the tile
};

// LDS image of one FP16 row of z: H halves and a 16-byte pad (the panel's
// own row format); the 1168-byte stride at H = 576 puts the 16 rows of one
// A read on distinct banks.
__host__ __device__ constexpr uint32_t slot_bytes(uint32_t H) { return 2u * (H + kPanelPad); }

// Layout: [PassShared][staging area].  The staging area holds the rows of
// z while candidates are scored, then a panel tile's hi rows and the head's
// epilogue scratch (HeadEpi).
__host__ __device__ constexpr uint32_t stage_slots(uint32_t H) {
  const uint32_t room = kLdsBudget - static_cast<uint32_t>(sizeof(PassShared)) - kCopySlack;
  const uint32_t n = room / slot_bytes(H);
  return n < kPassRowsMax ? n : kPassRowsMax;
}
// The panel part is rounded up to whole 1 KiB copies so that its last copy
// stays inside it.
__host__ __device__ constexpr uint32_t panel_part(uint32_t H) {
  return (kPanelRows * slot_bytes(H) + 1023u) / 1024u * 1024u;
}
__host__ __device__ constexpr uint32_t pass_lds_bytes(uint32_t H) {
  const uint32_t rows = stage_slots(H) * slot_bytes(H);
  const uint32_t head = panel_part(H) + static_cast<uint32_t>(sizeof(HeadEpi));
  return static_cast<uint32_t>(sizeof(PassShared)) + (rows > head ? rows : head) + kCopySlack;
}
static_assert(sizeof(PassShared) % 16 == 0, "the staging area starts 16-byte aligned");
static_assert(stage_slots(576) >= 112 && pass_lds_bytes(576) <= kLdsBudget,
              "the pass stages 112 rows of z at H = 576, one workgroup per CU");

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

// Copies the first n slots of a panel tile (slots of [hi | lo], kPanelPad
// halves after each) into LDS slots of slot_bytes(H): the hi half with its
// pad.  Wave w takes the 1 KiB copies w, w + 4, ...: piece q of the area is
// piece q % per of slot q / per; each lane steps its slot and piece from one
// copy of its wave to the next (no division per copy).  Lanes past the last
// piece copy piece 0.
template <uint32_t H>
__device__ __forceinline__ void stage_panel_rows(unsigned char* area, uint32_t n,
                                                 const uint16_t* base) {
  constexpr uint32_t per = slot_bytes(H) / 16u;
  constexpr uint32_t kStride = kWaves * kWave;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t pieces = n * per;
  const unsigned char* b = reinterpret_cast<const unsigned char*>(base);
  uint32_t q = wave * kWave + lane;
  uint32_t i = q / per;
  uint32_t pp = q - i * per;
  for (uint32_t c = wave; c * kWave < pieces; c += kWaves) {
    const uint32_t g = q < pieces ? __umul24(i, 2u * per) + pp : 0u;  // piece of the panel tile
    burst_to_lds(b + g * 16u, area + c * kWave * 16u);
    q += kStride;
    i += kStride / per;
    pp += kStride % per;
    if (pp >= per) {
      pp -= per;
      ++i;
    }
  }
}

// stage_rows for rows of z given by a slot -> byte offset map in LDS, eight
// copies per round: the eight map reads are issued together, then the eight
// copies (a loop of single copies pays an LDS round trip per copy).  Each
// lane steps its slot and piece from one copy of its wave to the next (the
// wave's copies are kWaves apart, kWaves kWave pieces), so a copy costs no
// division and no 64-bit multiply.
template <uint32_t H>
__device__ __forceinline__ void stage_rows_batched(unsigned char* area, uint32_t n,
                                                   const uint32_t* slot_off, const uint16_t* z) {
  constexpr uint32_t per = slot_bytes(H) / 16u;
  constexpr uint32_t kRound = 8;
  constexpr uint32_t kStride = kWaves * kWave;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t pieces = n * per;
  const uint32_t copies = (pieces + kWave - 1u) / kWave;
  const unsigned char* zb = reinterpret_cast<const unsigned char*>(z);
  uint32_t q = wave * kWave + lane;  // this lane's piece in the wave's next copy
  uint32_t i = q / per;
  uint32_t pp = q - i * per;
  for (uint32_t c0 = wave; c0 < copies; c0 += kWaves * kRound) {
    uint32_t off[kRound];
    uint32_t pq[kRound];
#pragma unroll
    for (uint32_t u = 0; u < kRound; ++u) {
      const bool in = q < pieces;
      off[u] = slot_off[in ? i : 0u];
      pq[u] = in && pp < H / 8u ? pp : 0u;
      q += kStride;
      i += kStride / per;
      pp += kStride % per;
      if (pp >= per) {
        pp -= per;
        ++i;
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < kRound; ++u) {
      const uint32_t c = c0 + u * kWaves;
      if (c < copies) burst_to_lds(zb + off[u] + pq[u] * 16u, area + c * kWave * 16u);
    }
  }
}

template <int kSteps>
__global__ __launch_bounds__(kThreads) void pass_kernel(PassArgs p) {
  constexpr uint32_t H = 32u * kSteps;
  constexpr uint32_t kSlot = slot_bytes(H);
  constexpr uint32_t kTileHalves = static_cast<uint32_t>(panel_tile_bytes(H) / 2u);
  constexpr uint32_t kPanelSlotHalves = 2u * (H + kPanelPad);  // one panel slot's [hi | lo]
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t src_row[kPanelRows];
  __shared__ float src_norm[kPanelRows];
  __shared__ float src_slack[kPanelRows];
  const FallbackArgs& f = p.head;
  const uint32_t panels = f.m > 0 ? panel_tiles(f.m) : 0u;
  PassShared& ps = *reinterpret_cast<PassShared*>(dyn);
  unsigned char* stage = dyn + sizeof(PassShared);
  // after the candidates: a panel tile's hi rows (tiles past the first),
  // then the head's epilogue
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
  // steps [s0, s1) of block tb's K range.  A whole block from all four waves
  // (4 x 18 KiB at H = 576) is more than the compute unit keeps in flight,
  // so the last wave's issue would stall until the first loads return; the
  // blocks that precede a workgroup barrier are issued in two halves, the
  // second after the barrier.
  auto load_steps = [&](uint32_t t, int tb, int s0, int s1) {
    const uint32_t token = t * kHeadTileTokens + (wave * kBlocks + tb) * 16u + col;
    const uint16_t* src = f.emb + static_cast<uint64_t>(token < f.V ? token : 0u) * H + kb * 8u;
#pragma unroll
    for (int s = s0; s < s1; ++s) bt[tb][s] = *reinterpret_cast<const half8_t*>(src + s * 32);
  };
  constexpr int kFirstHalf = kSteps / 2;
  auto load_block = [&](uint32_t t, int tb) { load_steps(t, tb, 0, kSteps); };
  // The head's A operand: a panel tile's hi rows staged in LDS (slot j in
  // LDS slot j); its MFMAs against every block of the tile
  // (only the tile's real rows; the A rows of the others read whatever the
  // LDS holds, and their scores are never used)
  auto stage_panel = [&](uint32_t pt) {
    const uint16_t* base = f.panel + static_cast<uint64_t>(pt) * kTileHalves;
    const uint32_t n = f.m - pt * kPanelRows < kPanelRows ? f.m - pt * kPanelRows : kPanelRows;
    stage_panel_rows<H>(panel, n, base);
  };
  auto head_lds = [&](HeadAcc<kBlocks>& h) {
#pragma unroll
    for (int tb = 0; tb < kBlocks; ++tb) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) h.acc[rb][tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // A reads kAhead steps ahead of their MFMAs (a step's six MFMAs do not
    // cover the LDS latency of its own reads)
    constexpr int kAhead = 2;
    const unsigned char* a_lane = panel + col * kSlot + kb * 16u;
    half8_t a[kAhead + 1][2];
    auto read_step = [&](int s) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        a[s % (kAhead + 1)][rb] = *reinterpret_cast<const half8_t*>(a_lane + rb * 16u * kSlot + s * 64);
      }
    };
#pragma unroll
    for (int s = 0; s < kAhead; ++s) read_step(s);
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      if (s + kAhead < kSteps) read_step(s + kAhead);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int tb = 0; tb < kBlocks; ++tb) {
          h.acc[rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s % (kAhead + 1)][rb], bt[tb][s],
                                                                 h.acc[rb][tb], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  MF_STAMP(0);
  for (uint32_t tile = t_begin; tile < t_end; ++tile) {
    const uint32_t t0 = tile * kHeadTileTokens;
    // (1) the small loads first, ahead of the table's: the plan's per-row
    // values (one row per thread; the range index is range-major, so
    // contiguous)
    const uint32_t ri = tid < rows ? tid : 0u;
    const RowMeta m = p.row_meta[ri];
    const uint32_t rt = p.row_tiles[ri];
    const uint4 ix = p.range_index[static_cast<uint64_t>(tile) * rows + ri];
    const float norm_r = p.row_norm[ri];
    const float slack_r = p.row_slack[ri];
    // panel tile 0's slots (stored just before the head: they land well
    // after the plan, and nothing earlier reads them)
    const HeadSlotLoad slot0 = head_slot_load(f, 0u, p.row_norm);
    __builtin_amdgcn_sched_barrier(0);
    // the tile's first block of table rows, behind the small loads: it
    // streams while the plan is scanned and the rows of z are staged (its
    // second half once the scans' barrier is passed)
    load_steps(tile, 0, 0, kFirstHalf);
    __builtin_amdgcn_sched_barrier(0);
    MF_STAMP(1);

    // (2) per row its span [lo, hi) in the tile; exclusive scans over the
    // rows: candidates and rows with candidates
    {
      const uint32_t lo_r = ix.x;
      const uint32_t hi_r = ix.y;
      const uint32_t rec_r = ix.z;
      const bool use = tid < rows && (m.kind & kRowRestricted) && !(rt & kRangesUnused) &&
                       hi_r > lo_r && hi_r <= m.count && rec_r < p.max_recs;
      const uint32_t n = use ? hi_r - lo_r : 0u;
      const uint32_t has = n > 0u ? 1u : 0u;
      if (tid < rows) {
        ps.begin[tid] = m.list_begin + lo_r;
        ps.count[tid] = n;
        ps.lo[tid] = lo_r;
        ps.rec[tid] = rec_r;
        ps.rf1[tid] = __builtin_fmaf(p.coef, norm_r, p.coef2);
        ps.rf2[tid] = slack_r;
      }
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
        ps.wave_n[wave] = in_n;
        ps.wave_h[wave] = in_h;
      }
      __syncthreads();
      uint32_t bn = in_n - n;
      uint32_t bh = in_h - has;
      for (uint32_t w = 0; w < wave; ++w) {
        bn += ps.wave_n[w];
        bh += ps.wave_h[w];
      }
      if (tid <= rows) {  // tid == rows: the totals
        ps.prefix[tid] = bn;
        ps.rprefix[tid] = bh;
      }
      if (tid == kThreads - 1 && rows == kPassRowsMax) {
        ps.prefix[rows] = bn + n;
        ps.rprefix[rows] = bh + has;
      }
      __syncthreads();
    }
    MF_STAMP(2);

    // (3) batches of whole rows.  The first is scored block by block as the
    // table rows land; the others (rows past the LDS stage) afterwards.
    HeadAcc<kBlocks> h;
    uint32_t r0 = 0u;
    // the batch body, compiled separately for the first batch (which issues
    // the table rows) and the others, so that no control-flow join makes
    // the compiler's memory waits conservative
    auto run_batch = [&](auto first_c) -> bool {
      constexpr bool first = decltype(first_c)::value;
      // (the common case, every remaining row in one batch, without the
      // searches)
      const bool fits = ps.prefix[rows] - ps.prefix[r0] <= kPairBatch &&
                        ps.rprefix[rows] - ps.rprefix[r0] <= slots;
      uint32_t r1 = rows;
      if (!fits) {
        const uint32_t r1a = last_within(ps.prefix, rows, r0, kPairBatch);
        const uint32_t r1b = last_within(ps.rprefix, rows, r0, slots);
        r1 = r1a < r1b ? r1a : r1b;
      }
      const uint32_t k0 = ps.prefix[r0];
      const uint32_t nb = ps.prefix[r1] - k0;
      const uint32_t s0 = ps.rprefix[r0];
      const uint32_t nz = ps.rprefix[r1] - s0;
      if (tid < kHeadTileBlocks * kSlotClasses) ps.bcount[tid] = 0u;
      if (tid >= r0 && tid < r1) {
        const uint32_t n = ps.count[tid];
        if (n > 0u) {
          ps.slot_off[ps.rprefix[tid] - s0] = tid * (2u * H);
          // the row of each of its candidates (a row has at most one
          // tile's worth)
          const uint32_t base = ps.prefix[tid] - k0;
          for (uint32_t j = 0; j < n; ++j) ps.prow[base + j] = static_cast<uint16_t>(tid);
        }
      }
      if (tid < rows) {
        ps.row_lower[tid] = order_bits(-__builtin_huge_valf());
        ps.row_upper[tid] = order_bits(-__builtin_huge_valf());
        ps.row_flags[tid] = 0u;
      }
      __syncthreads();  // slot rows, candidate rows, cleared counters
      if constexpr (first) {
        // block 0's second half: its issue waits for the first half's loads
        // to drain, which the batch set-up above no longer does
        __builtin_amdgcn_sched_barrier(0);
        load_steps(tile, 0, kFirstHalf, kSteps);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (first) MF_STAMP(3);
      // the batch's rows of z straight into LDS (block 0 of the table rows
      // streams ahead of them), then its candidate ids (lanes past the
      // batch load candidate k0 again, a valid list position, instead of
      // branching around their loads; a batch without candidates reads list
      // entry 0, which the host guarantees readable), then -- first batch
      // -- the second block of table rows
      uint32_t row[2];
      uint32_t at[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t k = tid + u * kThreads;
        const uint32_t kk = k < nb ? k : 0u;
        const uint32_t r = ps.prow[kk];
        row[u] = r < rows ? r : rows - 1u;
        at[u] = nb > 0u ? ps.begin[row[u]] + (k0 + kk - ps.prefix[row[u]]) : 0u;
      }
      __builtin_amdgcn_sched_barrier(0);
      stage_rows_batched<H>(stage, nz, ps.slot_off, p.z_hi);
      __builtin_amdgcn_sched_barrier(0);
      uint32_t tok[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) tok[u] = p.tokens[at[u]];
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (first) MF_STAMP(4);
      // every load has landed (block 0, the staged rows, the ids: a wait the
      // compiler sees, so that it counts the later table loads in order);
      // first batch: block 1 (it streams while block 0 is scored; block 2 is
      // issued once block 0 is scored)
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (first) MF_STAMP(5);
      if constexpr (first) load_steps(tile, 1, 0, kFirstHalf);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (first) MF_STAMP(16);
      // buckets: each candidate in its 16-token block's bucket
      uint32_t blk[2];
      uint32_t slot[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t k = k0 + tid + u * kThreads;
        const uint32_t c = tok[u] - t0;
        blk[u] = (k < k0 + nb && c < kHeadTileTokens) ? c / 16u : kHeadTileBlocks;
        slot[u] = ps.rprefix[row[u]] - s0;
        if (k < k0 + nb) {
          ps.ptok[k - k0] = tok[u];
          ps.pupper[k - k0] = __builtin_huge_valf();
          if (blk[u] < kHeadTileBlocks) {
            atomicAdd(&ps.bcount[blk[u] * kSlotClasses + slot[u] % kSlotClasses], 1u);
          } else {
            atomicOr(&ps.row_flags[row[u]], kRowAll);  // an id outside the tile: rescore in full
          }
        }
      }
      __syncthreads();
      if constexpr (first) MF_STAMP(17);
      if (wave == 0) {
        // lane b < 12: block b's classes in order (each class's first rank
        // into bfill), its padded size, and an exclusive scan over blocks
        uint32_t n = 0u;
        if (lane < kHeadTileBlocks) {
          uint32_t c[kSlotClasses];
#pragma unroll
          for (uint32_t q = 0; q < kSlotClasses; ++q) c[q] = ps.bcount[lane * kSlotClasses + q];
#pragma unroll
          for (uint32_t q = 0; q < kSlotClasses; ++q) {
            ps.bfill[lane * kSlotClasses + q] = n;
            n += c[q];
          }
        }
        const uint32_t padded = (n + 15u) & ~15u;
        uint32_t incl = padded;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
          const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), d));
          if (static_cast<int>(lane) >= d) incl += o;
        }
        if (lane < kHeadTileBlocks) ps.bstart[lane] = incl - padded;
        if (lane == kHeadTileBlocks - 1) ps.bstart[kHeadTileBlocks] = incl;
      }
      for (uint32_t e = tid; e < kBucketSlots; e += kThreads) ps.bent[e] = pair_pack(0u, kNoPair, 0u, 0u);
      __syncthreads();
      if constexpr (first) MF_STAMP(18);
      // rank k of a candidate in its block (classes in order); the block's
      // P = size / 8 halves of groups take ranks k = j, j + P, ...: half
      // j = k % P is half j % 2 of group j / 2, entry k / P in it
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (blk[u] < kHeadTileBlocks) {
          const uint32_t k = atomicAdd(&ps.bfill[blk[u] * kSlotClasses + slot[u] % kSlotClasses], 1u);
          const uint32_t b0 = ps.bstart[blk[u]];
          const uint32_t P = (ps.bstart[blk[u] + 1] - b0) / 8u;
          const uint32_t j = k % P;
          const uint32_t at = b0 + (j / 2u) * 16u + half_col(j % 2u, k / P);
          const uint32_t r = row[u];
          ps.bent[at] = pair_pack(slot[u], tid + u * kThreads, (tok[u] - t0) % 16u, r);
        }
      }
      __syncthreads();  // buckets and staged rows visible
      if constexpr (first) {
        __builtin_amdgcn_sched_barrier(0);
        load_steps(tile, 1, kFirstHalf, kSteps);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (first) MF_STAMP(6);

      // (4) this wave's blocks in landing order: token norms (first batch),
      // the candidates 16 at a time, the next block's rows (first batch)
      //
      // A block's groups run as a software pipeline over two halves of the
      // K range: while the MFMAs of one half run, the other half's A rows
      // (the next group's first half, or this group's second) are read from
      // LDS, and the previous group's scores leave the accumulators between
      // this group's halves, after its MFMAs had a whole half to finish.
      // The loop holds no wait but the ones for its A rows: a lane holds
      // D[i][lane % 16] for the four candidates i = 4 (lane / 16) + e (one
      // 16-byte read of their bucket entries), and writes the element whose
      // candidate's column is lane % 16 to pscore; bounds and row maxima
      // follow once every block is scored.  Reads of a group past the
      // block's last re-read the last group (no branch around LDS reads,
      // whose waits the compiler counts in order).
      constexpr int kHalf = (kSteps + 1) / 2;
      auto dump = [&](const floatx4& acc, const uint4& gq) {
        const uint32_t g[4] = {gq.x, gq.y, gq.z, gq.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t k = (g[e] >> 8) & 0x3FFu;
          if (k != kNoPair && ((g[e] >> 18) & 15u) == col) ps.pscore[k] = acc[e];
        }
      };
      auto score_block = [&](const half8_t(&b)[kSteps], uint32_t qa, uint32_t qz) {
        half8_t a0[kHalf];
        half8_t a1[kHalf];
        auto a_src = [&](uint32_t ge) { return stage + (ge & 0xFFu) * kSlot + kb * 16u; };
        auto entries = [&](uint32_t q) { return *reinterpret_cast<const uint4*>(&ps.bent[q * 16u + 4u * kb]); };
        auto read_half = [&](half8_t(&dst)[kHalf], const unsigned char* from, int h0) {
#pragma unroll
          for (int s = 0; s < kHalf; ++s) {
            if (h0 + s < kSteps) dst[s] = *reinterpret_cast<const half8_t*>(from + (h0 + s) * 64);
          }
        };
        auto mfma_half = [&](const half8_t(&a)[kHalf], int h0, floatx4& acc) {
#pragma unroll
          for (int s = 0; s < kHalf; ++s) {
            if (h0 + s < kSteps) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s], b[h0 + s], acc, 0, 0, 0);
          }
        };
        uint32_t ge = ps.bent[qa * 16u + col];
        uint4 gq = entries(qa);
        const unsigned char* from = a_src(ge);
        read_half(a0, from, 0);
        // nothing pending yet: entries without a candidate
        floatx4 pacc = {0.0f, 0.0f, 0.0f, 0.0f};
        const uint32_t none = pair_pack(0u, kNoPair, 0u, 0u);
        uint4 pq = {none, none, none, none};
        for (uint32_t q = qa; q < qz; ++q) {
          const uint32_t qn = q + 1u < qz ? q + 1u : q;
          const uint32_t ge_n = ps.bent[qn * 16u + col];
          const uint4 gq_n = entries(qn);
          read_half(a1, from, kHalf);
          floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
          mfma_half(a0, 0, acc);
          dump(pacc, pq);
          const unsigned char* from_n = a_src(ge_n);
          read_half(a0, from_n, 0);
          mfma_half(a1, kHalf, acc);
          pacc = acc;
          pq = gq;
          ge = ge_n;
          gq = gq_n;
          from = from_n;
        }
        dump(pacc, pq);
      };
#pragma unroll
      for (int tb = 0; tb < kBlocks; ++tb) {
        const uint32_t blk_id = wave * kBlocks + tb;
        if constexpr (first) {
          // Gram diagonal: token norm bounds of the block (this wave's own)
          // (one chain: a dependent MFMA on the same accumulator issues
          // back to back)
          h.gram[tb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int s = 0; s < kSteps; ++s) {
            h.gram[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bt[tb][s], bt[tb][s], h.gram[tb], 0, 0, 0);
          }
          const uint32_t e = col % 4u;
          const float d = e == 0u ? h.gram[tb][0]
                                  : (e == 1u ? h.gram[tb][1] : (e == 2u ? h.gram[tb][2] : h.gram[tb][3]));
          if (col / 4u == kb) ps.tn[blk_id * 16u + col] = __fsqrt_rn(d) * (1.0f + 0x1p-7f);
          wave_sync();
        }
        const uint32_t qa = __builtin_amdgcn_readfirstlane(ps.bstart[blk_id] / 16u);
        const uint32_t qz = __builtin_amdgcn_readfirstlane(ps.bstart[blk_id + 1] / 16u);
        if (qa < qz) score_block(bt[tb], qa, qz);
        if constexpr (first) MF_STAMP(7 + tb);
        if constexpr (first) {
          if (tb == 0) {
            __builtin_amdgcn_sched_barrier(0);
            load_block(tile, 2);
            __builtin_amdgcn_sched_barrier(0);
            MF_STAMP(22);
          }
        }
      }
      __syncthreads();  // every candidate scored; the staging area is free
      if constexpr (first) MF_STAMP(10);
      // the last batch: panel tile 0's hi rows land while the records are
      // written
      const bool last = r1 >= rows || nb == 0u;
      if (last && panels > 0u) stage_panel(0u);
      if constexpr (first) MF_STAMP(20);

      // each candidate's bound (the token's norm bound, the row's terms),
      // its row's maxima of g - b and g + b (order-preserving integer bits);
      // a non-finite score or bound marks the record "rescore all".  An id
      // outside the tile was never scored (its row is rescored in full).
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t kk = tid + u * kThreads;
        if (kk < nb) {
          const uint32_t c = ps.ptok[kk] - t0;
          if (c < kHeadTileTokens) {
            const uint32_t r = ps.prow[kk];
            const float gs = ps.pscore[kk];
            const float bnd = __builtin_fmaf(ps.tn[c], ps.rf1[r], ps.rf2[r]);
            const bool ok = __builtin_isfinite(gs) && __builtin_isfinite(bnd) && bnd < 0x1p100f;
            if (ok) {
              atomicMax(&ps.row_lower[r], order_bits(gs - bnd));
              atomicMax(&ps.row_upper[r], order_bits(gs + bnd));
              ps.pupper[kk] = gs + bnd;
            } else {
              atomicOr(&ps.row_flags[r], kRowAll);
            }
          }
        }
      }
      __syncthreads();
      if constexpr (first) MF_STAMP(11);

      // (5) one window record per (row, tile).  The best lower bound came
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
          if (!(ps.row_flags[r] & kRowAll) && up >= from_order_bits(ps.row_lower[r])) {
            const uint32_t i = atomicAdd(&ps.row_flags[r], 1u) & ~kRowAll;
            if (i < static_cast<uint32_t>(kTileMembers)) {
              const uint32_t j = k0 + kk - ps.prefix[r];
              TileRecord* rec = p.records + static_cast<uint64_t>(r) * p.max_recs + ps.rec[r];
              // g - b of a member is only used against the row's window
              rec->m[i] = TileMember{ps.ptok[kk], ps.lo[r] + j, -__builtin_huge_valf(), up};
            }
          }
        }
      }
      __syncthreads();
      for (uint32_t r = r0 + tid; r < r1; r += kThreads) {
        const uint32_t n = ps.count[r];
        if (n == 0u) continue;
        const uint32_t fl = ps.row_flags[r];
        const bool all = (fl & kRowAll) != 0u;
        const uint32_t members = fl & ~kRowAll;
        const bool ordinary = !all && members <= static_cast<uint32_t>(kTileMembers);
        TileRecord* rec = p.records + static_cast<uint64_t>(r) * p.max_recs + ps.rec[r];
        const uint32_t lo = ps.lo[r];
        // the header in two 16-byte stores: {best_lower, flags, min_token,
        // min_pos} and {begin, count, n_members, upper_max}
        uint4* hd = reinterpret_cast<uint4*>(rec);
        hd[0] = uint4{__float_as_uint(from_order_bits(ps.row_lower[r])),
                      ordinary ? 0u : (all ? kTileRescoreAll : kTileRescoreAll | kTileCrowded),
                      ps.ptok[ps.prefix[r] - k0], lo};
        hd[1] = uint4{lo, n, ordinary ? members : 0u, __float_as_uint(from_order_bits(ps.row_upper[r]))};
      }
      __syncthreads();  // the batch's LDS is free again
      if constexpr (first) MF_STAMP(12);
      r0 = r1;
      return r0 < rows && nb > 0u;
    };
    if (run_batch(std::true_type{})) {
      while (run_batch(std::false_type{})) {
      }
    }

    // (6) the unrestricted rows: the head against each panel tile's hi rows
    // (panel tile 0 was staged by the last batch) and its records
    head_slot_store(f, 0u, slot0, src_row, src_norm, src_slack);
    for (uint32_t pt = 0; pt < panels; ++pt) {
      if (pt > 0u) {
        stage_panel(pt);  // the previous tile's readers are done
        head_slots(f, pt * kPanelRows, src_row, src_norm, src_slack);
      }
      wait_vector_memory();
      __syncthreads();
      MF_STAMP(13);
      head_lds(h);
      MF_STAMP(14);
      head_records<kWaves, kBlocks, true>(f, h, epi, src_row, src_norm, src_slack,
                                          pt * kPanelRows, tile, tiles);
    }
  }
  MF_STAMP(15);
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
