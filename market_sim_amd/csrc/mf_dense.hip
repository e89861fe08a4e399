// The dense head: one pass over the FP16 table in 192-token tiles that
// scores every row of a panel against every token of the tile with MFMA, and
// keeps, per (row, tile), the window record of the tokens the row allows.
//
// Its rows (slots): the unrestricted rows of the call (all tokens allowed),
// then the restricted rows with long ascending lists that the norm launch
// marked kRowDense.  For such a row the gather would read one 4 KiB table
// row per candidate (at H = 2048, 1.5 M candidates are 6.5 GB); the dense
// head reads each table row once per panel of 256 slots and pays in MFMA
// work instead (2 H flops per slot and token).
//
// Workgroup: a panel of 256 slots (16 blocks of 16) x one tile of 12 token
// blocks, eight waves.  MFMA wave w (0-3) takes the row blocks of parity
// w % 2 and the six token blocks of half w / 2 (8 x 6 MFMA blocks,
// v_mfma_f32_16x16x32_f16); waves 4-7 issue the copies (a wave issuing
// copies stalls while the address unit is busy, and an MFMA wave would idle
// with it).  K runs in 32-feature steps; each step's A rows (the slots' FP16
// hi of z = x * w, from L2) and B rows (the tile's table rows, from HBM) are
// copied straight into LDS (global_load_lds, 16 bytes per lane), three steps
// in flight beside the one being multiplied; one barrier per step hands it
// over.  LDS rows are 64 bytes; piece p of row r sits at p ^ swz(r), so the
// 16 rows one fragment read touches fall on distinct banks.  The MFMA waves
// also sum the squares of the table fragments they read (FP32, any order),
// which gives the token norms of the bounds.
//
// Epilogue per tile: the slot's allowed tokens of the tile come from the
// norm launch's span index (a 192-bit mask and the list position of the
// first id), copied into LDS during the previous tile; per slot the best
// lower bound over allowed tokens, the members (fl(g + b) >= L) and one
// TileRecord in the MFMA head's format (list positions for restricted rows,
// token ids for unrestricted ones).
//
// Workgroups: one per compute unit.  Each computes the slot list itself (a
// prefix over the rows' kinds), so P = ceil(slots / 256) panels of equal
// size (to one slot); row blocks past a panel's slots get no MFMA.  The
// compute units of an XCD (blockIdx % 8) form groups of P workgroups that
// run the same run of tiles, one panel each, so the table tiles of a group
// are read from HBM once and from the XCD's L2 by the other panels.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kMmaWaves = 4;
constexpr int kCopyWaves = 4;
constexpr int kWaves = kMmaWaves + kCopyWaves;
constexpr int kThreads = kWaves * kWave;
static_assert(kMmaWaves * kWave == static_cast<int>(kDensePanelSlots), "one MFMA thread per slot");
constexpr int kRBw = 8;  // row blocks per MFMA wave
constexpr int kTBw = 6;  // token blocks per MFMA wave
constexpr int kNormBw = 3;  // token blocks whose norms the MFMA wave forms
constexpr int kStages = 4;
constexpr uint32_t kABytes = kDensePanelSlots * 64u;  // one 32-feature step of every slot
constexpr uint32_t kBBytes = kHeadTileTokens * 64u;   // one step of the tile's table rows
constexpr uint32_t kStageBytes = kABytes + kBBytes;
constexpr int kADma = static_cast<int>(kABytes / 1024u / kCopyWaves);  // 1 KiB copies per wave
constexpr int kBDma = static_cast<int>(kBBytes / 1024u / kCopyWaves);
constexpr int kDmaPerWave = kADma + kBDma;
static_assert(kADma == 4 && kBDma == 3, "copy split");
// epilogue rows in the stage area: [slot][33] arrays of the lanes' values
// (two of floats, one of bytes), then the tile's records staged for the
// store
constexpr uint32_t kEpiRow = 33;
constexpr uint32_t kEpiRowsBytes = kDensePanelSlots * kEpiRow * 4u;
constexpr uint32_t kEpiBlockBytes = (kDensePanelSlots * kEpiRow + 15u) / 16u * 16u;  // bytes
static_assert(2u * kEpiRowsBytes + kEpiBlockBytes + kDensePanelSlots * 96u <=
                  kStages * kStageBytes,
              "epilogue rows and staged records in the stages");
static_assert(kMmaWaves * kTBw / 2 == static_cast<int>(kHeadTileTokens / 16u), "tile");

enum : uint32_t { kSlotNone = 0u, kSlotAll = 1u, kSlotList = 2u };

struct DenseShared {
  uint32_t slot_row[kDensePanelSlots];
  float slot_norm[kDensePanelSlots];
  float slot_slack[kDensePanelSlots];
  uint32_t slot_kind[kDensePanelSlots];
  uint4 span[2][kDensePanelSlots][2];  // per tile parity: {m0,m1,m2,lo},{m3,m4,m5,cnt}
  float tn[kMmaWaves];
  uint32_t wave_sum[kWaves];
};

__host__ __device__ constexpr uint32_t dense_lds_bytes() {
  return kStages * kStageBytes + static_cast<uint32_t>(sizeof(DenseShared));
}

__device__ __forceinline__ uint32_t swz(uint32_t r) { return ((r >> 1) ^ (r >> 3)) & 3u; }

// The slot list of the launch: unrestricted rows first (fb_rows order), then
// the kRowDense rows in row order; panel p of P takes slots [p0, p0 + n)
// with p0 = p S / P (S slots), so the panels differ by one slot at most.
// Fills this panel's slot table.
__device__ void dense_slots(const DenseArgs& a, DenseShared& sh, uint32_t p0, uint32_t n,
                            bool map) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  const uint32_t per = (a.rows + kThreads - 1) / kThreads;
  const uint32_t r0 = tid * per < a.rows ? tid * per : a.rows;
  const uint32_t r1 = r0 + per < a.rows ? r0 + per : a.rows;
  uint32_t local = 0u;
  for (uint32_t r = r0; r < r1; ++r) local += (a.row_meta[r].kind & kRowDense) ? 1u : 0u;
  uint32_t incl = local;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), d));
    if (static_cast<int>(lane) >= d) incl += o;
  }
  if (tid < kDensePanelSlots) sh.slot_kind[tid] = kSlotNone;
  if (lane == kWave - 1) sh.wave_sum[wave] = incl;
  __syncthreads();
  uint32_t before = incl - local;
#pragma unroll
  for (uint32_t w = 0; w < kWaves; ++w) before += w < wave ? sh.wave_sum[w] : 0u;
  // unrestricted slots of this panel (a listed row that is not unrestricted,
  // or not a row, gets no slot work)
  {
    const uint32_t gs = p0 + tid;
    if (tid < n && gs < a.fb_m) {
      const uint32_t r = a.fb_rows[gs];
      if (r < a.rows && (a.row_meta[r].kind & kRowUnrestricted)) {
        sh.slot_row[tid] = r;
        sh.slot_kind[tid] = kSlotAll;
      }
    }
  }
  // dense rows of this panel
  uint32_t k = a.fb_m + before;
  for (uint32_t r = r0; r < r1; ++r) {
    if (a.row_meta[r].kind & kRowDense) {
      if (k >= p0 && k < p0 + n) {
        sh.slot_row[k - p0] = r;
        sh.slot_kind[k - p0] = kSlotList;
      }
      ++k;
    }
  }
  __syncthreads();
  if (tid < kDensePanelSlots) {
    const uint32_t kind = sh.slot_kind[tid];
    const uint32_t r = kind != kSlotNone ? sh.slot_row[tid] : 0u;
    sh.slot_norm[tid] = kind != kSlotNone ? a.row_norm[r] : 0.0f;
    sh.slot_slack[tid] = kind != kSlotNone ? a.row_slack[r] : 0.0f;
    if (kind == kSlotNone) sh.slot_row[tid] = 0u;  // a valid row for the copies
    if (map && kind != kSlotNone) a.fb_map[r] = p0 + tid;
  }
  __syncthreads();
}

// Wait until at most kAfter steps of this copy wave's copies are in flight.
template <int kAfter>
__device__ __forceinline__ void wait_steps() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAfter * kDmaPerWave) : "memory");
}

// A workgroup barrier without __syncthreads' release fence, which would wait
// for every LDS-DMA copy in flight (vector memory count 0) and empty the
// pipeline.  The wave's own LDS operations are complete when it arrives.
__device__ __forceinline__ void step_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__global__ __launch_bounds__(kThreads) void dense_kernel(DenseArgs a) {
  extern __shared__ __align__(16) unsigned char dyn[];
  DenseShared& sh = *reinterpret_cast<DenseShared*>(dyn + kStages * kStageBytes);
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const bool copier = wave >= static_cast<uint32_t>(kMmaWaves);
  const uint32_t cw = wave % kCopyWaves;  // copy wave index (copy waves)
  const uint32_t wm = wave % 2u;  // row-block parity (MFMA waves)
  const uint32_t wn = (wave / 2u) % 2u;  // token half (MFMA waves)
  const uint32_t col = lane % 16u;
  const uint32_t kb = lane / 16u;
  // workgroup -> (group, panel): the compute units of one XCD in groups of
  // P consecutive local indices.  The slot count is computed first with
  // panel 0's table (every workgroup needs it).
  const uint32_t xcds = 8u;
  const uint32_t per_xcd = gridDim.x / xcds;
  const uint32_t x = blockIdx.x % xcds;
  const uint32_t l = blockIdx.x / xcds;
  uint32_t n_slots;
  {
    // the count does not depend on the panel; the table of the true panel
    // is built below
    const uint32_t per = (a.rows + kThreads - 1) / kThreads;
    const uint32_t r0 = tid * per < a.rows ? tid * per : a.rows;
    const uint32_t r1 = r0 + per < a.rows ? r0 + per : a.rows;
    uint32_t local = 0u;
    for (uint32_t r = r0; r < r1; ++r) local += (a.row_meta[r].kind & kRowDense) ? 1u : 0u;
    local = wave_sum_u32(local);
    if (lane == 0) sh.wave_sum[wave] = local;
    __syncthreads();
    n_slots = a.fb_m;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) n_slots += sh.wave_sum[w];
    __syncthreads();
  }
  const uint32_t P = (n_slots + kDensePanelSlots - 1) / kDensePanelSlots;
  if (P == 0u || P > per_xcd) return;  // the launcher bounds P by per_xcd
  const uint32_t gpx = per_xcd / P;
  if (l >= gpx * P) return;
  const uint32_t panel = l % P;
  const uint32_t p0 = panel * n_slots / P;
  const uint32_t pn = (panel + 1u) * n_slots / P - p0;
  // row blocks with slots; wave parity wm takes blocks 2 i + wm, i < nact
  const uint32_t nrb = (pn + 15u) / 16u;
  const uint32_t nact = nrb > wm ? (nrb - wm + 1u) / 2u : 0u;
  const uint32_t grp = x * gpx + l / P;
  const uint32_t groups = xcds * gpx;
  const uint32_t tiles = a.ranges;
  const uint32_t t_begin = static_cast<uint32_t>(static_cast<uint64_t>(tiles) * grp / groups);
  const uint32_t t_end = static_cast<uint32_t>(static_cast<uint64_t>(tiles) * (grp + 1u) / groups);
  dense_slots(a, sh, p0, pn, grp == 0u);
  const uint32_t H = a.H;
  const uint32_t steps = H / 32u;
  // The tile's LDS epilogue areas (the stage area, free after the K loop):
  // per-lane values of each slot in rows of 33 words (word 16 half + column
  // of slot s's row, padded so the four slots of one write sit on different
  // banks), then the tile's records, staged for the store.
  float* gl1 = reinterpret_cast<float*>(dyn);                          // best
  float* gl2 = reinterpret_cast<float*>(dyn + kEpiRowsBytes);          // second best
  uint8_t* glj = dyn + 2u * kEpiRowsBytes;  // token block of the best
  TileRecord* stage_rec = reinterpret_cast<TileRecord*>(dyn + 2u * kEpiRowsBytes + kEpiBlockBytes);
  // the staged records out, 16 bytes per thread and step (each record is
  // contiguous in global memory); no wait for these stores before the next
  // tile, only for the LDS reads
  auto store_records = [&](uint32_t tile) {
    constexpr uint32_t kPieces = sizeof(TileRecord) / 16u;
    const uint4* from = reinterpret_cast<const uint4*>(stage_rec);
    uint32_t u0 = tid;
    asm volatile("" : "+v"(u0));
    for (uint32_t u = u0; u < kDensePanelSlots * kPieces; u += kThreads) {
      const uint32_t s = u / kPieces;
      if (sh.slot_kind[s] == kSlotNone) continue;
      uint4* to = reinterpret_cast<uint4*>(a.records + (static_cast<uint64_t>(p0) + s) * tiles + tile);
      to[u % kPieces] = from[u];
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  // The copy waves: every tile's steps, then the barriers of the MFMA
  // waves' epilogue.  (Separate loops for the two kinds of waves, so that
  // neither holds the other's registers.)
  auto copy_tiles = [&]() {
    // per-lane copy sources of a copy wave: A rows (4 copies of 16 rows),
    // span records (2 copies of 32 slots)
    uint32_t aoff[kADma];
  #pragma unroll
    for (int j = 0; j < kADma; ++j) {
      const uint32_t r = (cw * kADma + j) * 16u + lane / 4u;
      aoff[j] = sh.slot_row[r] * H + (((lane % 4u) ^ swz(r)) * 8u);
    }
    uint32_t srow[2];
  #pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t s = ((cw * 2u + j) * kWave + lane) / 2u;
      srow[j] = sh.slot_kind[s] == kSlotList ? sh.slot_row[s] : 0u;
    }
    auto issue_span = [&](uint32_t tile) {
      uint4* dst = &sh.span[tile & 1u][0][0];
  #pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t idx = (cw * 2u + j) * kWave + lane;
        const uint4* src = a.spans + (static_cast<uint64_t>(tile) * a.rows + srow[j]) * 2u + (idx % 2u);
        burst_to_lds(src, dst + (cw * 2u + j) * kWave);
      }
    };
    if (t_begin < t_end) issue_span(t_begin);
    for (uint32_t tile = t_begin; tile < t_end; ++tile) {
      const uint32_t tok0 = tile * kHeadTileTokens;
      const uint32_t nt = a.V - tok0 < kHeadTileTokens ? a.V - tok0 : kHeadTileTokens;
      if (tile + 1u < t_end) issue_span(tile + 1u);
      const uint16_t* tbase = a.emb + static_cast<uint64_t>(tok0) * H;
      uint32_t boff[kBDma];
#pragma unroll
      for (int j = 0; j < kBDma; ++j) {
        const uint32_t t = (cw * kBDma + j) * 16u + lane / 4u;
        const uint32_t tc = t < nt ? t : nt - 1u;
        boff[j] = tc * H + (((lane % 4u) ^ swz(t)) * 8u);
      }
      auto issue = [&](uint32_t s) {
        unsigned char* st = dyn + (s % kStages) * kStageBytes;
        const uint32_t f = s * 32u;
#pragma unroll
        for (int j = 0; j < kADma; ++j) {
          burst_to_lds(a.z_hi + aoff[j] + f, st + (cw * kADma + j) * 1024u);
        }
#pragma unroll
        for (int j = 0; j < kBDma; ++j) {
          burst_to_lds(tbase + boff[j] + f, st + kABytes + (cw * kBDma + j) * 1024u);
        }
      };
      // steps 0 .. kStages - 2 in flight; then per step s the copies of step
      // s + kStages - 1 go into the stage of step s - 1 (every MFMA wave is
      // done with it), and step s + 1 is handed over once it has landed.
      // Past the last step the last one is copied again (into a stage
      // nobody reads), so that every step issues the same copies.
#pragma unroll
      for (int s = 0; s < kStages - 1; ++s) issue(static_cast<uint32_t>(s) < steps ? s : steps - 1u);
      wait_steps<kStages - 2>();
      step_barrier();  // step 0 in LDS
      for (uint32_t s = 0; s < steps; ++s) {
        issue(s + kStages - 1 < steps ? s + kStages - 1 : steps - 1u);
        wait_steps<kStages - 2>();
        step_barrier();  // step s + 1 in LDS, step s read by every MFMA wave
      }
      // the copies past the last step, and the span copies, have landed;
      // then the MFMA waves' epilogue phases (the same barriers)
      wait_vector_memory();
      __syncthreads();
      __syncthreads();
      __syncthreads();
      __syncthreads();
      store_records(tile);
    }
  };
  // The MFMA waves (thread tid is slot tid), with NACT of the wave's row
  // blocks holding slots (a variant per count, so the loop has no branch
  // around an MFMA).
  auto mfma_tiles = [&]<int NACT>() {
    for (uint32_t tile = t_begin; tile < t_end; ++tile) {
      const uint32_t tok0 = tile * kHeadTileTokens;
      const uint32_t nt = a.V - tok0 < kHeadTileTokens ? a.V - tok0 : kHeadTileTokens;
      const uint32_t b = tile & 1u;
      // (the MFMA waves hold the slots: thread tid is slot tid)
      floatx4 acc[kRBw][kTBw];
#pragma unroll
      for (int i = 0; i < kRBw; ++i) {
#pragma unroll
        for (int j = 0; j < kTBw; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      // per lane: the sums of squares of its features of the tokens of its
      // three norm blocks
      float tsq[kNormBw] = {0.0f, 0.0f, 0.0f};
      step_barrier();  // step 0 in LDS
      for (uint32_t s = 0; s < steps; ++s) {
        const unsigned char* st = dyn + (s % kStages) * kStageBytes;
        half8_t fb[kTBw];
#pragma unroll
        for (int j = 0; j < kTBw; ++j) {
          const uint32_t t = (wn * kTBw + j) * 16u + col;
          fb[j] = *reinterpret_cast<const half8_t*>(st + kABytes + t * 64u + ((kb ^ swz(t)) * 16u));
        }
        // the row blocks' A fragments one ahead of their MFMAs
        auto read_a = [&](int i) {
          const uint32_t r = (2u * static_cast<uint32_t>(i) + wm) * 16u + col;
          return *reinterpret_cast<const half8_t*>(st + r * 64u + ((kb ^ swz(r)) * 16u));
        };
        half8_t fa = read_a(0);
#pragma unroll
        for (int j = 0; j < kNormBw; ++j) {
          const half8_t g = wm == 0u ? fb[j] : fb[kNormBw + j];  // (wm is wave-uniform)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float v = static_cast<float>(g[e]);
            tsq[j] = __builtin_fmaf(v, v, tsq[j]);
          }
        }
#pragma unroll
        for (int i = 0; i < NACT; ++i) {
          const half8_t fn = read_a(i + 1 < NACT ? i + 1 : i);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < kTBw; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa, fb[j], acc[i][j], 0, 0, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
          fa = fn;
        }
        step_barrier();  // this wave is done with step s
      }
      __syncthreads();  // every copy landed

      // token norms: lanes c, c + 16, c + 32, c + 48 hold the four K
      // quarters of column c's sum; a NaN norm (non-finite table row)
      // propagates
      {
        // (the lane's indices made opaque here, so that the compiler forms
        // them after the K loop instead of holding them through it)
        uint32_t el = lane;
        asm volatile("" : "+v"(el));
        const uint32_t ecol = el % 16u;
        const uint32_t t0 = (wn * kTBw + wm * kNormBw) * 16u + ecol;
        const int up16 = static_cast<int>((el ^ 16u) * 4u);
        const int up32 = static_cast<int>((el ^ 32u) * 4u);
        float tn_local = 0.0f;
        bool tn_nan = false;
#pragma unroll
        for (int j = 0; j < kNormBw; ++j) {
          float q = tsq[j];
          q += __int_as_float(__builtin_amdgcn_ds_bpermute(up16, __float_as_int(q)));
          q += __int_as_float(__builtin_amdgcn_ds_bpermute(up32, __float_as_int(q)));
          const uint32_t t = t0 + 16u * static_cast<uint32_t>(j);
          if (el < 16u && t < nt) {
            const float v = __fsqrt_rn(q) * (1.0f + 0x1p-7f);
            tn_nan |= v != v;
            tn_local = __builtin_fmaxf(tn_local, v);
          }
        }
        const bool any_nan = __ballot(tn_nan) != 0ull;
        const float m = wave_max(tn_local);
        if (lane == 0) sh.tn[wave] = any_nan ? __builtin_nanf("") : m;
      }
      // the allowed words of every slot in its span record: unrestricted
      // slots allow the tile's tokens below nt, empty slots nothing
      // (thread tid's slot index made opaque here for the same reason)
      uint32_t es = tid;
      asm volatile("" : "+v"(es));
      {
        const uint32_t kind = sh.slot_kind[es];
        if (kind != kSlotList) {
          uint32_t w[6];
#pragma unroll
          for (int k = 0; k < 6; ++k) {
            const uint32_t lo = k * 32u;
            w[k] = kind == kSlotNone ? 0u
                   : (nt >= lo + 32u ? 0xFFFFFFFFu : (nt > lo ? (1u << (nt - lo)) - 1u : 0u));
          }
          sh.span[b][es][0] = uint4{w[0], w[1], w[2], tok0};
          sh.span[b][es][1] = uint4{w[3], w[4], w[5], kind == kSlotNone ? 0u : nt};
        }
      }
      __syncthreads();
      // lane bases: slot (i, q) of this lane is sbase + 32 i + q (opaque to
      // the compiler, so that the epilogue's addresses are formed here and not
      // hoisted out of the tile loop, where they would outlive the registers)
      uint32_t sbase = wm * 16u + 4u * kb;
      asm volatile("" : "+v"(sbase));
      const uint4* spn = &sh.span[b][sbase][wn];
      const uint32_t sel0 = 1u << col;
      const uint32_t sel1 = 1u << (16u + col);
      const uint32_t lw = sbase * kEpiRow + wn * 16u + col;  // this lane's word of slot sbase
      // per slot and MFMA lane: the best and second best allowed scores of
      // the lane's six tokens and the block of the best (the best is NaN when
      // one of its allowed scores is not finite); the row blocks past the
      // panel's slots hold none of its slots
#pragma unroll
      for (int i = 0; i < NACT; ++i) {
        uint4 w4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) w4[q] = spn[(32 * i + q) * 2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t w[3] = {w4[q].x, w4[q].y, w4[q].z};
          // arithmetic form (one condition per select, no lane-mask logic):
          // va = the score or -inf, vb - vb is NaN exactly when an allowed score is
          // not finite
          float m1 = -__builtin_huge_valf();
          float m2 = -__builtin_huge_valf();
          float badacc = 0.0f;
          uint32_t j1 = 0u;
#pragma unroll
          for (int j = 0; j < kTBw; ++j) {
            const bool allowed = (w[j / 2] & (j % 2 == 0 ? sel0 : sel1)) != 0u;
            const float v = acc[i][j][q];
            const float va = allowed ? v : -__builtin_huge_valf();
            const float vb = allowed ? v : 0.0f;
            badacc += vb - vb;
            m2 = __builtin_fmaxf(m2, __builtin_fminf(m1, va));
            j1 = va > m1 ? static_cast<uint32_t>(j) : j1;
            m1 = __builtin_fmaxf(m1, va);
          }
          gl1[lw + (32 * i + q) * kEpiRow] = badacc != badacc ? __builtin_nanf("") : m1;
          gl2[lw + (32 * i + q) * kEpiRow] = m2;
          glj[lw + (32 * i + q) * kEpiRow] = static_cast<uint8_t>(j1);
        }
      }
      __syncthreads();
      // the slot's record (thread s), written into its LDS stage.  G = the
      // best allowed score, b the bound, L = fl(G - b); the members are the
      // lane bests with fl(g + b) >= L (a lane's other scores are at most its
      // second best: when that qualifies too, the record is crowded)
      {
        float tn_max = sh.tn[0];
#pragma unroll
        for (int w = 1; w < kMmaWaves; ++w) {
          const float v = sh.tn[w];
          tn_max = (tn_max != tn_max || v != v) ? __builtin_nanf("") : __builtin_fmaxf(tn_max, v);
        }
        const uint32_t s = es;
        const uint32_t kind = sh.slot_kind[s];
        const uint4 h0 = sh.span[b][s][0];
        const uint4 h1 = sh.span[b][s][1];
        const uint32_t lo = h0.w;
        const uint32_t cnt = h1.w;
        TileRecord& rec = stage_rec[s];
        if (cnt == 0u) {
          reinterpret_cast<uint4*>(&rec)[0] =
              uint4{__float_as_uint(-__builtin_huge_valf()), 0u, kInvalidToken, lo};
          reinterpret_cast<uint4*>(&rec)[1] =
              uint4{lo, 0u, 0u, __float_as_uint(-__builtin_huge_valf())};
        } else {
          const float* r1 = gl1 + s * kEpiRow;
          const float* r2 = gl2 + s * kEpiRow;
          float G = -__builtin_huge_valf();
          bool fin = true;
#pragma unroll
          for (int u = 0; u < 32; ++u) {
            const float v = r1[u];
            fin &= v == v;
            G = __builtin_fmaxf(G, v);
          }
          const float bs = __builtin_fmaf(tn_max, __builtin_fmaf(a.coef, sh.slot_norm[s], a.coef2),
                                          sh.slot_slack[s]);
          const float L = G - bs;
          const bool finite = fin && bs < 0x1p100f;
          uint32_t members = 0u;  // bit u: lane u's best is a member
          bool crowded = false;
#pragma unroll
          for (int u = 0; u < 32; ++u) {
            members |= (r1[u] + bs >= L) ? (1u << u) : 0u;
            crowded |= r2[u] + bs >= L;
          }
          const uint32_t total = static_cast<uint32_t>(__popc(members));
          const bool ordinary = finite && !crowded && total <= static_cast<uint32_t>(kTileMembers);
          const uint32_t ws[6] = {h0.x, h0.y, h0.z, h1.x, h1.y, h1.z};
          // the tile's lowest allowed token (cnt > 0 bits)
          uint32_t first = kHeadTileTokens;
#pragma unroll
          for (int u = 5; u >= 0; --u) {
            if (ws[u] != 0u) first = u * 32u + static_cast<uint32_t>(__builtin_ctz(ws[u]));
          }
          const uint32_t flags =
              ordinary ? 0u : (finite ? kTileRescoreAll | kTileCrowded : kTileRescoreAll);
          reinterpret_cast<uint4*>(&rec)[0] = uint4{__float_as_uint(L), flags, tok0 + first, lo};
          reinterpret_cast<uint4*>(&rec)[1] =
              uint4{lo, cnt, ordinary ? total : 0u, __float_as_uint(G + bs)};
          if (ordinary) {
            uint32_t k = 0u;
            uint32_t left = members;
            while (left != 0u) {
              const uint32_t u = static_cast<uint32_t>(__builtin_ctz(left));
              left &= left - 1u;
              // half u / 16, column u % 16, block of the half glj
              const uint32_t off = ((u / 16u) * kTBw + glj[s * kEpiRow + u]) * 16u + (u % 16u);
              const float v = r1[u];
              // list position: lo + the allowed tokens below off
              uint32_t pos = tok0 + off;
              if (kind == kSlotList) {
                uint32_t rank = 0u;
#pragma unroll
                for (uint32_t t = 0; t < 6u; ++t) {
                  const uint32_t below = off >= (t + 1u) * 32u ? 0xFFFFFFFFu
                                         : (off > t * 32u ? (1u << (off - t * 32u)) - 1u : 0u);
                  rank += static_cast<uint32_t>(__popc(ws[t] & below));
                }
                pos = lo + rank;
              }
              rec.m[k] = TileMember{tok0 + off, pos, v - bs, v + bs};
              ++k;
            }
          }
        }
      }
      __syncthreads();
      store_records(tile);
    }
  };
  if (copier) {
    copy_tiles();
    return;
  }
  switch (nact) {
    case 8: mfma_tiles.template operator()<8>(); break;
    case 7: mfma_tiles.template operator()<7>(); break;
    case 6: mfma_tiles.template operator()<6>(); break;
    case 5: mfma_tiles.template operator()<5>(); break;
    case 4: mfma_tiles.template operator()<4>(); break;
    case 3: mfma_tiles.template operator()<3>(); break;
    case 2: mfma_tiles.template operator()<2>(); break;
    case 1: mfma_tiles.template operator()<1>(); break;
    default: mfma_tiles.template operator()<0>(); break;
  }
}

}  // namespace

hipError_t launch_dense(const DenseArgs& args, hipStream_t stream) {
  if (args.H % 32u != 0 || args.H / 32u < static_cast<uint32_t>(kStages) || args.groups < 8u ||
      args.groups % 8u != 0 || args.z_hi == nullptr || args.spans == nullptr) {
    return hipErrorInvalidValue;
  }
  // every slot needs a panel of this launch: a workgroup past its XCD's
  // panels would return without writing its records and fb_map entries,
  // and the finalize would read stale records
  if (static_cast<uint64_t>(args.fb_m) + args.rows >
      static_cast<uint64_t>(args.groups / 8u) * kDensePanelSlots) {
    return hipErrorInvalidValue;
  }
  const uint32_t lds = dense_lds_bytes();
  hipLaunchKernelGGL(dense_kernel, dim3(args.groups), dim3(kThreads), lds, stream, args);
  return hipGetLastError();
}

}  // namespace mf
