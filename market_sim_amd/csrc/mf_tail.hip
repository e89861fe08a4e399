// The decode tail on gfx950 (mf_decode_tail_f16):
//
//   K1 tail_norm_kernel      final RMSNorm in the reference order, per-row
//                            metadata (list, kind), FP16 hi/lo split (all
//                            rows for the MFMA gather; the unrestricted rows
//                            again as the MFMA head's panel); presets the
//                            outputs of invalid and unrestricted rows
//   K2 gather_kernel         streams the allowed embedding rows of one tile
//                            (a chunk of one row's list) and writes a tile
//                            record: the candidates whose [g - b, g + b]
//                            interval reaches the tile's best lower bound
//   (K4 vocab_head_kernel, mf_mfma.hip, writes the same records for
//    unrestricted rows)
//   K3 finalize_kernel       per row: merges tile records, rescores the
//                            surviving candidates in the reference order,
//                            selects (greedy.cu rules), advances the DFA
//
// K2 carries no atomics and no reference-order work, so it is a pure stream
// of embedding rows; the serial reference-order chains live in K1 and K3,
// where every row runs in parallel.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"
#include "mf_finalize.hpp"
#include "mf_plan.hpp"
#include "mf_prep.hpp"

namespace mf {
namespace {

constexpr int kThreads = 256;

// Workgroup i < items runs prep item i (mf_prep.hpp): row i < rows, else
// slot i - rows of the MFMA head's panel, with its first wave.  With a range
// index, workgroup items + r indexes row r's list for the table pass with
// all kWalkWaves waves.
__global__ __launch_bounds__(kWalkWaves * kWave) void tail_norm_kernel(TailNormArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ float inverse_shared;
  const uint32_t items = a.rows + (a.fb_panel != nullptr ? a.fb_m : 0u);
  const uint32_t wave = threadIdx.x / kWave;
  if (blockIdx.x < items) {
    if (wave == 0) {
      prep_item(a, blockIdx.x, lds, &inverse_shared, true);
    }
    return;
  }
  const uint32_t r = blockIdx.x - items;
  if (a.dense_spans != nullptr) {
    dense_walk(a, r, reinterpret_cast<uint32_t*>(lds));
    return;
  }
  const RangeLds L = RangeLds::at(reinterpret_cast<uint32_t*>(lds), a.ranges);
  const RangeRow w = range_row(a, r);
  if (!w.indexed) {
    if (threadIdx.x == 0) a.row_tiles[r] = 0u;
    return;
  }
  range_walk(a, w, L, wave);
  __syncthreads();
  range_end(a, r, w, L);
}

// The dense head's rows, after the norm launch.  The indexed lists
// (dense_flag) are ranked by length (longest first, then by row); the head
// takes the D longest, D filling whole panels of kDensePanelSlots slots
// after the dense_fb unrestricted rows: the room the unrestricted rows leave
// in their panels (which read the table anyway) is filled for free, and a
// further panel is added only while the lists it would take hold at least
// dense_panel_ids ids (a panel's pass over the table costs about as much
// as gathering that many candidate rows).  One workgroup of kChooseThreads;
// dynamic LDS: dense_sort 4-byte keys, dense_sort the power of two >= rows.
// Up to kChooseThreads candidates are ranked by counting (thread i counts
// the keys above key i and stores it at that rank: one barrier), more by a
// bitonic sort (a barrier per stage).
constexpr int kChooseThreads = 1024;
__global__ __launch_bounds__(kChooseThreads) void dense_choose_kernel(TailNormArgs a) {
  // 32-bit keys (count << 13) | (8191 - row): descending order is longest
  // first, then by row (rows < 8192, counts < 2^19 here), all distinct
  extern __shared__ __align__(16) uint32_t keys[];
  constexpr uint32_t kChooseWaves = kChooseThreads / kWave;
  __shared__ uint32_t wave_part[kChooseWaves];
  __shared__ uint64_t wave_ids[kChooseWaves];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  // the candidates, compacted in row order: thread segments and a block
  // scan (a segment's flags and counts loaded together)
  const uint32_t per = (a.rows + kChooseThreads - 1u) / kChooseThreads;
  const uint32_t r0 = tid * per < a.rows ? tid * per : a.rows;
  const uint32_t r1 = r0 + per < a.rows ? r0 + per : a.rows;
  uint32_t local = 0u;
  // (rows <= kChooseThreads, the common case: the thread's row's flag and
  // count in one round trip, kept for the compaction)
  const bool one = per == 1u && r0 < r1;
  const uint32_t flag0 = one ? a.dense_flag[r0] : 0u;
  const uint32_t count0 = one ? a.row_meta[r0].count : 0u;
  if (one) {
    local = flag0 != 0u ? 1u : 0u;
  } else {
    for (uint32_t r = r0; r < r1; ++r) local += a.dense_flag[r] != 0u ? 1u : 0u;
  }
  uint32_t incl = local;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), d));
    if (static_cast<int>(lane) >= d) incl += o;
  }
  if (lane == kWave - 1) wave_part[wave] = incl;
  __syncthreads();
  uint32_t at = incl - local;
  uint32_t nc = 0u;
  for (uint32_t w = 0; w < kChooseWaves; ++w) {
    at += w < wave ? wave_part[w] : 0u;
    nc += wave_part[w];
  }
  if (nc == 0u) return;
  if (one) {
    if (flag0 != 0u) keys[at] = (count0 << 13) | (8191u - r0);
  } else {
    for (uint32_t r = r0; r < r1; ++r) {
      const uint32_t count = a.row_meta[r].count;
      if (a.dense_flag[r] != 0u) keys[at++] = (count << 13) | (8191u - r);
    }
  }
  uint32_t n2 = 1u;
  while (n2 < nc) n2 <<= 1;
  for (uint32_t i = nc + tid; i < n2; i += kChooseThreads) keys[i] = 0u;
  __syncthreads();
  if (nc <= static_cast<uint32_t>(kChooseThreads)) {
    // rank of key tid: the keys above it (every lane reads the same four
    // keys at a time, then the last nc % 4 one by one)
    const uint32_t mine = tid < nc ? keys[tid] : 0u;
    uint32_t rank = 0u;
    const uint4* k4 = reinterpret_cast<const uint4*>(keys);
    for (uint32_t i = 0; i < nc / 4u; ++i) {
      const uint4 v = k4[i];
      rank += (v.x > mine ? 1u : 0u) + (v.y > mine ? 1u : 0u) + (v.z > mine ? 1u : 0u) +
              (v.w > mine ? 1u : 0u);
    }
    for (uint32_t i = nc & ~3u; i < nc; ++i) rank += keys[i] > mine ? 1u : 0u;
    __syncthreads();
    if (tid < nc) keys[rank] = mine;
    __syncthreads();
  } else {
    // bitonic sort, descending: n2 / 2 compare-exchanges per stage
    for (uint32_t k = 2; k <= n2; k <<= 1) {
      for (uint32_t j = k >> 1; j > 0; j >>= 1) {
        for (uint32_t p = tid; p < n2 / 2u; p += kChooseThreads) {
          const uint32_t i = (p / j) * 2u * j + (p % j);
          const uint32_t l = i + j;
          const uint32_t x = keys[i];
          const uint32_t y = keys[l];
          const bool descending = (i & k) == 0u;
          if (descending ? x < y : x > y) {
            keys[i] = y;
            keys[l] = x;
          }
        }
        __syncthreads();
      }
    }
  }
  // D: the free room of the unrestricted rows' panels, then whole panels
  // while their lists hold enough ids
  const uint32_t fb = a.dense_fb;
  const uint32_t fb_panels = (fb + kDensePanelSlots - 1u) / kDensePanelSlots;
  uint32_t D = fb_panels * kDensePanelSlots - fb;
  D = D < nc ? D : nc;
  while (D < nc) {
    const uint32_t end = D + kDensePanelSlots < nc ? D + kDensePanelSlots : nc;
    uint64_t ids = 0u;
    for (uint32_t i = D + tid; i < end; i += kChooseThreads) ids += keys[i] >> 13;
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) {
      const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(ids & 0xFFFFFFFFu), m));
      const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(ids >> 32), m));
      ids += (static_cast<uint64_t>(hi) << 32) | lo;
    }
    if (lane == 0) wave_ids[wave] = ids;
    __syncthreads();
    uint64_t total = 0u;
    for (uint32_t w = 0; w < kChooseWaves; ++w) total += wave_ids[w];
    __syncthreads();
    if (total < a.dense_panel_ids) break;
    D = end;
  }
  for (uint32_t i = tid; i < D; i += kChooseThreads) {
    const uint32_t r = 8191u - (keys[i] & 8191u);
    a.row_meta[r].kind |= kRowDense;
  }
}

// ---------------------------------------------------------------------------
// K2: gather
// ---------------------------------------------------------------------------

struct GatherShared {
  float sc[kGatherTileMax];
  float bd[kGatherTileMax];
  uint32_t tk[kGatherTileMax];
  uint32_t bad;
};

__device__ __forceinline__ float half_lane(const uint4& q, int k) {
  const uint16_t* h = reinterpret_cast<const uint16_t*>(&q);
  return half_to_float(h[k]);
}

// Fast scores, H known at compile time: G lanes per candidate, each lane
// owning L = H / (8 G) 16-byte slices (slice i*G + lane: a group reads G*16
// contiguous bytes per load); U candidates per group in flight.
template <int H, int G, int U>
__device__ void gather_scores_vec(const GatherArgs& a, const float* ys, GatherShared& sh,
                                  uint32_t n) {
  constexpr int L = H / (8 * G);
  constexpr int kGroups = kThreads / G;
  static_assert(L * 8 * G == H, "H must split into 16-byte lane slices");
  const int lane = threadIdx.x % G;
  const int grp = threadIdx.x / G;
  float yv[L][8];
#pragma unroll
  for (int i = 0; i < L; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) yv[i][k] = ys[(i * G + lane) * 8 + k];
  }
  for (uint32_t base = 0; base < n; base += kGroups * U) {
    uint4 ev[U][L];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t c = base + u * kGroups + grp;
      ok[u] = c < n;
      const uint32_t t = ok[u] ? sh.tk[c] : 0u;
      const uint4* row = reinterpret_cast<const uint4*>(a.emb + static_cast<uint64_t>(t) * H) + lane;
#pragma unroll
      for (int i = 0; i < L; ++i) ev[u][i] = ok[u] ? row[i * G] : uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float acc = 0.0f;
      float acca = 0.0f;
#pragma unroll
      for (int i = 0; i < L; ++i) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float e = half_lane(ev[u][i], k);
          acc = __builtin_fmaf(e, yv[i][k], acc);
          acca = __builtin_fmaf(__builtin_fabsf(e), __builtin_fabsf(yv[i][k]), acca);
        }
      }
#pragma unroll
      for (int m = G / 2; m > 0; m >>= 1) {
        acc += __shfl_xor(acc, m, G);
        acca += __shfl_xor(acca, m, G);
      }
      const uint32_t c = base + u * kGroups + grp;
      if (lane == 0 && ok[u]) {
        sh.sc[c] = acc;
        sh.bd[c] = __builtin_fmaf(a.coef, acca, a.slack);
      }
    }
  }
}

// Fast scores for any H: one wave per candidate, element-strided.
__device__ void gather_scores_generic(const GatherArgs& a, const float* ys, GatherShared& sh,
                                      uint32_t n) {
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  for (uint32_t c = w; c < n; c += kThreads / kWave) {
    const uint16_t* row = a.emb + static_cast<uint64_t>(sh.tk[c]) * a.H;
    float acc = 0.0f;
    float acca = 0.0f;
    for (uint32_t f = lane; f < a.H; f += kWave) {
      const float e = half_to_float(row[f]);
      acc = __builtin_fmaf(e, ys[f], acc);
      acca = __builtin_fmaf(__builtin_fabsf(e), __builtin_fabsf(ys[f]), acca);
    }
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) {
      acc += __shfl_xor(acc, m);
      acca += __shfl_xor(acca, m);
    }
    if (lane == 0) {
      sh.sc[c] = acc;
      sh.bd[c] = __builtin_fmaf(a.coef, acca, a.slack);
    }
  }
}

// Scores already computed by the MFMA projection (the full-head comparator).
__device__ void gather_scores_lookup(const GatherArgs& a, uint32_t r, GatherShared& sh,
                                     uint32_t n) {
  const float* srow = a.scores + static_cast<uint64_t>(r) * a.V;
  const float yn = a.row_norm[r];
  const float row_slack = a.row_slack[r];
  for (uint32_t c = threadIdx.x; c < n; c += kThreads) {
    const uint32_t t = sh.tk[c];
    sh.sc[c] = srow[t];
    sh.bd[c] = __builtin_fmaf(a.tok_norm[t], __builtin_fmaf(a.coef, yn, a.coef2), row_slack);
  }
}

// One tile: candidates [k*tile, k*tile + n) of row r's list.  All threads
// call; wave 0 writes the record.  ys keeps row `staged`'s hidden vector.
template <ScoreSource kSrc, int kH, int kG>
__device__ void gather_tile(const GatherArgs& a, uint32_t r, uint32_t k, uint32_t list_begin,
                            uint32_t count, bool virtual_list, float* ys, GatherShared& sh,
                            uint32_t& staged) {
  constexpr bool lookup = kSrc == ScoreSource::kLookup;
  const uint32_t begin = k * a.tile;
  const uint32_t n = count - begin < a.tile ? count - begin : a.tile;
  __syncthreads();  // the previous tile is done with sh and ys
  if constexpr (!lookup) {
    if (staged != r) {
      for (uint32_t f = threadIdx.x; f < a.H; f += kThreads) {
        ys[f] = a.y[static_cast<uint64_t>(r) * a.H + f];
      }
      staged = r;
    }
  }
  uint32_t bad = 0u;
  for (uint32_t c = threadIdx.x; c < n; c += kThreads) {
    const uint32_t t = virtual_list ? begin + c : a.tokens[list_begin + begin + c];
    bad |= t >= a.V ? 1u : 0u;
    sh.tk[c] = t < a.V ? t : 0u;
  }
  const bool invalid = __syncthreads_or(bad) != 0;
  if (!invalid) {
    if constexpr (lookup) {
      gather_scores_lookup(a, r, sh, n);
    } else if constexpr (kH > 0) {
      gather_scores_vec<kH, kG, 2>(a, ys, sh, n);
    } else {
      gather_scores_generic(a, ys, sh, n);
    }
  }
  __syncthreads();
  if (threadIdx.x >= kWave) return;

  // wave 0 summarizes the tile
  const uint32_t lane = threadIdx.x;
  TileRecord* rec = a.records + static_cast<uint64_t>(r) * a.max_tiles + k;
  uint32_t fin = 1u;
  float lo = -__builtin_huge_valf();
  float up = -__builtin_huge_valf();
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
  for (uint32_t c = lane; c < n; c += kWave) {
    const float g = sh.sc[c];
    const float b = sh.bd[c];
    fin &= (__builtin_isfinite(g) && __builtin_isfinite(b) && b < 0x1p100f) ? 1u : 0u;
    lo = __builtin_fmaxf(lo, g - b);
    up = __builtin_fmaxf(up, g + b);
    if (sh.tk[c] < mt) {
      mt = sh.tk[c];
      mp = begin + c;
    }
  }
  const bool all_finite = wave_sum_u32(fin ^ 1u) == 0u;
  const float L = wave_max(lo);
  const float U = wave_max(up);
  wave_min_token(mt, mp);
  // members: candidates with g + b >= L, ranked in list order by ballot
  const bool ordinary = all_finite && !invalid;
  uint32_t total = 0u;
  for (uint32_t c0 = 0; c0 < n; c0 += kWave) {
    const uint32_t c = c0 + lane;
    const bool member = ordinary && c < n && sh.sc[c] + sh.bd[c] >= L;
    const uint64_t mask = __ballot(member);
    if (member) {
      const uint32_t rank = total + __popcll(mask & ((1ull << lane) - 1ull));
      if (rank < kTileMembers) {
        const float g = sh.sc[c];
        const float b = sh.bd[c];
        rec->m[rank] = TileMember{sh.tk[c], begin + c, g - b, g + b};
      }
    }
    total += __popcll(mask);
  }
  if (lane == 0) {
    uint32_t flags = 0u;
    if (invalid) flags |= kTileInvalid;
    if (!invalid && (!all_finite || total > kTileMembers)) flags |= kTileRescoreAll;
    if (!invalid && all_finite && total > kTileMembers) flags |= kTileCrowded;
    rec->best_lower = L;
    rec->upper_max = U;
    rec->flags = flags;
    rec->min_token = mt;
    rec->min_pos = mp;
    rec->begin = begin;
    rec->count = n;
    rec->n_members = flags ? 0u : total;
  }
}

// Grid mode (any number of rows): blockIdx.x = k * rows + r.
template <ScoreSource kSrc, int kH, int kG>
__global__ __launch_bounds__(kThreads) void gather_kernel(GatherArgs a) {
  extern __shared__ __align__(16) float ys[];
  __shared__ GatherShared sh;
  const uint32_t r = blockIdx.x % a.rows;
  const uint32_t k = blockIdx.x / a.rows;
  const RowMeta meta = a.row_meta[r];
  if (!row_gathered(meta, kSrc == ScoreSource::kLookup) || k * a.tile >= meta.count) return;
  uint32_t staged = kInvalidToken;
  gather_tile<kSrc, kH, kG>(a, r, k, meta.list_begin, meta.count,
                            (meta.kind & kRowUnrestricted) != 0, ys, sh, staged);
}

// Planned mode (rows <= kPlanRowsMax): the tile plan (mf_plan.hpp), then
// each workgroup walks its contiguous range [W*b/G, W*(b+1)/G) of the W
// tiles -- no idle workgroups, and consecutive tiles of one row reuse the
// staged hidden vector.
template <ScoreSource kSrc, int kH, int kG>
__global__ __launch_bounds__(kThreads) void gather_planned_kernel(GatherArgs a) {
  extern __shared__ __align__(16) float ys[];
  __shared__ GatherShared sh;
  __shared__ TilePlan<kThreads> plan;
  const uint64_t W = plan_tiles<kThreads>(a.row_meta, a.rows, a.tile,
                                          kSrc == ScoreSource::kLookup, plan);
  const uint64_t G = gridDim.x;
  const uint32_t w0 = static_cast<uint32_t>(W * blockIdx.x / G);
  const uint32_t w1 = static_cast<uint32_t>(W * (blockIdx.x + 1) / G);
  if (w0 >= w1) return;
  uint32_t r = plan_row_of<kThreads>(plan, a.rows, w0);
  uint32_t staged = kInvalidToken;
  for (uint32_t w = w0; w < w1; ++w) {
    while (plan.prefix[r + 1] <= w) ++r;
    gather_tile<kSrc, kH, kG>(a, r, w - plan.prefix[r], plan.begin[r], plan.count[r],
                              (plan.kind[r] & kRowUnrestricted) != 0, ys, sh, staged);
  }
}

// ---------------------------------------------------------------------------
// K3: finalize (one wave per row; the per-row work is finalize_row in
// mf_finalize.hpp)
// ---------------------------------------------------------------------------

constexpr uint32_t kStage = 8;  // embedding rows staged in LDS per rescore pass
// The rescoring keeps its operands in registers (rescore_segmented) when H
// is a multiple of kChainSeg of at most kWave segments and the table is
// 16-byte aligned; LDS then stages one embedding row (the all-NaN rows'
// lowest id) instead of kStage, which lets more rows share a compute unit.
__host__ __device__ inline uint32_t finalize_stage_rows(uint32_t H, const void* emb) {
  const bool segmented = H % kChainSeg == 0u && H <= kChainSeg * kWave &&
                         (reinterpret_cast<uintptr_t>(emb) & 15u) == 0;
  return segmented ? 1u : kStage;
}
constexpr uint32_t kCandMax = 2 * kWave * kTileMembers;

template <uint32_t kYRegs>
__global__ __launch_bounds__(kWave) void finalize_kernel(FinalizeArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ uint32_t cand_token[kCandMax];
  __shared__ uint32_t cand_pos[kCandMax];
  __shared__ FinalizeWords words;
  const FinalizeLds L{lds, reinterpret_cast<uint16_t*>(lds + a.H), finalize_stage_rows(a.H, a.emb),
                      cand_token, cand_pos, kCandMax, &words};
  const uint32_t r = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  const RowMeta meta = a.row_meta[r];
  const float* yrow = a.y + static_cast<uint64_t>(r) * a.H;
  if constexpr (kYRegs > 0) {
    // rows of at most 256 kYRegs features: the hidden vector's loads stay
    // in flight in registers while the record headers load; stored to LDS
    // before the first rescore
    float4 yv[kYRegs];
    const uint32_t n4 = a.H / 4u;
#pragma unroll
    for (uint32_t u = 0; u < kYRegs; ++u) {
      const uint32_t q = lane + u * kWave;
      yv[u] = q < n4 ? reinterpret_cast<const float4*>(yrow)[q] : float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    finalize_row(a, r, meta, L, [&]() {
#pragma unroll
      for (uint32_t u = 0; u < kYRegs; ++u) {
        const uint32_t q = lane + u * kWave;
        if (q < n4) reinterpret_cast<float4*>(L.ys)[q] = yv[u];
      }
    });
  } else {
    if ((a.H & 3u) == 0) {
      copy16_to_lds<4>(reinterpret_cast<uint4*>(L.ys), reinterpret_cast<const uint4*>(yrow), a.H / 4,
                       lane, kWave);
    } else {
      for (uint32_t f = lane; f < a.H; f += kWave) L.ys[f] = yrow[f];
    }
    finalize_row(a, r, meta, L, []() {});
  }
}

} // namespace

hipError_t launch_tail_norm(const TailNormArgs& args, hipStream_t stream) {
  const size_t norm_lds = 3u * static_cast<size_t>(args.H) * sizeof(float);
  const size_t walk_lds =
      args.range_index != nullptr ? range_lds_words(args.ranges) * sizeof(uint32_t)
      : args.dense_spans != nullptr ? dense_lds_words(args.ranges) * sizeof(uint32_t)
                                    : 0u;
  const uint32_t slots = args.fb_panel != nullptr ? args.fb_m : 0u;
  const uint32_t walks = args.range_index != nullptr || args.dense_spans != nullptr ? args.rows : 0u;
  const uint32_t threads = walks > 0 ? kWalkWaves * kWave : kWave;
  hipLaunchKernelGGL(tail_norm_kernel, dim3(args.rows + slots + walks), dim3(threads),
                     norm_lds > walk_lds ? norm_lds : walk_lds, stream, args);
  if (args.dense_spans != nullptr) {
    hipLaunchKernelGGL(dense_choose_kernel, dim3(1), dim3(kChooseThreads),
                       static_cast<size_t>(args.dense_sort) * sizeof(uint32_t), stream, args);
  }
  return hipGetLastError();
}

template <ScoreSource kSrc, int kH, int kG>
static void launch_gather_variant(const GatherArgs& a, hipStream_t stream) {
  const size_t lds = kSrc == ScoreSource::kLookup ? 0 : static_cast<size_t>(a.H) * sizeof(float);
  const uint64_t slots = static_cast<uint64_t>(a.rows) * a.max_tiles;
  if (a.rows <= kPlanRowsMax && a.groups > 0) {
    // persistent grid: compute units x resident workgroups of this variant
    static int resident = 0;
    if (resident == 0) {
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &n, reinterpret_cast<const void*>(gather_planned_kernel<kSrc, kH, kG>), kThreads,
              lds) != hipSuccess || n <= 0) {
        n = 2;
      }
      resident = n;
    }
    const uint64_t want = static_cast<uint64_t>(a.groups) * static_cast<uint64_t>(resident);
    const uint32_t g = static_cast<uint32_t>(slots < want ? slots : want);
    hipLaunchKernelGGL((gather_planned_kernel<kSrc, kH, kG>), dim3(g), dim3(kThreads), lds,
                       stream, a);
  } else {
    hipLaunchKernelGGL((gather_kernel<kSrc, kH, kG>), dim3(static_cast<uint32_t>(slots)),
                       dim3(kThreads), lds, stream, a);
  }
}

hipError_t launch_gather(ScoreSource source, const GatherArgs& a, hipStream_t stream) {
  const bool aligned = (reinterpret_cast<uintptr_t>(a.emb) & 15u) == 0;
  if (source == ScoreSource::kMfma) return launch_gather_mfma(a, stream);
  if (source == ScoreSource::kLookup) {
    launch_gather_variant<ScoreSource::kLookup, 0, 64>(a, stream);
  } else if (a.H == 576 && aligned) {
    launch_gather_variant<ScoreSource::kDotF32, 576, 8>(a, stream);
  } else if (a.H == 2048 && aligned) {
    launch_gather_variant<ScoreSource::kDotF32, 2048, 32>(a, stream);
  } else {
    launch_gather_variant<ScoreSource::kDotF32, 0, 64>(a, stream);
  }
  return hipGetLastError();
}

hipError_t launch_finalize(const FinalizeArgs& a, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(a.H) * sizeof(float) +
                     static_cast<size_t>(finalize_stage_rows(a.H, a.emb)) * a.H * sizeof(uint16_t);
  if (a.H % 4u == 0 && a.H <= 4u * kWave * 4u) {
    hipLaunchKernelGGL(finalize_kernel<4>, dim3(a.rows), dim3(kWave), lds, stream, a);
  } else if (a.H % 4u == 0 && a.H <= 4u * kWave * 8u) {
    hipLaunchKernelGGL(finalize_kernel<8>, dim3(a.rows), dim3(kWave), lds, stream, a);
  } else {
    hipLaunchKernelGGL(finalize_kernel<0>, dim3(a.rows), dim3(kWave), lds, stream, a);
  }
  return hipGetLastError();
}

} // namespace mf
