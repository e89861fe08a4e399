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
#include "mf_plan.hpp"

namespace mf {
namespace {

constexpr int kThreads = 256;

// Sum of squares in the reference order (operators.cpp:527-531): every square
// rounded (lanes compute them in parallel into sq[]), then added in column
// order by one lane.  Blocks of 16 values alternate between two register
// sets: the LDS reads of block i + 1 are issued before the adds of block i
// (sched_barrier keeps the scheduler from sinking them to their use, which
// would pay an LDS round trip per block).
__device__ __forceinline__ void load16(const float4* q, uint32_t i, float4 (&v)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = q[4 * i + k];
}
__device__ __forceinline__ float add16(float s, const float4 (&v)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    s = s + v[k].x;
    s = s + v[k].y;
    s = s + v[k].z;
    s = s + v[k].w;
  }
  return s;
}
__device__ float sequential_sum(const float* sq, uint32_t H) {
  float s = 0.0f;
  uint32_t c = 0;
  if ((H & 31u) == 0) {
    const float4* q = reinterpret_cast<const float4*>(sq);
    const uint32_t n16 = H / 16;  // even
    float4 a[4], b[4];
    load16(q, 0, a);
    for (uint32_t i = 0; i < n16; i += 2) {
      load16(q, i + 1, b);
      __builtin_amdgcn_sched_barrier(0);
      s = add16(s, a);
      __builtin_amdgcn_sched_barrier(0);
      load16(q, i + 2 < n16 ? i + 2 : i, a);
      __builtin_amdgcn_sched_barrier(0);
      s = add16(s, b);
      __builtin_amdgcn_sched_barrier(0);
    }
    c = H;
  }
  for (; c < H; ++c) s = s + sq[c];
  return s;
}

// Workgroup r < rows normalizes row r; workgroup rows + j normalizes row
// fb_rows[j] again for slot j of the MFMA head's panel (the same code on the
// same data, so the same bits) and writes only the slot.
__global__ __launch_bounds__(kWave) void tail_norm_kernel(TailNormArgs a) {
  extern __shared__ __align__(16) float lds[];
  float* xs = lds;
  float* sq = lds + a.H;
  __shared__ float inverse_shared;
  const bool slot = blockIdx.x >= a.rows;
  const uint32_t j = blockIdx.x - a.rows;  // the slot (slot workgroups)
  uint64_t r = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  const uint32_t H = a.H;
  if (slot) {
    r = a.fb_rows[j];
    if (r >= a.rows) {
      if (lane == 0) {
        a.fb_slot_row[j] = kInvalidToken;
        a.fb_slot_norm[j] = 0.0f;
      }
      return;
    }
  }
  // the row's state first: its list offsets depend on it
  uint32_t s = 0u;
  if (!slot && lane == 0) s = a.row_state[r];
  float* ws = lds + 2u * H;  // weight (when given)
  const bool weighted = a.weight != nullptr;
  if ((H & 3u) == 0) {
    // x and the weight: four float4 loads of each per lane in flight before
    // the LDS stores
    constexpr uint32_t kBatch = 4;
    const float4* x4 = reinterpret_cast<const float4*>(a.x + r * H);
    const float4* w4 = reinterpret_cast<const float4*>(a.weight);
    const uint32_t n = H / 4;
    for (uint32_t base = lane; base < n; base += kWave * kBatch) {
      float4 v[kBatch];
      float4 wv[kBatch];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t q = base + u * kWave;
        v[u] = q < n ? x4[q] : float4{0.0f, 0.0f, 0.0f, 0.0f};
        wv[u] = (weighted && q < n) ? w4[q] : float4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t q = base + u * kWave;
        if (q < n) {
          reinterpret_cast<float4*>(xs)[q] = v[u];
          reinterpret_cast<float4*>(sq)[q] =
              float4{v[u].x * v[u].x, v[u].y * v[u].y, v[u].z * v[u].z, v[u].w * v[u].w};
          if (weighted) reinterpret_cast<float4*>(ws)[q] = wv[u];
        }
      }
    }
  } else {
    for (uint32_t c = lane; c < H; c += kWave) {
      const float v = a.x[r * H + c];
      xs[c] = v;
      sq[c] = v * v;
      if (weighted) ws[c] = a.weight[c];
    }
  }
  __syncthreads();
  RowMeta meta{0u, 0u, 0u, kRowInvalid};
  if (lane == 0) {
    // the offsets loads are in flight during the serial sum
    uint32_t b = 0u, e = 0u;
    if (!slot && s < a.states) {
      b = a.offsets[s];
      e = a.offsets[s + 1];
    }
    if (weighted) {
      const float sum_squares = sequential_sum(sq, H);
      const float mean = div_rn(sum_squares, static_cast<float>(H));
      inverse_shared = div_rn(1.0f, sqrt_rn(mean + a.epsilon));
    }
    if (!slot) {
      meta.state = s;
      if (s == kStateUnrestricted) {
        meta.kind = kRowUnrestricted;
        meta.count = a.V;
      } else if (s < a.states && e > b && e <= a.nnz && e - b <= a.max_count) {
        meta = RowMeta{b, e - b, s, kRowRestricted};
      }
      a.row_meta[r] = meta;
      if (meta.kind != kRowRestricted) {
        // invalid rows keep these; unrestricted rows are overwritten by the
        // finalize kernel when the MFMA head was given them
        a.out_token[r] = kInvalidToken;
        if (a.out_score != nullptr) a.out_score[r] = __builtin_nanf("");
        if (a.out_next != nullptr) a.out_next[r] = kInvalidToken;
      }
      if (a.fb_map != nullptr) a.fb_map[r] = kInvalidToken;
    }
  }
  __syncthreads();
  const float inverse = inverse_shared;
  const bool split = a.y_hi != nullptr;
  // slot workgroups: the slot's [hi | lo] rows of the panel
  uint16_t* panel_hi = nullptr;
  if (slot) {
    panel_hi = a.fb_panel + static_cast<uint64_t>(j / kPanelRows) * (panel_tile_bytes(H) / 2u) +
               static_cast<uint64_t>(j % kPanelRows) * 2u * (H + kPanelPad);
  }
  float norm_sq = 0.0f;
  for (uint32_t c = lane; c < H; c += kWave) {
    float v = xs[c];
    if (weighted) {
      const float scaled = v * inverse;
      v = scaled * ws[c];
    }
    norm_sq = __builtin_fmaf(v, v, norm_sq);
    const _Float16 hi = static_cast<_Float16>(v);
    const uint16_t lo = float_to_half_rne(v - static_cast<float>(hi));
    if (slot) {
      panel_hi[c] = __builtin_bit_cast(uint16_t, hi);
      panel_hi[H + kPanelPad + c] = lo;
    } else {
      a.y[r * H + c] = v;
      if (split) {
        a.y_hi[r * H + c] = __builtin_bit_cast(uint16_t, hi);
        a.y_lo[r * H + c] = lo;
      }
    }
  }
  norm_sq = wave_sum_f32(norm_sq);
  if (lane == 0) {
    // FP32 sum of H squares is within a relative H 2^-24 of the exact value;
    // the factor covers that and the sqrt for any H <= 2^16
    const float bound = __fsqrt_rn(norm_sq) * (1.0f + 0x1p-7f);
    if (slot) {
      a.fb_slot_norm[j] = bound;
      a.fb_slot_row[j] = static_cast<uint32_t>(r);
    } else {
      a.row_norm[r] = bound;
    }
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
  for (uint32_t c = threadIdx.x; c < n; c += kThreads) {
    const uint32_t t = sh.tk[c];
    sh.sc[c] = srow[t];
    sh.bd[c] = __builtin_fmaf(a.tok_norm[t], __builtin_fmaf(a.coef, yn, a.coef2), a.slack);
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
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
  for (uint32_t c = lane; c < n; c += kWave) {
    const float g = sh.sc[c];
    const float b = sh.bd[c];
    fin &= (__builtin_isfinite(g) && __builtin_isfinite(b) && b < 0x1p100f) ? 1u : 0u;
    lo = __builtin_fmaxf(lo, g - b);
    if (sh.tk[c] < mt) {
      mt = sh.tk[c];
      mp = begin + c;
    }
  }
  const bool all_finite = wave_sum_u32(fin ^ 1u) == 0u;
  const float L = wave_max(lo);
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
    rec->best_lower = L;
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
// K3: finalize
// ---------------------------------------------------------------------------

constexpr int kStage = 8;  // embedding rows staged in LDS per rescore pass

// Reference-order chain over LDS-resident FP32 y and FP16 row (see
// canonical_dot): same arithmetic, LDS reads issued a vector ahead.
template <bool kMulAdd>
__device__ __forceinline__ void chain_load(const uint4* e, const float4* y, uint32_t i,
                                           uint4 (&ev)[2], float4 (&yv)[4]) {
  ev[0] = e[2 * i];
  ev[1] = e[2 * i + 1];
#pragma unroll
  for (int k = 0; k < 4; ++k) yv[k] = y[4 * i + k];
}
template <bool kMulAdd>
__device__ __forceinline__ float chain16(float s, const uint4 (&ev)[2], const float4 (&yv)[4]) {
  const float yf[16] = {yv[0].x, yv[0].y, yv[0].z, yv[0].w, yv[1].x, yv[1].y, yv[1].z, yv[1].w,
                        yv[2].x, yv[2].y, yv[2].z, yv[2].w, yv[3].x, yv[3].y, yv[3].z, yv[3].w};
  const uint16_t* h = reinterpret_cast<const uint16_t*>(&ev[0]);
#pragma unroll
  for (int k = 0; k < 16; ++k) s = order_step<kMulAdd>(s, yf[k], half_to_float(h[k]));
  return s;
}

// One candidate's score in a reference order from LDS (the same arithmetic
// as canonical_dot).  Blocks of 16 features alternate between two register
// sets so that block i + 1's LDS reads are in flight during block i's chain.
template <bool kMulAdd>
__device__ float chain_lds(const float* ys, const uint16_t* row, uint32_t H) {
  float s = 0.0f;
  uint32_t f = 0;
  if ((H & 31u) == 0 && (reinterpret_cast<uintptr_t>(row) & 15u) == 0) {
    const uint4* e = reinterpret_cast<const uint4*>(row);
    const float4* y = reinterpret_cast<const float4*>(ys);
    const uint32_t n16 = H / 16;  // even
    uint4 ea[2], eb[2];
    float4 ya[4], yb[4];
    chain_load<kMulAdd>(e, y, 0, ea, ya);
    for (uint32_t i = 0; i < n16; i += 2) {
      chain_load<kMulAdd>(e, y, i + 1, eb, yb);
      __builtin_amdgcn_sched_barrier(0);
      s = chain16<kMulAdd>(s, ea, ya);
      __builtin_amdgcn_sched_barrier(0);
      chain_load<kMulAdd>(e, y, i + 2 < n16 ? i + 2 : i, ea, ya);
      __builtin_amdgcn_sched_barrier(0);
      s = chain16<kMulAdd>(s, eb, yb);
      __builtin_amdgcn_sched_barrier(0);
    }
    f = H;
  }
  for (; f < H; ++f) s = order_step<kMulAdd>(s, ys[f], half_to_float(row[f]));
  return s;
}

constexpr uint32_t kCandMax = 2 * kWave * kTileMembers;
constexpr uint32_t kRecBlock = 4;  // tile records per lane loaded together

struct FinalizeShared {
  uint32_t cand_token[kCandMax];
  uint32_t cand_pos[kCandMax];
  uint32_t n_cand;
  uint32_t token;
  uint32_t pos;
  float score;
  uint32_t need_score;
};

// Rescores candidates cand_token[0..n) of one row in the reference order,
// kStage rows at a time staged in LDS; returns the wave's best.
__device__ Best rescore_candidates(const FinalizeArgs& a, const float* ys, uint16_t* es,
                                   const FinalizeShared& sh, uint32_t n) {
  const uint32_t lane = threadIdx.x;
  const uint32_t H = a.H;
  Best best = best_identity();
  for (uint32_t base = 0; base < n; base += kStage) {
    const uint32_t m = n - base < kStage ? n - base : kStage;
    __syncthreads();
    if ((H & 7u) == 0) {
      // every row's pieces in flight before their stores (kStage rows of
      // H / 8 pieces over 64 lanes)
      constexpr uint32_t kBatch = 10;
      const uint32_t per = H / 8;
      const uint32_t total = m * per;
      for (uint32_t q0 = lane; q0 < total; q0 += kWave * kBatch) {
        uint4 v[kBatch];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
          const uint32_t q = q0 + u * kWave;
          const uint32_t j = q / per;
          v[u] = q < total
                     ? reinterpret_cast<const uint4*>(
                           a.emb + static_cast<uint64_t>(sh.cand_token[base + j]) * H)[q % per]
                     : uint4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
          const uint32_t q = q0 + u * kWave;
          if (q < total) reinterpret_cast<uint4*>(es + (q / per) * H)[q % per] = v[u];
        }
      }
    } else {
      for (uint32_t q = lane; q < m * H; q += kWave) {
        const uint32_t j = q / H;
        es[q] = a.emb[static_cast<uint64_t>(sh.cand_token[base + j]) * H + (q % H)];
      }
    }
    __syncthreads();
    if (lane < m) {
      const float s = a.order == 1 ? chain_lds<true>(ys, es + lane * H, H)
                                   : chain_lds<false>(ys, es + lane * H, H);
      best = best_of(best, best_leaf(s, sh.cand_token[base + lane], sh.cand_pos[base + lane]));
    }
  }
  return wave_best(best);
}

__global__ __launch_bounds__(kWave) void finalize_kernel(FinalizeArgs a) {
  extern __shared__ __align__(16) float lds[];
  float* ys = lds;                                            // H floats
  uint16_t* es = reinterpret_cast<uint16_t*>(lds + a.H);      // kStage rows
  __shared__ FinalizeShared sh;
  const uint32_t r = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  // the loads that need nothing else go first: the row's hidden vector, its
  // metadata and its MFMA-head slot
  if ((a.H & 3u) == 0) {
    copy16_to_lds<4>(reinterpret_cast<uint4*>(ys),
                     reinterpret_cast<const uint4*>(a.y + static_cast<uint64_t>(r) * a.H), a.H / 4,
                     lane, kWave);
  } else {
    for (uint32_t f = lane; f < a.H; f += kWave) ys[f] = a.y[static_cast<uint64_t>(r) * a.H + f];
  }
  const RowMeta meta = a.row_meta[r];
  const uint32_t fb_slot = a.fb_map != nullptr ? a.fb_map[r] : kInvalidToken;
  const TileRecord* recs;
  uint32_t ntiles;
  if (meta.kind & kRowRestricted) {
    recs = a.records + static_cast<uint64_t>(r) * a.max_tiles;
    ntiles = (meta.count + a.tile - 1) / a.tile;
  } else if ((meta.kind & kRowUnrestricted) && a.fb_records != nullptr) {
    const uint32_t m = fb_slot;
    if (m == kInvalidToken) return;
    recs = a.fb_records + static_cast<uint64_t>(m) * a.fb_tiles;
    ntiles = a.fb_tiles;
  } else if ((meta.kind & kRowUnrestricted) && a.lookup_unrestricted) {
    recs = a.records + static_cast<uint64_t>(r) * a.max_tiles;
    ntiles = (meta.count + a.tile - 1) / a.tile;
  } else {
    return;
  }
  const bool virtual_list = meta.kind & kRowUnrestricted;
  __syncthreads();
  // pass 1: validity, the best lower bound of ordinary tiles, lowest id
  uint32_t inv = 0u;
  uint32_t any_all = 0u;
  float lg = -__builtin_huge_valf();
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
  // Per tile the header (best_lower, flags, min_token, min_pos), the counts
  // (begin, count, n_members) and the first member, kRecBlock tiles per lane
  // loaded before any is used: one round trip per block.  A row of at most
  // kWave kRecBlock tiles (every gather row up to 16384 candidates, every
  // MFMA-head row up to 49152 tokens) keeps them in registers for the
  // member collection below.
  const bool resident = ntiles <= kWave * kRecBlock;
  uint4 h[kRecBlock];
  uint4 c[kRecBlock];
  TileMember m0[kRecBlock];
  for (uint32_t base = 0; base < ntiles; base += kWave * kRecBlock) {
#pragma unroll
    for (uint32_t u = 0; u < kRecBlock; ++u) {
      const uint32_t t = base + u * kWave + lane;
      const bool in = t < ntiles;
      // past the row's tiles: an empty ordinary tile (no members, lowest
      // bound, no token)
      h[u] = in ? *reinterpret_cast<const uint4*>(&recs[t])
                : uint4{__float_as_uint(-__builtin_huge_valf()), 0u, kInvalidToken, 0u};
      c[u] = in ? *reinterpret_cast<const uint4*>(&recs[t].begin) : uint4{0u, 0u, 0u, 0u};
      m0[u] = in ? recs[t].m[0] : TileMember{0u, 0u, 0.0f, -__builtin_huge_valf()};
    }
#pragma unroll
    for (uint32_t u = 0; u < kRecBlock; ++u) {
      const uint32_t flags = h[u].y;
      inv |= (flags & kTileInvalid) ? 1u : 0u;
      any_all |= (flags & kTileRescoreAll) ? 1u : 0u;
      if (flags == 0u) lg = __builtin_fmaxf(lg, __uint_as_float(h[u].x));
      if (h[u].z < mt) {
        mt = h[u].z;
        mp = h[u].w;
      }
    }
  }
  const bool invalid = wave_sum_u32(inv) != 0u;
  if (invalid) {
    // an id outside the vocabulary makes the row invalid (greedy.cu:163-166)
    if (lane == 0) {
      a.out_token[r] = kInvalidToken;
      if (a.out_score != nullptr) a.out_score[r] = __builtin_nanf("");
      if (a.out_next != nullptr) a.out_next[r] = kInvalidToken;
    }
    return;
  }
  const bool has_all = wave_sum_u32(any_all) != 0u;
  lg = wave_max(lg);
  wave_min_token(mt, mp);
  __syncthreads();

  // tiles that need every candidate rescored (non-finite values, crowded
  // windows): exact scores, which then also bound the window
  Best best = best_identity();
  if (has_all) {
    for (uint32_t t = 0; t < ntiles; ++t) {
      const TileRecord& q = recs[t];
      if (!(q.flags & kTileRescoreAll)) continue;
      for (uint32_t c0 = 0; c0 < q.count; c0 += kWave) {
        const uint32_t c = c0 + lane;
        if (lane == 0) sh.n_cand = q.count - c0 < kWave ? q.count - c0 : kWave;
        if (c < q.count) {
          const uint32_t p = q.begin + c;
          sh.cand_token[lane] = virtual_list ? p : a.tokens[meta.list_begin + p];
          sh.cand_pos[lane] = p;
        }
        __syncthreads();
        best = best_of(best, rescore_candidates(a, ys, es, sh, sh.n_cand));
      }
    }
    if (best.token != kInvalidToken) lg = __builtin_fmaxf(lg, best.score);
  }

  // ordinary tiles: members whose upper bound reaches lg (at most
  // kTileMembers per tile), collected over all tiles without a barrier per
  // sweep (the record loads of every sweep are in flight together), then
  // rescored together.  If the buffer would overflow, the collection is
  // redone below in flushed sweeps.
  if (lane == 0) sh.n_cand = 0u;
  __syncthreads();
  uint32_t overflow = 0u;
  for (uint32_t base = 0; base < ntiles; base += kWave * kRecBlock) {
    // a row with more blocks reloads each block's flags, member counts and
    // first member (one round trip); the (rare) further members are read
    // afterwards
    if (!resident) {
#pragma unroll
      for (uint32_t u = 0; u < kRecBlock; ++u) {
        const uint32_t t = base + u * kWave + lane;
        const bool in = t < ntiles;
        h[u] = in ? *reinterpret_cast<const uint4*>(&recs[t]) : uint4{0u, kTileInvalid, 0u, 0u};
        c[u] = in ? *reinterpret_cast<const uint4*>(&recs[t].begin) : uint4{0u, 0u, 0u, 0u};
        m0[u] = in ? recs[t].m[0] : TileMember{0u, 0u, 0.0f, -__builtin_huge_valf()};
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < kRecBlock; ++u) {
      const uint32_t t = base + u * kWave + lane;
      if (h[u].y != 0u || t >= ntiles) continue;
      const uint32_t nm = c[u].z < kTileMembers ? c[u].z : kTileMembers;
      for (uint32_t j = 0; j < nm; ++j) {
        const TileMember mm = j == 0 ? m0[u] : recs[t].m[j];
        if (mm.upper >= lg) {
          const uint32_t slot = atomicAdd(&sh.n_cand, 1u);
          if (slot < kCandMax) {
            sh.cand_token[slot] = mm.token;
            sh.cand_pos[slot] = mm.pos;
          } else {
            overflow = 1u;
          }
        }
      }
    }
  }
  __syncthreads();
  if (wave_sum_u32(overflow) == 0u) {
    const uint32_t nc = sh.n_cand;
    if (nc > 0) best = best_of(best, rescore_candidates(a, ys, es, sh, nc));
  } else {
  __syncthreads();
  if (lane == 0) sh.n_cand = 0u;
  __syncthreads();
  for (uint32_t t0 = 0; t0 < ntiles; t0 += kWave) {
    const uint32_t t = t0 + lane;
    if (t < ntiles) {
      const TileRecord& q = recs[t];
      if (q.flags == 0u) {
        const uint32_t nm = q.n_members < kTileMembers ? q.n_members : kTileMembers;
        for (uint32_t j = 0; j < nm; ++j) {
          const TileMember mm = q.m[j];
          if (mm.upper >= lg) {
            const uint32_t slot = atomicAdd(&sh.n_cand, 1u);
            sh.cand_token[slot] = mm.token;
            sh.cand_pos[slot] = mm.pos;
          }
        }
      }
    }
    __syncthreads();
    const uint32_t nc = sh.n_cand;
    // flush when the next sweep could overflow the buffer, and at the end
    if (nc > 0 && (nc > kCandMax - kWave * kTileMembers || t0 + kWave >= ntiles)) {
      best = best_of(best, rescore_candidates(a, ys, es, sh, nc));
      __syncthreads();
      if (lane == 0) sh.n_cand = 0u;
      __syncthreads();
    }
  }
  }

  if (lane == 0) {
    sh.need_score = best.token == kInvalidToken ? 1u : 0u;
    sh.token = sh.need_score ? mt : best.token;
    sh.pos = sh.need_score ? mp : best.pos;
    sh.score = best.score;
  }
  __syncthreads();
  // a row whose scores are all NaN selects its lowest id (greedy.cu:206-211)
  // and reports that id's reference-order score
  const uint32_t token = sh.token;
  const uint32_t pos = sh.pos;
  float score = sh.score;
  if (sh.need_score) {
    const uint32_t H = a.H;
    if ((H & 7u) == 0) {
      copy16_to_lds<2>(reinterpret_cast<uint4*>(es),
                       reinterpret_cast<const uint4*>(a.emb + static_cast<uint64_t>(token) * H),
                       H / 8, lane, kWave);
    } else {
      for (uint32_t q = lane; q < H; q += kWave) es[q] = a.emb[static_cast<uint64_t>(token) * H + q];
    }
    __syncthreads();
    score = a.order == 1 ? chain_lds<true>(ys, es, H) : chain_lds<false>(ys, es, H);
  }
  if (lane == 0) {
    uint32_t next = kInvalidToken;
    if (virtual_list) {
      next = kStateUnrestricted;
    } else if (a.state_next != nullptr) {
      next = a.state_next[meta.list_begin + pos];
    } else if (a.next_table != nullptr) {
      next = static_cast<uint32_t>(a.next_table[static_cast<uint64_t>(meta.state) * a.V + token]);
    }
    a.out_token[r] = token;
    if (a.out_score != nullptr) a.out_score[r] = score;
    if (a.out_next != nullptr) a.out_next[r] = next;
  }
}

} // namespace

hipError_t launch_tail_norm(const TailNormArgs& args, hipStream_t stream) {
  const size_t lds = (args.weight != nullptr ? 3u : 2u) * static_cast<size_t>(args.H) * sizeof(float);
  const uint32_t slots = args.fb_panel != nullptr ? args.fb_m : 0u;
  hipLaunchKernelGGL(tail_norm_kernel, dim3(args.rows + slots), dim3(kWave), lds, stream, args);
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
                     static_cast<size_t>(kStage) * a.H * sizeof(uint16_t);
  hipLaunchKernelGGL(finalize_kernel, dim3(a.rows), dim3(kWave), lds, stream, a);
  return hipGetLastError();
}

} // namespace mf
