// Per-row finalize of the decode tail, run by ONE wave: merges the row's
// tile records, rescores the window survivors in the reference order,
// selects with the reference rule (greedy.cu:84-100, 177-211) and advances
// the DFA.  Every synchronization inside is a wave barrier, so the same code
// serves the one-wave finalize kernel and any wave of a larger workgroup (the
// restricted gather finalizes a row in the wave that writes its last tile
// record).  LDS scratch comes in through FinalizeLds.
#pragma once

#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {

struct FinalizeWords {
  uint32_t n_cand;
  uint32_t token;
  uint32_t pos;
  float score;
  uint32_t need_score;
};

// One wave's finalize scratch.  cand_max must be a multiple of
// 2 kTileMembers; stage_rows >= 1.
struct FinalizeLds {
  float* ys;            // [H] the row's normalized hidden vector
  uint16_t* es;         // [stage_rows][H] embedding rows being rescored
  uint32_t stage_rows;
  uint32_t* cand_token; // [cand_max]
  uint32_t* cand_pos;   // [cand_max]
  uint32_t cand_max;
  FinalizeWords* w;
};

// Reference-order chain over LDS-resident FP32 y and FP16 row (the same
// arithmetic as canonical_dot), LDS reads issued a vector ahead.
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

// One candidate's score in a reference order from LDS.  Blocks of 16
// features alternate between two register sets so that block i + 1's LDS
// reads are in flight during block i's chain.
template <bool kMulAdd>
__device__ float chain_lds(const float* ys, const uint16_t* row, uint32_t H) {
  float s = 0.0f;
  uint32_t f = 0;
  if ((H & 31u) == 0 && (reinterpret_cast<uintptr_t>(row) & 15u) == 0 &&
      (reinterpret_cast<uintptr_t>(ys) & 15u) == 0) {
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

// Reference-order scores with the operands in registers.  Features are cut
// into segments of kChainSeg; with nseg = H / kChainSeg segments, lane
// nseg c + k holds segment k of y and of candidate c's table row (FP32), so
// 64 / nseg candidates are scored at once.  The chain runs segment by
// segment: the lanes holding segment k take their kChainSeg steps from
// registers, then every value moves one lane up, which hands each partial
// sum to the lane holding the next segment of the same candidate.  The
// steps and their order are those of the reference chain; only the place of
// the running sum changes.  Candidate c's score ends in lane nseg c + nseg - 1.
constexpr uint32_t kChainSeg = 64;
template <bool kMulAdd>
__device__ __forceinline__ Best rescore_segmented(const FinalizeArgs& a, const FinalizeLds& L,
                                                  uint32_t n) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t H = a.H;
  const uint32_t nseg = H / kChainSeg;
  const uint32_t per_pass = kWave / nseg;
  const uint32_t c = lane / nseg;
  const uint32_t k = lane % nseg;
  Best best = best_identity();
  for (uint32_t base = 0; base < n; base += per_pass) {
    const uint32_t m = n - base < per_pass ? n - base : per_pass;
    const bool active = c < m;
    const uint32_t j = base + (active ? c : 0u);
    const uint32_t token = L.cand_token[j];
    // segment k of the table row (global) and of y (LDS)
    const uint4* e4 = reinterpret_cast<const uint4*>(a.emb + static_cast<uint64_t>(token) * H + k * kChainSeg);
    uint4 ep[kChainSeg / 8];
#pragma unroll
    for (uint32_t q = 0; q < kChainSeg / 8; ++q) ep[q] = e4[q];
    const float4* y4 = reinterpret_cast<const float4*>(L.ys + k * kChainSeg);
    float yv[kChainSeg];
#pragma unroll
    for (uint32_t q = 0; q < kChainSeg / 4; ++q) {
      const float4 v = y4[q];
      yv[4 * q] = v.x;
      yv[4 * q + 1] = v.y;
      yv[4 * q + 2] = v.z;
      yv[4 * q + 3] = v.w;
    }
    float ev[kChainSeg];
#pragma unroll
    for (uint32_t q = 0; q < kChainSeg / 8; ++q) {
      const uint16_t* hv = reinterpret_cast<const uint16_t*>(&ep[q]);
#pragma unroll
      for (uint32_t i = 0; i < 8; ++i) ev[8 * q + i] = half_to_float(hv[i]);
    }
    float s = 0.0f;
    for (uint32_t seg = 0; seg < nseg; ++seg) {
      if (k == seg) {
#pragma unroll
        for (uint32_t i = 0; i < kChainSeg; ++i) s = order_step<kMulAdd>(s, yv[i], ev[i]);
      }
      if (seg + 1 < nseg) s = lane_shift_right(s);
    }
    if (active && k == nseg - 1u) best = best_of(best, best_leaf(s, token, L.cand_pos[j]));
  }
  return wave_best(best);
}

// Rescores candidates cand_token[0..n) of one row in the reference order:
// in registers (rescore_segmented) when H is a multiple of kChainSeg of at
// most kWave segments, else stage_rows rows at a time staged in LDS;
// returns the wave's best.
__device__ inline Best rescore_candidates(const FinalizeArgs& a, const FinalizeLds& L,
                                          uint32_t n) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t H = a.H;
  if (H % kChainSeg == 0u && H <= kChainSeg * kWave &&
      (reinterpret_cast<uintptr_t>(a.emb) & 15u) == 0) {
    wave_sync();
    return a.order == 1 ? rescore_segmented<true>(a, L, n) : rescore_segmented<false>(a, L, n);
  }
  Best best = best_identity();
  for (uint32_t base = 0; base < n; base += L.stage_rows) {
    const uint32_t m = n - base < L.stage_rows ? n - base : L.stage_rows;
    wave_sync();
    if ((H & 7u) == 0) {
      // every row's pieces in flight before their stores
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
                           a.emb + static_cast<uint64_t>(L.cand_token[base + j]) * H)[q % per]
                     : uint4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
          const uint32_t q = q0 + u * kWave;
          if (q < total) reinterpret_cast<uint4*>(L.es + (q / per) * H)[q % per] = v[u];
        }
      }
    } else {
      for (uint32_t q = lane; q < m * H; q += kWave) {
        const uint32_t j = q / H;
        L.es[q] = a.emb[static_cast<uint64_t>(L.cand_token[base + j]) * H + (q % H)];
      }
    }
    wave_sync();
    if (lane < m) {
      const float s = a.order == 1 ? chain_lds<true>(L.ys, L.es + lane * H, H)
                                   : chain_lds<false>(L.ys, L.es + lane * H, H);
      best = best_of(best, best_leaf(s, L.cand_token[base + lane], L.cand_pos[base + lane]));
    }
  }
  return wave_best(best);
}

// Adds the members of ordinary tile t (upper >= lg) to the candidate buffer.
// Returns 1 if the buffer had no room for one of them.
__device__ __forceinline__ uint32_t collect_members(const TileRecord* recs, uint32_t t,
                                                    uint32_t n_members, const TileMember& first,
                                                    float lg, const FinalizeLds& L) {
  uint32_t overflow = 0u;
  const uint32_t nm = n_members < kTileMembers ? n_members : kTileMembers;
  // the other members' loads issued together (one line with the header)
  TileMember ms[kTileMembers];
  ms[0] = first;
#pragma unroll
  for (uint32_t j = 1; j < static_cast<uint32_t>(kTileMembers); ++j) {
    ms[j] = j < nm ? recs[t].m[j] : TileMember{0u, 0u, 0.0f, -__builtin_huge_valf()};
  }
#pragma unroll
  for (uint32_t j = 0; j < static_cast<uint32_t>(kTileMembers); ++j) {
    const TileMember mm = ms[j];
    if (j < nm && mm.upper >= lg) {
      const uint32_t slot = atomicAdd(&L.w->n_cand, 1u);
      if (slot < L.cand_max) {
        L.cand_token[slot] = mm.token;
        L.cand_pos[slot] = mm.pos;
      } else {
        overflow = 1u;
      }
    }
  }
  return overflow;
}

// A lower bound, in the scale of the row's records, of the exact score s:
// s itself for records scored on y, else s / inv rounded down (the division
// is within half an ulp; the margins cover it and subnormal quotients).  No
// bound (-inf) when inv or the quotient is not a positive finite number.
__device__ __forceinline__ float records_lower(const FinalizeArgs& a, uint32_t r, float s) {
  if (a.row_inv == nullptr) return s;
  const float inv = a.row_inv[r];
  const float q = s / inv;
  if (!(inv > 0.0f) || !__builtin_isfinite(q)) return -__builtin_huge_valf();
  return q - __builtin_fabsf(q) * 0x1p-20f - 0x1p-126f;
}

// Finalizes row r (meta = its metadata) with one wave.  stage_y() puts the
// row's normalized hidden vector into L.ys; it is called once the record
// headers are in flight, before the first rescore, so the caller can keep
// the vector's loads in flight meanwhile.  Writes token, score and next
// state of the row; rows that are neither gathered nor served by the MFMA
// head are left alone (their outputs were preset by the norm kernel).
template <typename StageY>
__device__ inline void finalize_row(const FinalizeArgs& a, uint32_t r, const RowMeta& meta,
                                    const FinalizeLds& L, StageY&& stage_y) {
  const uint32_t lane = threadIdx.x % kWave;
  const TileRecord* recs;
  uint32_t ntiles;
  // the per-row words the record pointer needs, loaded beside the metadata
  // (not after it)
  const uint32_t fb_slot = a.fb_map != nullptr ? a.fb_map[r] : kInvalidToken;
  const uint32_t row_tiles = a.row_tiles != nullptr ? a.row_tiles[r] : 0u;
  if ((meta.kind & kRowDense) && a.fb_records != nullptr) {
    // scored by the dense head: its records, list positions of the row's
    // ascending list
    const uint32_t m = fb_slot;
    if (m == kInvalidToken) return;
    recs = a.fb_records + static_cast<uint64_t>(m) * a.fb_tiles;
    ntiles = a.fb_tiles;
  } else if (meta.kind & kRowRestricted) {
    recs = a.records + static_cast<uint64_t>(r) * a.max_tiles;
    ntiles = a.row_tiles != nullptr ? (row_tiles & ~kRangesUnused)
                                    : (meta.count + a.tile - 1) / a.tile;
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
  // pass 1: validity, the best lower bound of ordinary tiles, lowest id.
  // Per tile the header (best_lower, flags, min_token, min_pos), the counts
  // (begin, count, n_members) and the first member, kRecBlock tiles per lane
  // loaded before any is used: one round trip per block.  A row of at most
  // kWave kRecBlock tiles keeps them in registers for the member collection.
  constexpr uint32_t kRecBlock = 4;
  uint32_t inv = 0u;
  uint32_t any_all = 0u;
  float lg = -__builtin_huge_valf();
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
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
      // ordinary and crowded tiles carry a valid best lower bound
      if (flags == 0u || flags == (kTileRescoreAll | kTileCrowded)) {
        lg = __builtin_fmaxf(lg, __uint_as_float(h[u].x));
      }
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
      uint32_t* next = next_state_slot(a.out_next, a.row_sequence, a.capacity, r);
      if (next != nullptr) *next = kInvalidToken;
    }
    return;
  }
  const bool has_all = wave_sum_u32(any_all) != 0u;
  lg = wave_max(lg);
  wave_min_token(mt, mp);
  stage_y();
  wave_sync();

  // tiles that need every candidate rescored (non-finite values, crowded
  // windows): exact scores, which then also bound the window.  A crowded
  // tile whose best upper bound is below the row's best lower bound holds
  // no winner and is skipped.
  // The tiles to rescore are found from the headers already in registers
  // (a ballot per block of tiles), not by reading every record in turn.
  Best best = best_identity();
  if (has_all) {
    const uint32_t chunk = L.cand_max < kWave ? L.cand_max : kWave;
    for (uint32_t base = 0; base < ntiles; base += kWave * kRecBlock) {
      if (!resident) {
#pragma unroll
        for (uint32_t u = 0; u < kRecBlock; ++u) {
          const uint32_t t = base + u * kWave + lane;
          const bool in = t < ntiles;
          h[u] = in ? *reinterpret_cast<const uint4*>(&recs[t]) : uint4{0u, 0u, 0u, 0u};
          c[u] = in ? *reinterpret_cast<const uint4*>(&recs[t].begin) : uint4{0u, 0u, 0u, 0u};
        }
      }
#pragma unroll
      for (uint32_t u = 0; u < kRecBlock; ++u) {
        const uint32_t t = base + u * kWave + lane;
        const uint32_t flags = h[u].y;
        const bool hopeless = (flags & kTileCrowded) && __uint_as_float(c[u].w) < lg;
        uint64_t need = __ballot(t < ntiles && (flags & kTileRescoreAll) && !hopeless);
        while (need != 0ull) {
          const int src = __builtin_ctzll(need);
          need &= need - 1ull;
          const uint32_t begin = static_cast<uint32_t>(__shfl(static_cast<int>(c[u].x), src));
          const uint32_t count = static_cast<uint32_t>(__shfl(static_cast<int>(c[u].y), src));
          for (uint32_t c0 = 0; c0 < count; c0 += chunk) {
            const uint32_t n = count - c0 < chunk ? count - c0 : chunk;
            wave_sync();
            if (lane < n) {
              const uint32_t p = begin + c0 + lane;
              L.cand_token[lane] = virtual_list ? p : a.tokens[meta.list_begin + p];
              L.cand_pos[lane] = p;
            }
            best = best_of(best, rescore_candidates(a, L, n));
          }
        }
      }
    }
    if (best.token != kInvalidToken) lg = __builtin_fmaxf(lg, records_lower(a, r, best.score));
  }

  // ordinary tiles: members whose upper bound reaches lg (at most
  // kTileMembers per tile), collected over all tiles, then rescored
  // together.  Per block of tiles, the further members of every tile that
  // reaches the window are loaded at once (one round trip), then appended in
  // lane order by ballot: no LDS atomic, whose returned slot would cost a
  // round trip per member.  If the buffer would overflow, the collection is
  // redone below in flushed sweeps.
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t nc = 0u;
  for (uint32_t base = 0; base < ntiles; base += kWave * kRecBlock) {
    // a row with more blocks reloads each block's flags, member counts and
    // first member (one round trip)
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
    // appends the members whose lanes have p set, in lane order
    auto append = [&](bool p, const TileMember& mm) {
      const uint64_t m = __ballot(p);
      if (m == 0ull) return;
      const uint32_t slot = nc + static_cast<uint32_t>(__popcll(m & below));
      if (p && slot < L.cand_max) {
        L.cand_token[slot] = mm.token;
        L.cand_pos[slot] = mm.pos;
      }
      nc += static_cast<uint32_t>(__popcll(m));
    };
    uint32_t nm[kRecBlock];
    uint32_t multi = 0u;
#pragma unroll
    for (uint32_t u = 0; u < kRecBlock; ++u) {
      const uint32_t t = base + u * kWave + lane;
      // no member of a tile whose best upper bound is below the window
      const bool take = h[u].y == 0u && t < ntiles && !(__uint_as_float(c[u].w) < lg);
      nm[u] = take ? (c[u].z < kTileMembers ? c[u].z : static_cast<uint32_t>(kTileMembers)) : 0u;
      multi |= nm[u] > 1u ? 1u : 0u;
    }
    if (__ballot(multi != 0u) == 0ull) {
      // the common case, every tile in the window holds one member: a short
      // path (one wave runs it, so its instruction count is its time)
#pragma unroll
      for (uint32_t u = 0; u < kRecBlock; ++u) append(nm[u] != 0u && m0[u].upper >= lg, m0[u]);
      continue;
    }
    TileMember ms[kRecBlock][kTileMembers];
#pragma unroll
    for (uint32_t u = 0; u < kRecBlock; ++u) {
      const uint32_t t = base + u * kWave + lane;
      ms[u][0] = m0[u];
#pragma unroll
      for (uint32_t j = 1; j < static_cast<uint32_t>(kTileMembers); ++j) {
        ms[u][j] = j < nm[u] ? recs[t].m[j] : TileMember{0u, 0u, 0.0f, -__builtin_huge_valf()};
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < kRecBlock; ++u) {
#pragma unroll
      for (uint32_t j = 0; j < static_cast<uint32_t>(kTileMembers); ++j) {
        append(j < nm[u] && ms[u][j].upper >= lg, ms[u][j]);
      }
    }
  }
  wave_sync();
  if (nc <= L.cand_max) {
    if (nc > 0) best = best_of(best, rescore_candidates(a, L, nc));
  } else {
    // flushed sweeps: a sweep of sw tiles adds at most sw kTileMembers =
    // cand_max / 2 candidates, so flushing above half keeps the buffer
    // within its size
    const uint32_t sw = L.cand_max / (2u * kTileMembers);
    wave_sync();
    if (lane == 0) L.w->n_cand = 0u;
    wave_sync();
    for (uint32_t t0 = 0; t0 < ntiles; t0 += sw) {
      const uint32_t t = t0 + lane;
      if (lane < sw && t < ntiles) {
        const TileRecord& q = recs[t];
        if (q.flags == 0u) collect_members(recs, t, q.n_members, q.m[0], lg, L);
      }
      wave_sync();
      const uint32_t n = L.w->n_cand;
      // flush when the next sweep could overflow the buffer, and at the end
      if (n > 0 && (n > L.cand_max / 2u || t0 + sw >= ntiles)) {
        best = best_of(best, rescore_candidates(a, L, n));
        wave_sync();
        if (lane == 0) L.w->n_cand = 0u;
        wave_sync();
      }
    }
  }

  if (lane == 0) {
    L.w->need_score = best.token == kInvalidToken ? 1u : 0u;
    L.w->token = L.w->need_score ? mt : best.token;
    L.w->pos = L.w->need_score ? mp : best.pos;
    L.w->score = best.score;
  }
  wave_sync();
  // a row whose scores are all NaN selects its lowest id (greedy.cu:206-211)
  // and reports that id's reference-order score
  const uint32_t token = L.w->token;
  const uint32_t pos = L.w->pos;
  float score = L.w->score;
  if (L.w->need_score) {
    const uint32_t H = a.H;
    if ((H & 7u) == 0) {
      copy16_to_lds<2>(reinterpret_cast<uint4*>(L.es),
                       reinterpret_cast<const uint4*>(a.emb + static_cast<uint64_t>(token) * H),
                       H / 8, lane, kWave);
    } else {
      for (uint32_t q = lane; q < H; q += kWave) L.es[q] = a.emb[static_cast<uint64_t>(token) * H + q];
    }
    wave_sync();
    score = a.order == 1 ? chain_lds<true>(L.ys, L.es, H) : chain_lds<false>(L.ys, L.es, H);
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
    uint32_t* slot = next_state_slot(a.out_next, a.row_sequence, a.capacity, r);
    if (slot != nullptr) *slot = next;
  }
  wave_sync();
}

}  // namespace mf
