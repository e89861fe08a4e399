// The decode tail's per-row preparation, one wave per item: the norm kernel
// runs one item per workgroup, the fused gather launch four per workgroup
// beside its gather workgroups.
//
// Item r < rows (a row): its list (the state through the sequence table, the
// state's CSR span, the validity rules) into row_meta, the preset outputs of
// rows the gather does not serve, the reference-order RMSNorm y and inv
// (operators.cpp:523-535), and -- when the caller asks -- the FP16 split of
// z = x * w with its bounds.  Item rows + j (a slot of the MFMA head): the
// split of row fb_rows[j] into slot j of the head's panel, with its bounds.
#pragma once

#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"
#include "mf_norm.hpp"

namespace mf {

// Row r's list: state s (through the sequence table: q = row_sequence[r],
// MF_STATE_INVALID when q is outside it), the CSR span [b, e) of s and the
// row's metadata (restricted when s < states and 0 < e - b <= max_count with
// e <= nnz; unrestricted for MF_STATE_UNRESTRICTED; invalid otherwise).
struct RowList {
  RowMeta meta;
  uint32_t q;  // state-table index (r without a table)
  uint32_t b;
  uint32_t e;
};

__device__ __forceinline__ RowList row_list(const TailNormArgs& a, uint32_t r) {
  RowList l;
  l.q = r;
  uint32_t s;
  if (a.row_sequence != nullptr) {
    l.q = a.row_sequence[r];
    s = l.q < a.capacity ? a.row_state[l.q] : kInvalidToken;
  } else {
    s = a.row_state[r];
  }
  l.b = 0u;
  l.e = 0u;
  if (s < a.states) {
    l.b = a.offsets[s];
    l.e = a.offsets[s + 1];
  }
  l.meta = RowMeta{0u, 0u, s, kRowInvalid};
  if (s == kStateUnrestricted) {
    l.meta = RowMeta{0u, a.V, s, kRowUnrestricted};
  } else if (s < a.states && l.e > l.b && l.e <= a.nnz && l.e - l.b <= a.max_count) {
    l.meta = RowMeta{l.b, l.e - l.b, s, kRowRestricted};
  }
  return l;
}

// Bound of ||z|| from the wave's per-lane sums of z^2, and the row's absolute
// error term from its per-lane sums of the rounded squares x^2.  1 / inv <=
// sqrt(x_sq (1 + 2^-9) / H + eps) (1 + 2^-9): the reference sums the same
// rounded squares in another order (relative H 2^-23 apart at most,
// H <= 8192), then divides, adds eps, takes the square root and the
// reciprocal (a few roundings); the 2^-9 margins cover all of them.  An
// infinite or NaN value (overflowing or non-finite x) makes every bound of
// the row infinite, and the row is then rescored in full.
__device__ __forceinline__ void z_bounds(float z_sq, float x_sq, bool weighted, uint32_t H,
                                         float epsilon, float slack_base, float slack_scaled,
                                         float& z_norm, float& slack) {
  z_sq = wave_sum_f32(z_sq);
  x_sq = wave_sum_f32(x_sq);
  // FP32 sum of H squares is within a relative H 2^-24 of the exact value;
  // the factor covers that and the sqrt for any H <= 2^16
  z_norm = __fsqrt_rn(z_sq) * (1.0f + 0x1p-7f);
  slack = slack_base;
  if (weighted) {
    const float scale =
        __fsqrt_rn(x_sq * (1.0f + 0x1p-9f) / static_cast<float>(H) + epsilon) * (1.0f + 0x1p-9f);
    slack = __builtin_fmaf(scale, slack_scaled, slack_base);
  }
}

// One wave, item `item`.  lds: the wave's own 3 H floats (16-byte aligned);
// inv_slot: one float of the wave's own.  split_rows: also write the row's
// FP16 split of z and its bounds (row_norm, row_slack); the fused gather
// computes those itself.
__device__ inline void prep_item(const TailNormArgs& a, uint32_t item, float* lds,
                                 float* inv_slot, bool split_rows) {
  const uint32_t H = a.H;
  const uint32_t lane = threadIdx.x % kWave;
  float* xs = lds;
  float* sq = lds + H;
  float* ws = lds + 2u * H;
  const bool slot = item >= a.rows;
  const uint32_t j = item - a.rows;  // the slot (slot items)
  uint64_t r = item;
  if (slot) {
    r = a.fb_rows[j];
    if (r >= a.rows) {
      if (lane == 0) {
        a.fb_slot_row[j] = kInvalidToken;
        a.fb_slot_norm[j] = 0.0f;
        a.fb_slot_slack[j] = 0.0f;
      }
      return;
    }
  }
  const bool weighted = a.weight != nullptr;
  // rows compute y here unless the chain waves of the gather launch do
  const bool chain = weighted && !slot && a.chain;
  const bool write_y = !slot && (!weighted || a.chain);
  const bool split = slot || (split_rows && a.y_hi != nullptr);
  // the row's list first: its loads are in flight during the staging
  RowList l{};
  if (!slot && lane == 0) l = row_list(a, static_cast<uint32_t>(r));
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
  wave_sync();
  // the reference-order chain: rows only (a slot needs z, not y), and only
  // when it is not deferred to the gather launch
  const float sum_squares = chain ? sequential_sum_wave(sq, H) : 0.0f;
  if (lane == 0) {
    if (chain) *inv_slot = norm_inverse(sum_squares, H, a.epsilon);
    if (!slot) {
      a.row_meta[r] = l.meta;
      if (l.meta.kind != kRowRestricted) {
        // invalid rows keep these; unrestricted rows are overwritten by the
        // finalize kernel when the MFMA head was given them.  A finished row
        // (empty list) holds its state when asked to.
        a.out_token[r] = kInvalidToken;
        if (a.out_score != nullptr) a.out_score[r] = __builtin_nanf("");
        if (a.out_next != nullptr && l.q < a.capacity) {
          const uint32_t s = l.meta.state;
          a.out_next[l.q] = (a.hold && s < a.states && l.e == l.b) ? s : kInvalidToken;
        }
      }
      if (a.fb_map != nullptr) a.fb_map[r] = kInvalidToken;
    }
  }
  wave_sync();
  const float inverse = chain ? *inv_slot : 1.0f;
  // slot items: the slot's [hi | lo] rows of the panel
  uint16_t* panel_hi = nullptr;
  if (slot) {
    panel_hi = a.fb_panel + static_cast<uint64_t>(j / kPanelRows) * (panel_tile_bytes(H) / 2u) +
               static_cast<uint64_t>(j % kPanelRows) * 2u * (H + kPanelPad);
  }
  // y = (x * inv) * w in the reference's roundings (operators.cpp:533-534)
  // for the rescore; z = x * w, the fast scores' operand, split into FP16
  // hi + lo.  z differs from y / inv by at most 3 roundings per element.
  float z_sq = 0.0f;
  float x_sq = 0.0f;
  // four features per lane at a time: 16-byte LDS reads, 16-byte y stores
  // and 8-byte stores of the FP16 hi and lo halves (per element the same
  // values; the bound sums x_sq and z_sq take any order)
  const uint32_t c4 = (H % 4u == 0u) ? H : 0u;
  for (uint32_t q = lane; q < c4 / 4u; q += kWave) {
    const float4 xv = reinterpret_cast<const float4*>(xs)[q];
    float4 yv = xv;
    float4 zv = xv;
    if (weighted) {
      const float4 wv = reinterpret_cast<const float4*>(ws)[q];
      const float4 sv = reinterpret_cast<const float4*>(sq)[q];
      yv = float4{(xv.x * inverse) * wv.x, (xv.y * inverse) * wv.y, (xv.z * inverse) * wv.z,
                  (xv.w * inverse) * wv.w};
      zv = float4{xv.x * wv.x, xv.y * wv.y, xv.z * wv.z, xv.w * wv.w};
      x_sq += (sv.x + sv.y) + (sv.z + sv.w);
    }
    if (write_y) reinterpret_cast<float4*>(a.y + r * H)[q] = yv;
    if (split) {
      const float zz[4] = {zv.x, zv.y, zv.z, zv.w};
      uint16_t hv[4], lv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        z_sq = __builtin_fmaf(zz[k], zz[k], z_sq);
        const _Float16 hi = static_cast<_Float16>(zz[k]);
        hv[k] = __builtin_bit_cast(uint16_t, hi);
        lv[k] = float_to_half_rne(zz[k] - static_cast<float>(hi));
      }
      const uint2 hp{static_cast<uint32_t>(hv[0]) | (static_cast<uint32_t>(hv[1]) << 16),
                     static_cast<uint32_t>(hv[2]) | (static_cast<uint32_t>(hv[3]) << 16)};
      const uint2 lp{static_cast<uint32_t>(lv[0]) | (static_cast<uint32_t>(lv[1]) << 16),
                     static_cast<uint32_t>(lv[2]) | (static_cast<uint32_t>(lv[3]) << 16)};
      if (slot) {
        reinterpret_cast<uint2*>(panel_hi)[q] = hp;
        reinterpret_cast<uint2*>(panel_hi + H + kPanelPad)[q] = lp;
      } else {
        reinterpret_cast<uint2*>(a.y_hi + r * H)[q] = hp;
        reinterpret_cast<uint2*>(a.y_lo + r * H)[q] = lp;
      }
    }
  }
  for (uint32_t c = c4 + lane; c < H; c += kWave) {
    const float xv = xs[c];
    float yv = xv;
    float zv = xv;
    if (weighted) {
      const float scaled = xv * inverse;
      yv = scaled * ws[c];
      zv = xv * ws[c];
      x_sq += sq[c];
    }
    if (write_y) a.y[r * H + c] = yv;
    if (split) {
      z_sq = __builtin_fmaf(zv, zv, z_sq);
      const _Float16 hi = static_cast<_Float16>(zv);
      const uint16_t lo = float_to_half_rne(zv - static_cast<float>(hi));
      if (slot) {
        panel_hi[c] = __builtin_bit_cast(uint16_t, hi);
        panel_hi[H + kPanelPad + c] = lo;
      } else {
        a.y_hi[r * H + c] = __builtin_bit_cast(uint16_t, hi);
        a.y_lo[r * H + c] = lo;
      }
    }
  }
  if (!split) {
    if (write_y && lane == 0) a.row_inv[r] = inverse;
    return;
  }
  float z_norm, slack;
  z_bounds(z_sq, x_sq, weighted, H, a.epsilon, a.slack, a.slack_scaled, z_norm, slack);
  if (lane == 0) {
    if (slot) {
      a.fb_slot_norm[j] = z_norm;
      a.fb_slot_slack[j] = slack;
      a.fb_slot_row[j] = static_cast<uint32_t>(r);
    } else {
      a.row_norm[r] = z_norm;
      a.row_slack[r] = slack;
      if (write_y) a.row_inv[r] = inverse;
    }
  }
}

// The range index of row r for the table pass (TailNormArgs range_index,
// row_tiles): per 192-token range g of the vocabulary, the positions
// [lo, hi) of the row's ids in the range and its record index among the
// row's non-empty ranges (0, 0, 0 for an empty range), range-major so the
// pass reads one range's entries of all rows contiguously.  Built by the
// kWalkWaves waves of a workgroup of its own (the norm items run in other
// workgroups of the same launch), with one workgroup barrier:
//
//   range_walk   wave `part` walks its share of the list's 64-id chunks,
//                each lane also loading its id's predecessor.  An id whose
//                predecessor lies in an earlier range opens its range: it
//                records its position as the range's lo, its rank among this
//                wave's openers, a bit in this wave's own bitmap (cleared by
//                the wave itself, so no wave waits for another before
//                walking), and its position as the hi of the predecessor's
//                range; the list's last id closes its own range at the end.
//   range_end    (after the barrier) every range g's entry: opened when a
//                wave's bit says so, ranks made record indices by adding the
//                opener counts of earlier waves; written out coalesced.
//
// A list that is not strictly ascending, or holds an id >= V, is not
// indexed: the row gets one record covering its whole list, "rescore all"
// (exact, in the finalize) or "invalid".  LDS: range_lds_words(ranges).
constexpr uint32_t kWalkWaves = 8;

__host__ __device__ constexpr uint32_t range_bit_words(uint32_t ranges) { return ranges / 32u + 1u; }
__host__ __device__ constexpr uint32_t range_lds_words(uint32_t ranges) {
  return 3u * ranges + kWalkWaves * (2u + range_bit_words(ranges));
}

struct RangeLds {
  uint32_t* lo;     // [ranges] position of each opened range's first id
  uint32_t* hi;     // [ranges] one past its last id
  uint32_t* rank;   // [ranges] rank of each opened range among its wave's openers
  uint32_t* count;  // [kWalkWaves] openers per wave
  uint32_t* flags;  // [kWalkWaves] bit 0: an id >= V, bit 1: not ascending
  uint32_t* bits;   // [kWalkWaves][range_bit_words] ranges each wave opened
  static __device__ RangeLds at(uint32_t* base, uint32_t ranges) {
    uint32_t* q = base + 3u * ranges;
    return RangeLds{base, base + ranges, base + 2u * ranges, q, q + kWalkWaves, q + 2u * kWalkWaves};
  }
};

struct RangeRow {
  uint32_t b;     // list start
  uint32_t c;     // list length
  bool indexed;   // a restricted row
};

// The row's list (every walk wave finds it itself).
__device__ inline RangeRow range_row(const TailNormArgs& a, uint32_t r) {
  const uint32_t lane = threadIdx.x % kWave;
  RowList l{};
  if (lane == 0) l = row_list(a, r);
  RangeRow w;
  w.b = __shfl(l.b, 0);
  w.c = __shfl(l.e, 0) - w.b;
  w.indexed = __shfl(l.meta.kind, 0) == kRowRestricted;
  return w;
}

__device__ inline void range_walk(const TailNormArgs& a, const RangeRow& w, const RangeLds& L,
                                  uint32_t part) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t G = a.ranges;
  const uint32_t b = w.b;
  const uint32_t c = w.c;
  const uint32_t words = range_bit_words(G);
  uint32_t* bits = L.bits + part * words;
  for (uint32_t i = lane; i < words; i += kWave) bits[i] = 0u;
  wave_sync();
  const uint32_t chunks = (c + kWave - 1) / kWave;
  const uint32_t lo = chunks * part / kWalkWaves * kWave;        // this wave's positions
  const uint32_t hi = chunks * (part + 1) / kWalkWaves * kWave;  // [lo, min(hi, c))
  uint32_t opened = 0u;
  bool bad = false;
  bool unsorted = false;
  // ids in batches of kChunks chunks of 64, two batches in flight, each
  // handled with compile-time registers; unconditional loads at clamped
  // positions (a load under a branch makes the compiler wait for every load
  // in flight at the join)
  constexpr uint32_t kChunks = 8;
  constexpr uint32_t kStep = kChunks * kWave;
  // positions past this wave's share load its last id (one address per
  // instruction), not the next wave's ids
  const uint32_t end = hi < c ? hi : c;
  const uint32_t last = end > 0u ? end - 1u : 0u;
  auto load = [&](uint32_t base, uint32_t (&ids)[kChunks], uint32_t (&pre)[kChunks]) {
#pragma unroll
    for (uint32_t u = 0; u < kChunks; ++u) {
      const uint32_t q = base + u * kWave + lane;
      const uint32_t qi = q < end ? q : last;
      ids[u] = a.tokens[b + qi];
      pre[u] = a.tokens[b + (qi > 0u ? qi - 1u : 0u)];
    }
  };
  auto walk = [&](uint32_t base, const uint32_t (&ids)[kChunks], const uint32_t (&pre)[kChunks]) {
#pragma unroll
    for (uint32_t u = 0; u < kChunks; ++u) {
      const uint32_t p = base + u * kWave + lane;
      const bool in = p < c && p < hi;
      const uint32_t t = in ? ids[u] : kInvalidToken;
      const uint32_t tp = p > 0u ? pre[u] : kInvalidToken;  // no predecessor at p = 0
      const uint32_t gt = t < a.V ? t / kHeadTileTokens : G;
      const uint32_t gp = tp < a.V ? tp / kHeadTileTokens : G;
      bad |= in && t >= a.V;
      unsorted |= in && p > 0 && t <= tp;
      const bool opens = in && gt < G && gt != gp;
      const uint64_t m = __ballot(opens);
      // LDS only: global stores under a branch would stall the loads
      if (opens) {
        L.lo[gt] = p;
        L.rank[gt] = opened + static_cast<uint32_t>(__popcll(m & ((1ull << lane) - 1ull)));
        atomicOr(&bits[gt / 32u], 1u << (gt % 32u));
        if (p > 0u && gp < G) L.hi[gp] = p;
      }
      if (in && p == c - 1u && gt < G) L.hi[gt] = c;
      opened += static_cast<uint32_t>(__popcll(m));
    }
  };
  uint32_t ia[kChunks], pa[kChunks], ib[kChunks], pb[kChunks];
  load(lo, ia, pa);
  for (uint32_t base = lo; base < hi && base < c; base += 2u * kStep) {
    load(base + kStep, ib, pb);
    walk(base, ia, pa);
    load(base + 2u * kStep, ia, pa);
    if (base + kStep < hi && base + kStep < c) walk(base + kStep, ib, pb);
  }
  const bool any_bad = __ballot(bad) != 0ull;
  const bool any_unsorted = __ballot(unsorted) != 0ull;
  if (lane == 0) {
    L.count[part] = opened;
    L.flags[part] = (any_bad ? 1u : 0u) | (any_unsorted ? 2u : 0u);
  }
}

// All kWalkWaves waves (after the barrier): range g = tid, tid + 64 kWalkWaves, ...
__device__ inline void range_end(const TailNormArgs& a, uint32_t r, const RangeRow& w,
                                 const RangeLds& L) {
  const uint32_t tid = threadIdx.x;
  const uint32_t G = a.ranges;
  const uint32_t rows = a.rows;
  const uint32_t words = range_bit_words(G);
  uint32_t base[kWalkWaves];
  uint32_t tiles = 0u;
  uint32_t flags = 0u;
#pragma unroll
  for (uint32_t i = 0; i < kWalkWaves; ++i) {
    base[i] = tiles;
    tiles += L.count[i];
    flags |= L.flags[i];
  }
  if (flags == 0u) {
    for (uint32_t g = tid; g < G; g += kWalkWaves * kWave) {
      uint4 e = {0u, 0u, 0u, 0u};
#pragma unroll
      for (uint32_t i = 0; i < kWalkWaves; ++i) {
        if ((L.bits[i * words + g / 32u] >> (g % 32u)) & 1u) e = uint4{L.lo[g], L.hi[g], L.rank[g] + base[i], 0u};
      }
      a.range_index[static_cast<uint64_t>(g) * rows + r] = e;
    }
    if (tid == 0) a.row_tiles[r] = tiles;
    return;
  }
  // a list that is not indexed: one whole-list record with its lowest id
  if (tid >= kWave) return;
  const uint32_t lane = tid;
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
  for (uint32_t p = lane; p < w.c; p += kWave) {
    const uint32_t t = a.tokens[w.b + p];
    if (t < mt) {
      mt = t;
      mp = p;
    }
  }
  wave_min_token(mt, mp);
  if (lane == 0) {
    TileRecord* rec = a.records + static_cast<uint64_t>(r) * a.max_recs;
    rec->best_lower = -__builtin_huge_valf();
    rec->flags = (flags & 1u) ? kTileInvalid : kTileRescoreAll;
    rec->min_token = mt;
    rec->min_pos = mp;
    rec->begin = 0u;
    rec->count = w.c;
    rec->n_members = 0u;
    rec->upper_max = __builtin_huge_valf();
    a.row_tiles[r] = 1u | kRangesUnused;
  }
}

// ---- dense index (the spans the dense head reads, mf_dense.hip) ------------
//
// Walk workgroup r (kWalkWaves waves) indexes row r's list when it is a
// candidate (restricted, at least dense_min ids): every id sets its bit in
// the LDS mask of its 192-token range; an id >= V or a list that is not
// strictly ascending leaves the row to the gather.  Then the ranges' counts
// are scanned (the list position of each range's first id) and the spans
// written out, range-major; dense_flag[r] says whether the row was indexed.
// Which indexed rows the dense head takes is decided after the launch
// (dense_choose_kernel, mf_tail.hip).  LDS: dense_lds_words(ranges).
__host__ __device__ constexpr uint32_t dense_lds_words(uint32_t ranges) {
  return 6u * ranges + 2u * kWalkWaves + 4u;
}

__device__ inline void dense_walk(const TailNormArgs& a, uint32_t r, uint32_t* lds) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  constexpr uint32_t kT = kWalkWaves * kWave;
  const uint32_t G = a.ranges;
  uint32_t* mask = lds;                      // [G][6]
  uint32_t* wsum = lds + 6u * G;             // [kWalkWaves]
  uint32_t* flags = wsum + 2u * kWalkWaves;  // [1]
  const RangeRow w = range_row(a, r);
  const bool cand = w.indexed && w.c >= a.dense_min;
  bool ok = false;
  if (cand) {
    for (uint32_t i = tid; i < 6u * G; i += kT) mask[i] = 0u;
    if (tid == 0) *flags = 0u;
    __syncthreads();
    const uint32_t b = w.b;
    const uint32_t c = w.c;
    bool bad = false;
    constexpr uint32_t kU = 16;  // loads in flight per thread
    for (uint32_t base = tid; base < c; base += kT * kU) {
      uint32_t t[kU], tp[kU];
#pragma unroll
      for (uint32_t u = 0; u < kU; ++u) {
        const uint32_t p = base + u * kT;
        const uint32_t pc = p < c ? p : c - 1u;
        t[u] = a.tokens[b + pc];
        tp[u] = a.tokens[b + (pc > 0u ? pc - 1u : 0u)];
      }
#pragma unroll
      for (uint32_t u = 0; u < kU; ++u) {
        const uint32_t p = base + u * kT;
        if (p < c) {
          bad |= t[u] >= a.V || (p > 0u && t[u] <= tp[u]);
          if (t[u] < a.V) {
            const uint32_t g = t[u] / kHeadTileTokens;
            atomicOr(&mask[g * 6u + (t[u] % kHeadTileTokens) / 32u], 1u << (t[u] % 32u));
          }
        }
      }
    }
    if (__ballot(bad) != 0ull && lane == 0) atomicOr(flags, 1u);
    __syncthreads();
    ok = *flags == 0u;
    if (ok) {
      // exclusive scan of the ranges' counts: thread segments, then waves
      const uint32_t per = (G + kT - 1u) / kT;
      const uint32_t g0 = tid * per < G ? tid * per : G;
      const uint32_t g1 = g0 + per < G ? g0 + per : G;
      uint32_t local = 0u;
      for (uint32_t g = g0; g < g1; ++g) {
#pragma unroll
        for (uint32_t k = 0; k < 6u; ++k) local += static_cast<uint32_t>(__popc(mask[g * 6u + k]));
      }
      uint32_t incl = local;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), d));
        if (static_cast<int>(lane) >= d) incl += o;
      }
      if (lane == kWave - 1) wsum[wave] = incl;
      __syncthreads();
      uint32_t run = incl - local;
      for (uint32_t v = 0; v < wave; ++v) run += wsum[v];
      for (uint32_t g = g0; g < g1; ++g) {
        const uint32_t* m = mask + g * 6u;
        uint32_t n = 0u;
#pragma unroll
        for (uint32_t k = 0; k < 6u; ++k) n += static_cast<uint32_t>(__popc(m[k]));
        uint4* out = a.dense_spans + (static_cast<uint64_t>(g) * a.rows + r) * 2u;
        out[0] = uint4{m[0], m[1], m[2], run};
        out[1] = uint4{m[3], m[4], m[5], n};
        run += n;
      }
    }
  }
  if (tid == 0) a.dense_flag[r] = ok ? 1u : 0u;
}

}  // namespace mf
