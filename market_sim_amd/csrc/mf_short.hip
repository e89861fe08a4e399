// One-kernel decode tail for packs of short lists (no unrestricted rows):
// the decode loop's case, and small packs of lists up to kShortPartsMax
// parts of a workgroup's stage.
//
// A row's list is cut into parts of per_part candidates, one workgroup of
// four waves each; every thread rescores one candidate in the reference
// order (greedy.cu:171-176), so every score is exact and no window, bound or
// record of fast scores is needed.  Wave 0 runs the norm's reference-order
// chain (operators.cpp:520-534) while waves 1-3 stage the part's candidate
// rows in LDS (24 pieces of 16 bytes per lane in flight).  The workgroup
// selects by the reference rule (greedy.cu:84-100, 177-211: highest score,
// lowest id on ties, NaN never wins, an all-NaN row takes its lowest id).
// With one part the workgroup writes the row's outputs and advances the
// DFA; with several, each part leaves its selection in a record and the last
// part to arrive merges the records (the same rule: the merge of the parts'
// selections is the selection over the whole list) and finishes the row.
// Records and counters are read and written with device-coherent accesses
// only, so no part writes back or invalidates an L2.
// The arithmetic is that of the multi-kernel path (row_list,
// sequential_sum, norm_inverse, chain_lds), so both give identical bits.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"
#include "mf_finalize.hpp"
#include "mf_prep.hpp"

namespace mf {
namespace {

constexpr uint32_t kShortWaves = 4;
constexpr uint32_t kShortThreads = kShortWaves * kWave;

// The selection of a list (or part of one): the best candidate, the lowest
// id and its position (for an all-NaN list), and whether an id lay outside
// the vocabulary.
struct ShortSel {
  Best best;
  uint32_t next;   // the best candidate's next state
  uint32_t mt;
  uint32_t mp;
  uint32_t mnext;  // the lowest id's next state
  uint32_t invalid;
};

struct ShortShared {
  RowMeta meta;
  uint32_t q;
  uint32_t b;
  uint32_t e;
  float inv;
  uint32_t invalid;
  Best best[kShortWaves];
  uint32_t mt[kShortWaves];
  uint32_t mp[kShortWaves];
  uint32_t cand[kShortListMax];
  uint32_t nx[kShortListMax];  // each candidate's next state
  ShortSel parts[kShortPartsMax];  // the last part's copy of every part's record
};

// Stages candidates base + j of the row, j = part, part + parts, ... < m,
// into staged row j (stride H + 8 halves: lanes reading rows j and j + 1 at
// one offset fall in different LDS banks).  Called by one wave; ids outside
// the vocabulary are not dereferenced (their staged row is zeros, and the
// row is reported invalid).
__device__ inline void stage_part(const TailNormArgs& n, const FinalizeArgs& f, ShortShared& sh,
                                  uint16_t* es, uint32_t base, uint32_t m, uint32_t part,
                                  uint32_t parts) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t H = n.H;
  const uint32_t rs = H + 8u;
  for (uint32_t j = part + parts * lane; j < m; j += parts * kWave) {
    sh.cand[j] = f.tokens[sh.b + base + j];
  }
  wave_sync();
  const uint32_t cnt = m > part ? (m - part + parts - 1u) / parts : 0u;
  constexpr uint32_t kBatch = 24;
  const uint32_t per = H / 8u;
  const uint32_t total = cnt * per;
  // piece q = q0 + u kWave of the staged rows is piece q % per of the
  // part's candidate q / per: each lane steps (candidate, piece) by kWave
  // pieces from one u to the next (one division per lane, not per piece)
  const uint32_t step_c = kWave / per;
  const uint32_t step_p = kWave % per;
  uint32_t c0 = lane / per;  // the lane's first piece of a batch
  uint32_t p0 = lane % per;
  for (uint32_t q0 = lane; q0 < total; q0 += kWave * kBatch) {
    uint4 v[kBatch];
    uint32_t c = c0;
    uint32_t pp = p0;
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t q = q0 + u * kWave;
      const uint32_t id = q < total ? sh.cand[part + parts * c] : kInvalidToken;
      v[u] = id < n.V ? reinterpret_cast<const uint4*>(f.emb + static_cast<uint64_t>(id) * H)[pp]
                      : uint4{0u, 0u, 0u, 0u};
      c += step_c;
      pp += step_p;
      if (pp >= per) {
        pp -= per;
        ++c;
      }
    }
    c = c0;
    pp = p0;
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t q = q0 + u * kWave;
      if (q < total) reinterpret_cast<uint4*>(es + (part + parts * c) * rs)[pp] = v[u];
      c += step_c;
      pp += step_p;
      if (pp >= per) {
        pp -= per;
        ++c;
      }
    }
    c0 = c;
    p0 = pp;
  }
}

__device__ __forceinline__ ShortSel merge_sel(ShortSel a, const ShortSel& b) {
  const Best m = best_of(a.best, b.best);
  if (m.token != a.best.token || m.pos != a.best.pos) a.next = b.next;
  a.best = m;
  if (b.mt < a.mt || (b.mt == a.mt && b.mp < a.mp)) {
    a.mt = b.mt;
    a.mp = b.mp;
    a.mnext = b.mnext;
  }
  a.invalid |= b.invalid;
  return a;
}

// Writes row r's outputs from the selection over its whole list (one thread).
__device__ inline void short_finish(const TailNormArgs& n, const FinalizeArgs& f, const float* ys,
                                    uint32_t r, const RowMeta& meta, const ShortSel& sel) {
  const uint32_t H = n.H;
  uint32_t* slot = next_state_slot(n.out_next, n.row_sequence, n.capacity, r);
  if (sel.invalid) {
    // an id outside the vocabulary makes the row invalid (greedy.cu:163-166)
    f.out_token[r] = kInvalidToken;
    if (f.out_score != nullptr) f.out_score[r] = __builtin_nanf("");
    if (slot != nullptr) *slot = kInvalidToken;
    return;
  }
  uint32_t token = sel.best.token;
  uint32_t next = sel.next;
  float score = sel.best.score;
  if (token == kInvalidToken) {
    // every score is NaN: the lowest id, with its own reference-order score
    token = sel.mt;
    next = sel.mnext;
    const uint16_t* row = f.emb + static_cast<uint64_t>(token) * H;
    score = f.order == 1 ? chain_lds<true>(ys, row, H) : chain_lds<false>(ys, row, H);
  }
  (void)meta;
  f.out_token[r] = token;
  if (f.out_score != nullptr) f.out_score[r] = score;
  if (slot != nullptr) *slot = next;
}

__global__ __launch_bounds__(kShortThreads) void short_tail_kernel(TailNormArgs n, FinalizeArgs f,
                                                                   ShortSplit split) {
  extern __shared__ __align__(16) float lds[];
  __shared__ ShortShared sh;
  const uint32_t H = n.H;
  const uint32_t tid = threadIdx.x;
  const uint32_t wave = tid / kWave;
  const uint32_t lane = tid % kWave;
  const uint32_t part = blockIdx.x;
  const uint32_t r = blockIdx.y;
  float* xs = lds;               // x, then y in place
  float* sq = lds + H;
  float* ws = lds + 2u * H;
  uint16_t* es = reinterpret_cast<uint16_t*>(lds + 3u * H);
  const bool weighted = n.weight != nullptr;

  // thread 0 walks the row's list while waves 1-3 bring in x (and its
  // squares) and the weight
  if (tid == 0) {
    const RowList l = row_list(n, r);
    sh.meta = l.meta;
    sh.q = l.q;
    sh.b = l.b;
    sh.e = l.e;
    sh.invalid = 0u;
  } else if (wave > 0) {
    const float4* x4 = reinterpret_cast<const float4*>(n.x + static_cast<uint64_t>(r) * H);
    const float4* w4 = reinterpret_cast<const float4*>(n.weight);
    for (uint32_t q = tid - kWave; q < H / 4u; q += kShortThreads - kWave) {
      const float4 v = x4[q];
      reinterpret_cast<float4*>(xs)[q] = v;
      reinterpret_cast<float4*>(sq)[q] = float4{v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w};
      if (weighted) reinterpret_cast<float4*>(ws)[q] = w4[q];
    }
  }
  __syncthreads();
  const RowMeta meta = sh.meta;
  const bool restricted = meta.kind == kRowRestricted;
  const uint32_t count = meta.count;
  // the row's parts: one unless a restricted list is longer than a part
  const uint32_t parts =
      restricted && count > split.per_part ? (count + split.per_part - 1u) / split.per_part : 1u;
  if (part >= parts) return;
  if (!restricted) {
    // invalid rows, finished rows (an empty list: the state is held when
    // asked to), and unrestricted rows, which this path is never given
    if (tid == 0) {
      f.out_token[r] = kInvalidToken;
      if (f.out_score != nullptr) f.out_score[r] = __builtin_nanf("");
      if (n.out_next != nullptr && sh.q < n.capacity) {
        const uint32_t s = meta.state;
        n.out_next[sh.q] = (n.hold && s < n.states && sh.e == sh.b) ? s : kInvalidToken;
      }
    }
    return;
  }
  // this part's candidates: list positions base .. base + m - 1
  const uint32_t base = part * split.per_part;
  const uint32_t m = count - base < split.per_part ? count - base : split.per_part;
  if (wave == 0) {
    const float sum_squares = weighted ? sequential_sum_wave(sq, H) : 0.0f;
    if (lane == 0) sh.inv = weighted ? norm_inverse(sum_squares, H, n.epsilon) : 1.0f;
  } else {
    stage_part(n, f, sh, es, base, m, wave - 1u, kShortWaves - 1u);
  }
  __syncthreads();
  // y = (x * inv) * w in the reference's roundings (operators.cpp:533-534)
  const float inv = sh.inv;
  if (weighted) {
    for (uint32_t c = tid; c < H; c += kShortThreads) xs[c] = (xs[c] * inv) * ws[c];
  }
  __syncthreads();

  Best best = best_identity();
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
  if (tid < m) {
    const uint32_t token = sh.cand[tid];
    const uint32_t pos = base + tid;
    if (token >= n.V) {
      sh.invalid = 1u;
    } else {
      // the candidate's next state, loaded under the chain (greedy.cu
      // leaves the advance to the caller; operators.cpp steps the DFA)
      uint32_t nx = kInvalidToken;
      if (f.state_next != nullptr) {
        nx = f.state_next[meta.list_begin + pos];
      } else if (f.next_table != nullptr) {
        nx = static_cast<uint32_t>(f.next_table[static_cast<uint64_t>(meta.state) * f.V + token]);
      }
      __builtin_amdgcn_sched_barrier(0);  // the load goes out before the chain
      const uint32_t rs = H + 8u;
      const float s = f.order == 1 ? chain_lds<true>(xs, es + tid * rs, H)
                                   : chain_lds<false>(xs, es + tid * rs, H);
      best = best_leaf(s, token, pos);
      mt = token;
      mp = pos;
      sh.nx[tid] = nx;
    }
  }
  best = wave_best(best);
  wave_min_token(mt, mp);
  if (lane == 0) {
    sh.best[wave] = best;
    sh.mt[wave] = mt;
    sh.mp[wave] = mp;
  }
  __syncthreads();
  if (wave != 0) return;
  // wave 0 finishes: the part's selection (the same in every lane)
  ShortSel sel{sh.best[0], 0u, sh.mt[0], sh.mp[0], 0u, sh.invalid};
  for (uint32_t w = 1; w < kShortWaves; ++w) {
    sel = merge_sel(sel, ShortSel{sh.best[w], 0u, sh.mt[w], sh.mp[w], 0u, 0u});
  }
  if (sel.best.token != kInvalidToken) sel.next = sh.nx[sel.best.pos - base];
  if (sel.mt != kInvalidToken) sel.mnext = sh.nx[sel.mp - base];
  if (parts == 1u) {
    if (lane == 0) short_finish(n, f, xs, r, meta, sel);
    return;
  }
  // The record and the arrival counter are device-coherent accesses
  // (relaxed atomics at agent scope), so no fence has to write back or
  // invalidate a whole L2: the record's stores are complete before this
  // part arrives, and the last part reads the records after its arrival.
  uint32_t* rec = reinterpret_cast<uint32_t*>(split.records + static_cast<uint64_t>(r) * split.parts);
  constexpr uint32_t kWords = sizeof(ShortPartRecord) / 4u;
  static_assert(kWords == 8, "a record is eight words");
  if (lane == 0) {
    const uint32_t mine[8] = {__float_as_uint(sel.best.score), sel.best.token, sel.best.pos,
                              sel.next, sel.mt, sel.mp, sel.mnext, sel.invalid};
#pragma unroll
    for (uint32_t k = 0; k < 8u; ++k) {
      __hip_atomic_store(rec + part * kWords + k, mine[k], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  uint32_t arrived = 0u;
  if (lane == 0) {
    arrived = __hip_atomic_fetch_add(split.counts + r, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
  }
  arrived = __builtin_amdgcn_readfirstlane(arrived);
  if (arrived != parts - 1u) return;
  asm volatile("" ::: "memory");
  // the last part: every record is complete; lane k reads part k's, and the
  // counter is zero again for the next call
  if (lane == 0) __hip_atomic_store(split.counts + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane < parts) {
    uint32_t x[8];
#pragma unroll
    for (uint32_t i = 0; i < 8u; ++i) {
      x[i] = __hip_atomic_load(rec + lane * kWords + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    sh.parts[lane] = ShortSel{Best{__uint_as_float(x[0]), x[1], x[2]}, x[3], x[4], x[5], x[6], x[7]};
  }
  wave_sync();
  if (lane != 0) return;
  ShortSel all{best_identity(), kInvalidToken, kInvalidToken, 0u, kInvalidToken, 0u};
  for (uint32_t k = 0; k < parts; ++k) all = merge_sel(all, sh.parts[k]);
  short_finish(n, f, xs, r, meta, all);
}

}  // namespace

uint32_t short_stage_rows(uint32_t H, uint32_t max_count) {
  const uint64_t fixed = 3ull * H * sizeof(float);
  const uint64_t per = 2ull * (H + 8u);
  if (fixed + per > kShortLdsBytes) return 0u;
  uint64_t rows = (kShortLdsBytes - fixed) / per;
  if (rows > kShortListMax) rows = kShortListMax;
  const uint32_t want = max_count == 0 ? 1u : max_count;
  return static_cast<uint32_t>(rows < want ? rows : want);
}

hipError_t launch_short(const TailNormArgs& n, const FinalizeArgs& f, const ShortSplit& split,
                        hipStream_t stream) {
  const uint32_t stage_rows = short_stage_rows(n.H, split.per_part);
  if (n.H % 8u != 0 || stage_rows == 0 || split.per_part == 0 || stage_rows < split.per_part ||
      split.per_part > kShortListMax || split.parts == 0 || split.parts > kShortPartsMax ||
      static_cast<uint64_t>(split.per_part) * split.parts < n.max_count ||
      (split.parts > 1u && (split.records == nullptr || split.counts == nullptr ||
                            n.rows > kShortCountRows))) {
    return hipErrorInvalidValue;
  }
  const size_t lds = 3u * static_cast<size_t>(n.H) * sizeof(float) +
                     static_cast<size_t>(split.per_part) * 2u * (n.H + 8u);
  hipLaunchKernelGGL(short_tail_kernel, dim3(split.parts, n.rows), dim3(kShortThreads), lds,
                     stream, n, f, split);
  return hipGetLastError();
}

}  // namespace mf
