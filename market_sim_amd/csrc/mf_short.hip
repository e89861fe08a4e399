// One-kernel decode tail for packs of short lists (every list at most
// kShortListMax ids, no unrestricted rows): the decode loop's case.
//
// One workgroup of four waves per row; every thread rescores one candidate
// in the reference order (greedy.cu:171-176), so every score is exact and
// no window, bound or record is needed.  Wave 0 runs the norm's
// reference-order chain (operators.cpp:520-534) while waves 1-3 stage the
// first round of candidate rows in LDS (every list of at most 128 ids in
// one round at H <= 576; 24 pieces of 16 bytes per lane in flight).  The workgroup selects by
// the reference rule (greedy.cu:84-100, 177-211: highest score, lowest id on
// ties, NaN never wins, an all-NaN row takes its lowest id) and advances the
// DFA.  The arithmetic is that of the multi-kernel path (row_list,
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
  for (uint32_t q0 = lane; q0 < total; q0 += kWave * kBatch) {
    uint4 v[kBatch];
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t q = q0 + u * kWave;
      const uint32_t j = part + parts * (q / per);
      const uint32_t id = q < total ? sh.cand[j] : kInvalidToken;
      v[u] = id < n.V ? reinterpret_cast<const uint4*>(f.emb + static_cast<uint64_t>(id) * H)[q % per]
                      : uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t q = q0 + u * kWave;
      if (q < total) {
        const uint32_t j = part + parts * (q / per);
        reinterpret_cast<uint4*>(es + j * rs)[q % per] = v[u];
      }
    }
  }
}

// Writes row r's outputs from the workgroup's per-wave results (thread 0).
__device__ inline void short_select(const TailNormArgs& n, const FinalizeArgs& f,
                                    const ShortShared& sh, const float* ys, uint32_t r,
                                    const RowMeta& meta) {
  const uint32_t H = n.H;
  uint32_t* slot = next_state_slot(n.out_next, n.row_sequence, n.capacity, r);
  if (sh.invalid) {
    // an id outside the vocabulary makes the row invalid (greedy.cu:163-166)
    f.out_token[r] = kInvalidToken;
    if (f.out_score != nullptr) f.out_score[r] = __builtin_nanf("");
    if (slot != nullptr) *slot = kInvalidToken;
    return;
  }
  Best b = sh.best[0];
  uint32_t mt = sh.mt[0];
  uint32_t mp = sh.mp[0];
  for (uint32_t w = 1; w < kShortWaves; ++w) {
    b = best_of(b, sh.best[w]);
    if (sh.mt[w] < mt || (sh.mt[w] == mt && sh.mp[w] < mp)) {
      mt = sh.mt[w];
      mp = sh.mp[w];
    }
  }
  uint32_t token = b.token;
  uint32_t pos = b.pos;
  float score = b.score;
  if (token == kInvalidToken) {
    // every score is NaN: the lowest id, with its own reference-order score
    token = mt;
    pos = mp;
    const uint16_t* row = f.emb + static_cast<uint64_t>(token) * H;
    score = f.order == 1 ? chain_lds<true>(ys, row, H) : chain_lds<false>(ys, row, H);
  }
  uint32_t next = kInvalidToken;
  if (f.state_next != nullptr) {
    next = f.state_next[meta.list_begin + pos];
  } else if (f.next_table != nullptr) {
    next = static_cast<uint32_t>(f.next_table[static_cast<uint64_t>(meta.state) * f.V + token]);
  }
  f.out_token[r] = token;
  if (f.out_score != nullptr) f.out_score[r] = score;
  if (slot != nullptr) *slot = next;
}

__global__ __launch_bounds__(kShortThreads) void short_tail_kernel(TailNormArgs n, FinalizeArgs f,
                                                                   uint32_t stage_rows) {
  extern __shared__ __align__(16) float lds[];
  __shared__ ShortShared sh;
  const uint32_t H = n.H;
  const uint32_t tid = threadIdx.x;
  const uint32_t wave = tid / kWave;
  const uint32_t lane = tid % kWave;
  const uint32_t r = blockIdx.x;
  float* xs = lds;               // x, then y in place
  float* sq = lds + H;
  float* ws = lds + 2u * H;
  uint16_t* es = reinterpret_cast<uint16_t*>(lds + 3u * H);
  const uint32_t rs = H + 8u;
  const bool weighted = n.weight != nullptr;

  if (tid == 0) {
    const RowList l = row_list(n, r);
    sh.meta = l.meta;
    sh.q = l.q;
    sh.b = l.b;
    sh.e = l.e;
    sh.invalid = 0u;
  }
  {
    const float4* x4 = reinterpret_cast<const float4*>(n.x + static_cast<uint64_t>(r) * H);
    const float4* w4 = reinterpret_cast<const float4*>(n.weight);
    for (uint32_t q = tid; q < H / 4u; q += kShortThreads) {
      const float4 v = x4[q];
      reinterpret_cast<float4*>(xs)[q] = v;
      reinterpret_cast<float4*>(sq)[q] = float4{v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w};
      if (weighted) reinterpret_cast<float4*>(ws)[q] = w4[q];
    }
  }
  __syncthreads();
  const RowMeta meta = sh.meta;
  if (meta.kind != kRowRestricted) {
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
  const uint32_t count = meta.count;
  const uint32_t m0 = count < stage_rows ? count : stage_rows;
  if (wave == 0) {
    const float sum_squares = weighted ? sequential_sum_wave(sq, H) : 0.0f;
    if (lane == 0) sh.inv = weighted ? norm_inverse(sum_squares, H, n.epsilon) : 1.0f;
  } else {
    stage_part(n, f, sh, es, 0u, m0, wave - 1u, kShortWaves - 1u);
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
  uint32_t bad = 0u;
  for (uint32_t base = 0; base < count; base += stage_rows) {
    const uint32_t m = count - base < stage_rows ? count - base : stage_rows;
    if (base > 0) {
      __syncthreads();
      stage_part(n, f, sh, es, base, m, wave, kShortWaves);
      __syncthreads();
    }
    if (tid < m) {
      const uint32_t token = sh.cand[tid];
      const uint32_t pos = base + tid;
      if (token >= n.V) {
        bad = 1u;
      } else {
        const float s = f.order == 1 ? chain_lds<true>(xs, es + tid * rs, H)
                                     : chain_lds<false>(xs, es + tid * rs, H);
        best = best_of(best, best_leaf(s, token, pos));
        if (token < mt) {
          mt = token;
          mp = pos;
        }
      }
    }
  }
  if (bad) sh.invalid = 1u;
  best = wave_best(best);
  wave_min_token(mt, mp);
  if (lane == 0) {
    sh.best[wave] = best;
    sh.mt[wave] = mt;
    sh.mp[wave] = mp;
  }
  __syncthreads();
  if (tid == 0) short_select(n, f, sh, xs, r, meta);
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

hipError_t launch_short(const TailNormArgs& n, const FinalizeArgs& f, hipStream_t stream) {
  const uint32_t stage_rows = short_stage_rows(n.H, n.max_count);
  if (n.H % 8u != 0 || stage_rows == 0 || n.max_count > kShortListMax) {
    return hipErrorInvalidValue;
  }
  const size_t lds = 3u * static_cast<size_t>(n.H) * sizeof(float) +
                     static_cast<size_t>(stage_rows) * 2u * (n.H + 8u);
  hipLaunchKernelGGL(short_tail_kernel, dim3(n.rows), dim3(kShortThreads), lds, stream, n,
                     f, stage_rows);
  return hipGetLastError();
}

}  // namespace mf
