// gfx950 kernels of the restricted head path: final RMSNorm, the CSR
// restricted head (gather + fast FP32 dot + exact window rescore + merge +
// DFA advance) and the selections over precomputed logits.
//
// Build: hipcc --offload-arch=gfx950 -ffp-contract=off (see csrc/Makefile).
// -ffp-contract=off keeps every reference-order multiply-add unfused unless
// written as an explicit fma.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// ---------------------------------------------------------------------------
// Final RMSNorm in the reference FP32 CPU order (src/cpu/operators.cpp:
// 523-535): one wave per row; lane 0 runs the sequential unfused sum of
// squares over the row staged in LDS, then every lane writes
// (x * inverse) * weight.  Optionally writes an upper bound of ||y||_2 per
// row for the MFMA bounds.
// ---------------------------------------------------------------------------
template <bool kHalfIn, bool kHalfW, bool kHalfOut>
__global__ __launch_bounds__(kWave) void rms_norm_kernel(
    const void* __restrict__ input, const void* __restrict__ weight,
    void* output, float* __restrict__ row_norm, uint32_t H, float epsilon) {
  extern __shared__ float xs[];
  __shared__ float inverse_shared;
  const uint64_t r = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  for (uint32_t c = lane; c < H; c += kWave) {
    xs[c] = kHalfIn ? half_to_float(static_cast<const uint16_t*>(input)[r * H + c])
                    : static_cast<const float*>(input)[r * H + c];
  }
  __syncthreads();
  if (lane == 0) {
    float sum_squares = 0.0f;
#pragma unroll 8
    for (uint32_t c = 0; c < H; ++c) {
      const float v = xs[c];
      const float sq = v * v;
      sum_squares = sum_squares + sq;
    }
    const float mean = div_rn(sum_squares, static_cast<float>(H));
    inverse_shared = div_rn(1.0f, sqrt_rn(mean + epsilon));
  }
  __syncthreads();
  const float inverse = inverse_shared;
  float norm_sq = 0.0f;
  for (uint32_t c = lane; c < H; c += kWave) {
    const float w = kHalfW ? half_to_float(static_cast<const uint16_t*>(weight)[c])
                           : static_cast<const float*>(weight)[c];
    const float scaled = xs[c] * inverse;
    const float y = scaled * w;
    if constexpr (kHalfOut) {
      static_cast<uint16_t*>(output)[r * H + c] = float_to_half_rne(y);
    } else {
      static_cast<float*>(output)[r * H + c] = y;
      norm_sq = __builtin_fmaf(y, y, norm_sq);
    }
  }
  if (row_norm != nullptr) {
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) {
      norm_sq += __shfl_xor(norm_sq, m);
    }
    if (lane == 0) {
      // The FP32 sum of H squares is within a relative H * 2^-24 of the exact
      // value; the factor below covers that and the sqrt rounding for any
      // H <= 2^16.
      row_norm[r] = __fsqrt_rn(norm_sq) * (1.0f + 0x1p-7f);
    }
  }
}

// The decode-tail norm: the same arithmetic for FP32 rows into y (or a plain
// copy when weight is null), row norms for the MFMA bounds, and the head's work
// plan.  Lane 0 classifies its row; the last workgroup to arrive scans the
// per-row chunk counts and assigns each head workgroup its first row.
__global__ __launch_bounds__(kWave) void norm_plan_kernel(
    const float* __restrict__ x, const float* __restrict__ weight,
    float* __restrict__ y, float* __restrict__ row_norm, uint32_t rows,
    uint32_t H, float epsilon, PlanArgs plan) {
  extern __shared__ float xs[];
  __shared__ float inverse_shared;
  __shared__ uint32_t last_shared;
  const uint64_t r = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  for (uint32_t c = lane; c < H; c += kWave) xs[c] = x[r * H + c];
  __syncthreads();
  if (lane == 0) {
    if (weight != nullptr) {
      float sum_squares = 0.0f;
#pragma unroll 8
      for (uint32_t c = 0; c < H; ++c) {
        const float v = xs[c];
        const float sq = v * v;
        sum_squares = sum_squares + sq;
      }
      const float mean = div_rn(sum_squares, static_cast<float>(H));
      inverse_shared = div_rn(1.0f, sqrt_rn(mean + epsilon));
    }
    // Unrestricted rows are preset invalid too: the MFMA fallback, launched
    // after the head on the same stream, overwrites the rows it was given.
    uint32_t chunks = 0u;
    const uint32_t s = plan.row_state[r];
    bool invalid = true;
    if (s != kStateUnrestricted && s < plan.states) {
      const uint32_t b = plan.offsets[s];
      const uint32_t e = plan.offsets[s + 1];
      if (e > b && e <= plan.nnz) {
        chunks = (e - b + plan.chunk - 1) / plan.chunk;
        invalid = chunks > plan.max_chunks;
        if (invalid) chunks = 0u;
      }
    }
    if (invalid) {
      plan.out_token[r] = kInvalidToken;
      if (plan.out_score != nullptr) plan.out_score[r] = __builtin_nanf("");
      if (plan.out_next != nullptr) plan.out_next[r] = kInvalidToken;
    }
    plan.chunks_per_row[r] = chunks;
  }
  __syncthreads();
  const float inverse = inverse_shared;
  float norm_sq = 0.0f;
  for (uint32_t c = lane; c < H; c += kWave) {
    float v = xs[c];
    if (weight != nullptr) {
      const float scaled = v * inverse;
      v = scaled * weight[c];
    }
    y[r * H + c] = v;
    norm_sq = __builtin_fmaf(v, v, norm_sq);
  }
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) norm_sq += __shfl_xor(norm_sq, m);
  if (lane == 0) {
    row_norm[r] = __fsqrt_rn(norm_sq) * (1.0f + 0x1p-7f);
    last_shared = atomic_arrive(plan.counter) == rows - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (last_shared == 0u) return;
  acquire_agent();
  // exclusive scan of chunks_per_row -> prefix (one wave, 64 rows per step)
  uint32_t running = 0u;
  for (uint32_t base = 0; base < rows; base += kWave) {
    const uint32_t idx = base + lane;
    const uint32_t v = idx < rows ? plan.chunks_per_row[idx] : 0u;
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t o = __shfl_up(incl, d);
      if (static_cast<int>(lane) >= d) incl += o;
    }
    if (idx < rows) plan.prefix[idx] = running + incl - v;
    running += __shfl(incl, kWave - 1);
  }
  if (lane == 0) {
    plan.prefix[rows] = running;
    *plan.counter = 0u;
  }
  // head workgroup b owns items [W*b/G, W*(b+1)/G); it starts at the row that
  // holds item W*b/G, i.e. b in [ceil(p*G/W), ceil(q*G/W)) for a row with
  // items [p, q).
  const uint64_t W = running;
  const uint64_t G = plan.head_groups;
  if (W == 0) return;
  uint32_t row_begin_items = 0u;
  for (uint32_t base = 0; base < rows; base += kWave) {
    const uint32_t idx = base + lane;
    const uint32_t v = idx < rows ? plan.chunks_per_row[idx] : 0u;
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t o = __shfl_up(incl, d);
      if (static_cast<int>(lane) >= d) incl += o;
    }
    if (idx < rows && v > 0) {
      const uint64_t p = row_begin_items + incl - v;
      const uint64_t q = p + v;
      const uint64_t b_lo = (p * G + W - 1) / W;
      const uint64_t b_hi = (q * G + W - 1) / W;
      for (uint64_t b = b_lo; b < b_hi && b < G; ++b) plan.start_row[b] = idx;
    }
    row_begin_items += __shfl(incl, kWave - 1);
  }
}

// Reference linear_f16 arithmetic on shapes the MFMA tiling does not cover:
// one output per thread, sequential fma over the input features
// (tests/cuda/cuda_tests.cu:170-181 order), rounded to FP16.
__global__ __launch_bounds__(256) void linear_f16_simple_kernel(
    const uint16_t* __restrict__ input, const uint16_t* __restrict__ weight,
    uint16_t* __restrict__ output, uint32_t rows, uint32_t in_features,
    uint32_t out_features) {
  const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<uint64_t>(rows) * out_features) return;
  const uint64_t r = idx / out_features;
  const uint64_t o = idx % out_features;
  float s = 0.0f;
  for (uint32_t f = 0; f < in_features; ++f) {
    s = __builtin_fmaf(half_to_float(input[r * in_features + f]),
                       half_to_float(weight[o * in_features + f]), s);
  }
  output[idx] = float_to_half_rne(s);
}

// ---------------------------------------------------------------------------
// Restricted head.
// ---------------------------------------------------------------------------

struct RowList {
  const uint32_t* ids; // null: virtual list 0..count-1 (whole vocabulary)
  uint32_t count;
  uint32_t state;
  uint32_t list_begin; // offset of the list in state_tokens (CSR mode)
  int status;          // 0 ok, 1 invalid row, 2 skip (handled elsewhere)
};

__device__ RowList resolve_row(const HeadArgs& a, uint32_t r, bool lookup) {
  RowList l{nullptr, 0u, 0u, 0u, 0};
  if (a.row_state != nullptr) {
    const uint32_t s = a.row_state[r];
    l.state = s;
    if (s == kStateUnrestricted) {
      if (lookup && a.lookup_unrestricted) {
        l.count = a.V;
        return l;
      }
      l.status = 2;
      return l;
    }
    if (s >= a.states) {
      l.status = 1;
      return l;
    }
    const uint32_t b = a.offsets[s];
    const uint32_t e = a.offsets[s + 1];
    if (e <= b || e > a.nnz ||
        (a.max_chunks > 0 && (e - b + a.chunk - 1) / a.chunk > a.max_chunks)) {
      l.status = 1;
      return l;
    }
    l.ids = a.tokens + b;
    l.list_begin = b;
    l.count = e - b;
    return l;
  }
  const uint32_t c = a.fixed_counts[r];
  if (c == 0 || c > a.max_allowed) {
    l.status = 1;
    return l;
  }
  l.ids = a.fixed_ids + static_cast<uint64_t>(r) * a.max_allowed;
  l.count = c;
  return l;
}

// Cross-wave reduction scratch of a 256-thread block.
struct Red {
  float red_f[kWaves];
  uint32_t red_u[kWaves];
  uint32_t red_u2[kWaves];
  uint32_t red_t[kWaves];
  uint32_t red_p[kWaves];
  float red_s[kWaves];
};

struct HeadShared : Red {
  float sc[kHeadChunkMax];  // fast score g
  float bd[kHeadChunkMax];  // bound b
  uint32_t tk[kHeadChunkMax];
  Record recs[kHeadMaxRecords];
  uint32_t members[kHeadChunkMax];
  uint32_t n_members;
  uint32_t last;
  Record rec;
};

__device__ __forceinline__ float block_max(Red& sh, float v) {
  v = wave_max(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x % kWave) == 0) sh.red_f[w] = v;
  __syncthreads();
  float out = sh.red_f[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) out = __builtin_fmaxf(out, sh.red_f[i]);
  return out;
}

__device__ __forceinline__ uint32_t block_sum(Red& sh, uint32_t v) {
  v = wave_sum_u32(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x % kWave) == 0) sh.red_u[w] = v;
  __syncthreads();
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) out += sh.red_u[i];
  return out;
}

__device__ __forceinline__ Best block_best(Red& sh, Best b) {
  b = wave_best(b);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x % kWave) == 0) {
    sh.red_s[w] = b.score;
    sh.red_t[w] = b.token;
    sh.red_p[w] = b.pos;
  }
  __syncthreads();
  Best out{sh.red_s[0], sh.red_t[0], sh.red_p[0]};
#pragma unroll
  for (int i = 1; i < kWaves; ++i) {
    out = best_of(out, Best{sh.red_s[i], sh.red_t[i], sh.red_p[i]});
  }
  return out;
}

__device__ __forceinline__ void block_min_token(Red& sh, uint32_t& t,
                                                uint32_t& p) {
  wave_min_token(t, p);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x % kWave) == 0) {
    sh.red_u2[w] = t;
    sh.red_p[w] = p;
  }
  __syncthreads();
  t = sh.red_u2[0];
  p = sh.red_p[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) {
    if (sh.red_u2[i] < t) {
      t = sh.red_u2[i];
      p = sh.red_p[i];
    }
  }
}

__device__ __forceinline__ float half_lane(const uint4& q, int k) {
  const uint16_t* h = reinterpret_cast<const uint16_t*>(&q);
  return half_to_float(h[k]);
}

// Fast scores for H known at compile time: G lanes per candidate, each lane
// owning L = H / (8 G) 16-byte slices of the row (slice i*G + lane, so a group
// reads G*16 contiguous bytes per load), U candidates in flight per group.
// The lane's slice of y stays in registers for the whole block.
template <int H, int G, int U>
__device__ void fast_scores_vec(const HeadArgs& a, const float* ys,
                                HeadShared& sh, uint32_t n) {
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
      for (int i = 0; i < L; ++i) {
        ev[u][i] = ok[u] ? row[i * G] : uint4{0u, 0u, 0u, 0u};
      }
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
__device__ void fast_scores_generic(const HeadArgs& a, const float* ys,
                                    HeadShared& sh, uint32_t n) {
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  for (uint32_t c = w; c < n; c += kWaves) {
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

__device__ void fast_scores_lookup(const HeadArgs& a, uint32_t r,
                                   HeadShared& sh, uint32_t n) {
  const float* srow = a.scores + static_cast<uint64_t>(r) * a.V;
  const float yn = a.row_norm[r];
  for (uint32_t c = threadIdx.x; c < n; c += kThreads) {
    const uint32_t t = sh.tk[c];
    sh.sc[c] = srow[t];
    sh.bd[c] = __builtin_fmaf(a.tok_norm[t], __builtin_fmaf(a.coef, yn, a.coef2), a.slack);
  }
}

template <ScoreSource kSrc, int kH, int kG>
__device__ void fast_scores(const HeadArgs& a, uint32_t r, const float* ys,
                            HeadShared& sh, uint32_t n) {
  if constexpr (kSrc == ScoreSource::kLookup) {
    fast_scores_lookup(a, r, sh, n);
  } else if constexpr (kH > 0) {
    fast_scores_vec<kH, kG, 2>(a, ys, sh, n);
  } else {
    fast_scores_generic(a, ys, sh, n);
  }
}

// Summarises one block of n candidates (scores in sh.sc / sh.bd, ids in
// sh.tk, list positions pos0 + c) into sh.rec.  All threads must call.
__device__ void summarize_block(const HeadArgs& a, const float* ys,
                                HeadShared& sh, uint32_t n, uint32_t pos0,
                                bool invalid) {
  const int tid = threadIdx.x;
  if (invalid) {
    if (tid == 0) {
      sh.rec = Record{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""),
                      kInvalidToken, 0u, kRecInvalid, kInvalidToken, 0u};
    }
    __syncthreads();
    return;
  }
  // pass 1: finiteness, best lower bound L, lowest id
  uint32_t finite = 1u;
  float lo = -__builtin_huge_valf();
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
  for (uint32_t c = tid; c < n; c += kThreads) {
    const float g = sh.sc[c];
    const float b = sh.bd[c];
    const bool ok = __builtin_isfinite(g) && __builtin_isfinite(b) && b < 0x1p100f;
    finite &= ok ? 1u : 0u;
    lo = __builtin_fmaxf(lo, g - b);
    if (sh.tk[c] < mt) {
      mt = sh.tk[c];
      mp = pos0 + c;
    }
  }
  const uint32_t all_finite = block_sum(sh, finite ^ 1u) == 0u;
  const float L = block_max(sh, lo);
  block_min_token(sh, mt, mp);
  if (tid == 0) sh.n_members = 0u;
  __syncthreads();
  // pass 2: the window {g + b >= L}; everything when not all finite
  for (uint32_t c = tid; c < n; c += kThreads) {
    const bool member = !all_finite || (sh.sc[c] + sh.bd[c] >= L);
    if (member) {
      const uint32_t slot = atomicAdd(&sh.n_members, 1u);
      sh.members[slot] = c;
    }
  }
  __syncthreads();
  const uint32_t nm = sh.n_members;
  if (all_finite && nm == 1u) {
    if (tid == 0) {
      const uint32_t c = sh.members[0];
      const float g = sh.sc[c];
      const float b = sh.bd[c];
      sh.rec = Record{g - b, g + b, g, sh.tk[c], pos0 + c, kRecFast, mt, mp};
    }
    __syncthreads();
    return;
  }
  // ambiguous window (or non-finite inputs): reference-order rescore
  Best best = best_identity();
  for (uint32_t i = tid; i < nm; i += kThreads) {
    const uint32_t c = sh.members[i];
    const uint32_t t = sh.tk[c];
    const float s = canonical_dot_order(a.order, ys, a.emb + static_cast<uint64_t>(t) * a.H, a.H);
    best = best_of(best, best_leaf(s, t, pos0 + c));
  }
  best = block_best(sh, best);
  if (tid == 0) {
    if (best.token == kInvalidToken) {
      const float nan = __builtin_nanf("");
      sh.rec = Record{nan, nan, nan, kInvalidToken, 0u, kRecAllNan, mt, mp};
    } else {
      sh.rec = Record{best.score, best.score, best.score, best.token, best.pos,
                      kRecExact, mt, mp};
    }
  }
  __syncthreads();
}

// Merges n records of one row (in sh.recs) and writes the row's outputs.
__device__ void finalize_row(const HeadArgs& a, uint32_t r, const RowList& rl,
                             const float* ys, HeadShared& sh, uint32_t n) {
  const int tid = threadIdx.x;
  uint32_t inv = 0u;
  float lo = -__builtin_huge_valf();
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
  for (uint32_t i = tid; i < n; i += kThreads) {
    const Record& q = sh.recs[i];
    inv |= (q.kind & kRecInvalid) ? 1u : 0u;
    if (q.kind & (kRecFast | kRecExact)) lo = __builtin_fmaxf(lo, q.lower);
    if (q.min_token < mt) {
      mt = q.min_token;
      mp = q.min_pos;
    }
  }
  const bool invalid = block_sum(sh, inv) != 0u;
  const float L = block_max(sh, lo);
  block_min_token(sh, mt, mp);
  Best best = best_identity();
  if (!invalid) {
    for (uint32_t i = tid; i < n; i += kThreads) {
      const Record& q = sh.recs[i];
      if ((q.kind & (kRecFast | kRecExact)) && q.upper >= L) {
        const float s = (q.kind & kRecExact)
                            ? q.value
                            : canonical_dot_order(a.order, ys,
                                                  a.emb + static_cast<uint64_t>(q.token) * a.H, a.H);
        best = best_of(best, best_leaf(s, q.token, q.pos));
      }
    }
  }
  best = block_best(sh, best);
  if (tid == 0) {
    uint32_t token = kInvalidToken;
    uint32_t next = kInvalidToken;
    float score = __builtin_nanf("");
    if (!invalid) {
      uint32_t pos = best.pos;
      if (best.token == kInvalidToken) {
        token = mt;
        pos = mp;
        score = canonical_dot_order(a.order, ys, a.emb + static_cast<uint64_t>(mt) * a.H, a.H);
      } else {
        token = best.token;
        score = best.score;
      }
      if (rl.ids == nullptr) {
        next = kStateUnrestricted;
      } else if (a.row_state != nullptr) {
        if (a.state_next != nullptr) {
          next = a.state_next[rl.list_begin + pos];
        } else if (a.next_table != nullptr) {
          next = static_cast<uint32_t>(a.next_table[static_cast<uint64_t>(rl.state) * a.V + token]);
        }
      }
    }
    a.out_token[r] = token;
    if (a.out_score != nullptr) a.out_score[r] = score;
    if (a.out_next != nullptr) a.out_next[r] = next;
  }
}

// Loads the ids of candidates [begin, begin + n) into sh.tk; returns whether
// any id is outside the vocabulary (the reference marks the row invalid).
__device__ bool load_block_ids(const HeadArgs& a, const RowList& rl,
                               HeadShared& sh, uint32_t begin, uint32_t n) {
  uint32_t bad = 0u;
  for (uint32_t c = threadIdx.x; c < n; c += kThreads) {
    const uint32_t t = rl.ids != nullptr ? rl.ids[begin + c] : begin + c;
    bad |= t >= a.V ? 1u : 0u;
    sh.tk[c] = t < a.V ? t : 0u;
  }
  return block_sum(sh, bad) != 0u;
}

// One (row, chunk) work item; with max_chunks == 0 the workgroup owns the
// whole row (all its blocks, records merged in LDS).  ys holds the row's FP32
// hidden vector when *staged == r.
template <ScoreSource kSrc, int kH, int kG>
__device__ void head_item(const HeadArgs& a, uint32_t r, uint32_t k, float* ys,
                          HeadShared& sh, uint32_t* staged) {
  const RowList rl = resolve_row(a, r, kSrc == ScoreSource::kLookup);
  if (rl.status == 2) return;
  if (rl.status == 1) {
    if (k == 0 && threadIdx.x == 0) {
      a.out_token[r] = kInvalidToken;
      if (a.out_score != nullptr) a.out_score[r] = __builtin_nanf("");
      if (a.out_next != nullptr) a.out_next[r] = kInvalidToken;
    }
    return;
  }
  const bool multi = a.max_chunks > 0;
  const uint32_t nblocks = (rl.count + a.chunk - 1) / a.chunk;
  if (multi && k >= nblocks) return;

  if (*staged != r) {
    __syncthreads();
    for (uint32_t f = threadIdx.x; f < a.H; f += kThreads) {
      ys[f] = kSrc == ScoreSource::kDotF16Hidden
                  ? half_to_float(a.hidden16[static_cast<uint64_t>(r) * a.H + f])
                  : a.y[static_cast<uint64_t>(r) * a.H + f];
    }
    *staged = r;
    __syncthreads();
  }

  const uint32_t first = multi ? k : 0u;
  const uint32_t last = multi ? k + 1 : nblocks;
  for (uint32_t blk = first; blk < last; ++blk) {
    const uint32_t begin = blk * a.chunk;
    const uint32_t n = rl.count - begin < a.chunk ? rl.count - begin : a.chunk;
    const bool invalid = load_block_ids(a, rl, sh, begin, n);
    if (!invalid) {
      fast_scores<kSrc, kH, kG>(a, r, ys, sh, n);
    }
    __syncthreads();
    summarize_block(a, ys, sh, n, begin, invalid);
    if (threadIdx.x == 0) sh.recs[multi ? 0 : blk] = sh.rec;
    __syncthreads();
  }

  if (!multi || nblocks == 1) {
    finalize_row(a, r, rl, ys, sh, multi ? 1u : nblocks);
    __syncthreads();
    return;
  }
  // several workgroups share the row: publish, and the last one merges
  Record* row_recs = a.records + static_cast<uint64_t>(r) * a.max_chunks;
  if (threadIdx.x == 0) {
    row_recs[k] = sh.rec;
    const uint32_t arrived = atomic_arrive(&a.counters[r]);
    sh.last = arrived == nblocks - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (sh.last == 0u) return;
  acquire_agent();
  for (uint32_t i = threadIdx.x; i < nblocks; i += kThreads) {
    sh.recs[i] = row_recs[i];
  }
  if (threadIdx.x == 0) a.counters[r] = 0u;
  __syncthreads();
  finalize_row(a, r, rl, ys, sh, nblocks);
  __syncthreads();
}

// Grid mode: blockIdx.x = k * rows + r.
template <ScoreSource kSrc, int kH, int kG>
__global__ __launch_bounds__(kThreads) void head_kernel(HeadArgs a) {
  extern __shared__ float ys[];
  __shared__ HeadShared sh;
  uint32_t staged = kInvalidToken;
  head_item<kSrc, kH, kG>(a, blockIdx.x % a.rows, blockIdx.x / a.rows, ys, sh, &staged);
}

// Planned mode: workgroup b walks its contiguous range of work items.
template <ScoreSource kSrc, int kH, int kG>
__global__ __launch_bounds__(kThreads) void head_planned_kernel(HeadArgs a) {
  extern __shared__ float ys[];
  __shared__ HeadShared sh;
  const uint64_t W = a.prefix[a.rows];
  const uint64_t G = gridDim.x;
  const uint64_t w0 = W * blockIdx.x / G;
  const uint64_t w1 = W * (blockIdx.x + 1) / G;
  if (w0 >= w1) return;
  uint32_t r = a.start_row[blockIdx.x];
  uint32_t staged = kInvalidToken;
  for (uint64_t w = w0; w < w1; ++w) {
    while (w >= static_cast<uint64_t>(a.prefix[r + 1])) ++r;
    head_item<kSrc, kH, kG>(a, r, static_cast<uint32_t>(w - a.prefix[r]), ys, sh, &staged);
  }
}

// ---------------------------------------------------------------------------
// Selection over precomputed logits (reference greedy.cu:21-131).
// ---------------------------------------------------------------------------

template <bool kHalf>
__device__ __forceinline__ float logit_at(const void* p, uint64_t i) {
  return kHalf ? half_to_float(static_cast<const uint16_t*>(p)[i])
               : static_cast<const float*>(p)[i];
}

template <bool kHalf>
__global__ __launch_bounds__(kThreads) void greedy_kernel(
    const void* __restrict__ logits, uint32_t* __restrict__ tokens, uint32_t V) {
  __shared__ Red sh;
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * V;
  Best best = best_identity();
  for (uint32_t c = threadIdx.x; c < V; c += kThreads) {
    best = best_of(best, best_leaf(logit_at<kHalf>(logits, base + c), c, c));
  }
  best = block_best(sh, best);
  if (threadIdx.x == 0) {
    // src/cuda/greedy.cu:57: no comparable value selects token 0
    tokens[blockIdx.x] = best.token == kInvalidToken ? 0u : best.token;
  }
}

template <bool kHalf>
__global__ __launch_bounds__(kThreads) void restricted_greedy_kernel(
    const void* __restrict__ logits, const uint32_t* __restrict__ allowed,
    const uint32_t* __restrict__ counts, uint32_t* __restrict__ tokens,
    uint32_t V, uint32_t max_allowed) {
  __shared__ Red sh;
  const uint32_t r = blockIdx.x;
  const uint32_t count = counts[r];
  const bool row_invalid = count == 0 || count > max_allowed;
  const uint64_t base = static_cast<uint64_t>(r) * V;
  Best best = best_identity();
  uint32_t bad = 0u;
  uint32_t mt = kInvalidToken;
  uint32_t mp = 0u;
  if (!row_invalid) {
    for (uint32_t j = threadIdx.x; j < count; j += kThreads) {
      const uint32_t t = allowed[static_cast<uint64_t>(r) * max_allowed + j];
      if (t >= V) {
        bad = 1u;
        continue;
      }
      if (t < mt) {
        mt = t;
        mp = j;
      }
      best = best_of(best, best_leaf(logit_at<kHalf>(logits, base + t), t, j));
    }
  }
  const bool invalid = block_sum(sh, bad) != 0u || row_invalid;
  best = block_best(sh, best);
  block_min_token(sh, mt, mp);
  if (threadIdx.x == 0) {
    tokens[r] = invalid ? kInvalidToken : (best.token == kInvalidToken ? mt : best.token);
  }
}

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(uint4* p, uint64_t n16) {
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n16;
       i += static_cast<uint64_t>(gridDim.x) * kThreads) {
    p[i] = uint4{0u, 0u, 0u, 0u};
  }
}

} // namespace

hipError_t launch_rms_norm(const void* input, bool half_input, const void* weight,
                           bool half_weight, void* output, bool half_output,
                           float* row_norm, uint32_t rows, uint32_t hidden,
                           float epsilon, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(hidden) * sizeof(float);
  const dim3 grid(rows), block(kWave);
  if (half_input && half_weight && half_output) {
    hipLaunchKernelGGL((rms_norm_kernel<true, true, true>), grid, block, lds, stream,
                       input, weight, output, nullptr, hidden, epsilon);
  } else if (!half_input && !half_weight && !half_output) {
    hipLaunchKernelGGL((rms_norm_kernel<false, false, false>), grid, block, lds, stream,
                       input, weight, output, row_norm, hidden, epsilon);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <ScoreSource kSrc, int kH, int kG>
void launch_head_variant(const HeadArgs& args, uint32_t groups, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(args.H) * sizeof(float);
  if (args.prefix != nullptr) {
    hipLaunchKernelGGL((head_planned_kernel<kSrc, kH, kG>), dim3(groups), dim3(kThreads), lds,
                       stream, args);
  } else {
    const uint32_t slots = args.max_chunks > 0 ? args.max_chunks : 1u;
    hipLaunchKernelGGL((head_kernel<kSrc, kH, kG>), dim3(args.rows * slots), dim3(kThreads), lds,
                       stream, args);
  }
}

hipError_t launch_head(ScoreSource source, const HeadArgs& args, uint32_t groups,
                       hipStream_t stream) {
  const bool aligned = (reinterpret_cast<uintptr_t>(args.emb) & 15u) == 0;
  switch (source) {
    case ScoreSource::kDotF32:
      if (args.H == 576 && aligned) {
        launch_head_variant<ScoreSource::kDotF32, 576, 8>(args, groups, stream);
      } else if (args.H == 2048 && aligned) {
        launch_head_variant<ScoreSource::kDotF32, 2048, 32>(args, groups, stream);
      } else {
        launch_head_variant<ScoreSource::kDotF32, 0, 64>(args, groups, stream);
      }
      break;
    case ScoreSource::kDotF16Hidden:
      if (args.H == 576 && aligned) {
        launch_head_variant<ScoreSource::kDotF16Hidden, 576, 8>(args, groups, stream);
      } else {
        launch_head_variant<ScoreSource::kDotF16Hidden, 0, 64>(args, groups, stream);
      }
      break;
    case ScoreSource::kLookup:
      launch_head_variant<ScoreSource::kLookup, 0, 64>(args, groups, stream);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_norm_plan(const float* x, const float* weight, float* y,
                            float* row_norm, uint32_t rows, uint32_t hidden,
                            float epsilon, const PlanArgs& plan, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(hidden) * sizeof(float);
  hipLaunchKernelGGL(norm_plan_kernel, dim3(rows), dim3(kWave), lds, stream, x, weight, y,
                     row_norm, rows, hidden, epsilon, plan);
  return hipGetLastError();
}

hipError_t launch_linear_f16_simple(const uint16_t* input, const uint16_t* weight,
                                    uint16_t* output, uint32_t rows, uint32_t in_features,
                                    uint32_t out_features, hipStream_t stream) {
  const uint64_t n = static_cast<uint64_t>(rows) * out_features;
  const uint64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(linear_f16_simple_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     stream, input, weight, output, rows, in_features, out_features);
  return hipGetLastError();
}

hipError_t launch_greedy(const void* logits, bool half, uint32_t* tokens,
                         uint32_t rows, uint32_t vocab, hipStream_t stream) {
  if (half) {
    hipLaunchKernelGGL((greedy_kernel<true>), dim3(rows), dim3(kThreads), 0, stream,
                       logits, tokens, vocab);
  } else {
    hipLaunchKernelGGL((greedy_kernel<false>), dim3(rows), dim3(kThreads), 0, stream,
                       logits, tokens, vocab);
  }
  return hipGetLastError();
}

hipError_t launch_restricted_greedy(const void* logits, bool half,
                                    const uint32_t* allowed, const uint32_t* counts,
                                    uint32_t* tokens, uint32_t rows, uint32_t vocab,
                                    uint32_t max_allowed, hipStream_t stream) {
  if (half) {
    hipLaunchKernelGGL((restricted_greedy_kernel<true>), dim3(rows), dim3(kThreads), 0,
                       stream, logits, allowed, counts, tokens, vocab, max_allowed);
  } else {
    hipLaunchKernelGGL((restricted_greedy_kernel<false>), dim3(rows), dim3(kThreads), 0,
                       stream, logits, allowed, counts, tokens, vocab, max_allowed);
  }
  return hipGetLastError();
}

hipError_t launch_fill_zero(void* address, uint64_t bytes, hipStream_t stream) {
  const uint64_t n16 = bytes / 16;
  if (n16 == 0) return hipSuccess;
  uint64_t blocks = (n16 + kThreads - 1) / kThreads;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                     stream, static_cast<uint4*>(address), n16);
  return hipGetLastError();
}

} // namespace mf
