// gfx950 kernels of the reference operators: RMSNorm, the fixed-width
// restricted output head (restricted_output_head_f16), the selections over
// precomputed logits and the small-shape linear_f16.  The decode tail lives
// in mf_tail.hip.
//
// Build: hipcc --offload-arch=gfx950 -ffp-contract=off (see csrc/Makefile).
// -ffp-contract=off keeps every reference-order multiply-add unfused unless
// written as an explicit fma.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"
#include "mf_norm.hpp"

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
// Rows up to this width also stage the weight in LDS (3 H floats in all).
constexpr uint32_t kNormStagedWeightMax = 8192;

template <bool kHalfIn, bool kHalfW, bool kHalfOut>
__global__ __launch_bounds__(kWave) void rms_norm_kernel(
    const void* __restrict__ input, const void* __restrict__ weight,
    void* output, float* __restrict__ row_norm, uint32_t H, float epsilon) {
  // [H] x, [H] x * x, and [H] weight when H <= kNormStagedWeightMax
  extern __shared__ __align__(16) float xs[];
  __shared__ float inverse_shared;
  const bool stage_w = H <= kNormStagedWeightMax;
  float* sq = xs + H;
  float* ws = xs + 2u * H;
  const uint64_t r = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  // x and the weight staged with four 4-element loads of each per lane in
  // flight before the LDS stores (one memory round trip per 1024 features)
  constexpr uint32_t kInBytes = kHalfIn ? 2u : 4u;
  constexpr uint32_t kWBytes = kHalfW ? 2u : 4u;
  const bool vec = (H & 3u) == 0 &&
                   (reinterpret_cast<uintptr_t>(input) & (4u * kInBytes - 1u)) == 0 &&
                   (reinterpret_cast<uintptr_t>(weight) & (4u * kWBytes - 1u)) == 0;
  auto load4 = [](const void* base, uint64_t q, auto half) -> float4 {
    if constexpr (decltype(half)::value) {
      const uint2 h = static_cast<const uint2*>(base)[q];
      return float4{half_to_float(static_cast<uint16_t>(h.x)), half_to_float(static_cast<uint16_t>(h.x >> 16)),
                    half_to_float(static_cast<uint16_t>(h.y)), half_to_float(static_cast<uint16_t>(h.y >> 16))};
    } else {
      return static_cast<const float4*>(base)[q];
    }
  };
  using HalfIn = std::integral_constant<bool, kHalfIn>;
  using HalfW = std::integral_constant<bool, kHalfW>;
  if (vec) {
    constexpr uint32_t kBatch = 4;
    const uint32_t n4 = H / 4u;
    for (uint32_t base = lane; base < n4; base += kWave * kBatch) {
      float4 v[kBatch];
      float4 w4[kBatch];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t q = base + u * kWave;
        v[u] = q < n4 ? load4(input, r * n4 + q, HalfIn{}) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        w4[u] = (stage_w && q < n4) ? load4(weight, q, HalfW{}) : float4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t q = base + u * kWave;
        if (q < n4) {
          reinterpret_cast<float4*>(xs)[q] = v[u];
          reinterpret_cast<float4*>(sq)[q] =
              float4{v[u].x * v[u].x, v[u].y * v[u].y, v[u].z * v[u].z, v[u].w * v[u].w};
          if (stage_w) reinterpret_cast<float4*>(ws)[q] = w4[u];
        }
      }
    }
  } else {
    for (uint32_t c = lane; c < H; c += kWave) {
      const float v = kHalfIn ? half_to_float(static_cast<const uint16_t*>(input)[r * H + c])
                              : static_cast<const float*>(input)[r * H + c];
      xs[c] = v;
      sq[c] = v * v;
      if (stage_w) {
        ws[c] = kHalfW ? half_to_float(static_cast<const uint16_t*>(weight)[c])
                       : static_cast<const float*>(weight)[c];
      }
    }
  }
  __syncthreads();
  // sum of the squares in feature order, then mean, + epsilon, sqrt and
  // reciprocal, each rounded once (rms_norm.cu:104-182)
  const float sum_squares = sequential_sum_wave(sq, H);
  if (lane == 0) inverse_shared = norm_inverse(sum_squares, H, epsilon);
  __syncthreads();
  const float inverse = inverse_shared;
  float norm_sq = 0.0f;
  for (uint32_t c = lane; c < H; c += kWave) {
    const float w = stage_w ? ws[c]
                    : kHalfW ? half_to_float(static_cast<const uint16_t*>(weight)[c])
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

// Rows too wide to stage whole in LDS (H > kNormStagedMax): the squares are
// staged kNormChunk features at a time and lane 0 adds them in feature order
// (one running sum across the chunks: the same chain as the staged kernel),
// then y = (x * inverse) * weight with x and the weight read again from
// global memory.
constexpr uint32_t kNormStagedMax = 16384;
constexpr uint32_t kNormChunk = 4096;

template <bool kHalfIn, bool kHalfW, bool kHalfOut>
__global__ __launch_bounds__(kWave) void rms_norm_wide_kernel(
    const void* __restrict__ input, const void* __restrict__ weight,
    void* output, float* __restrict__ row_norm, uint32_t H, float epsilon) {
  __shared__ float sq[kNormChunk];
  __shared__ float inverse_shared;
  const uint64_t r = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  auto x_at = [&](uint64_t c) -> float {
    return kHalfIn ? half_to_float(static_cast<const uint16_t*>(input)[r * H + c])
                   : static_cast<const float*>(input)[r * H + c];
  };
  auto w_at = [&](uint64_t c) -> float {
    return kHalfW ? half_to_float(static_cast<const uint16_t*>(weight)[c])
                  : static_cast<const float*>(weight)[c];
  };
  float sum = 0.0f;  // lane 0's chain
  for (uint32_t base = 0; base < H; base += kNormChunk) {
    const uint32_t n = H - base < kNormChunk ? H - base : kNormChunk;
    for (uint32_t c = lane; c < n; c += kWave) {
      const float v = x_at(base + c);
      sq[c] = v * v;
    }
    __syncthreads();
    if (lane == 0) {
      for (uint32_t c = 0; c < n; ++c) sum = sum + sq[c];
    }
    __syncthreads();
  }
  if (lane == 0) inverse_shared = norm_inverse(sum, H, epsilon);
  __syncthreads();
  const float inverse = inverse_shared;
  float norm_sq = 0.0f;
  for (uint32_t c = lane; c < H; c += kWave) {
    const float y = (x_at(c) * inverse) * w_at(c);
    if constexpr (kHalfOut) {
      static_cast<uint16_t*>(output)[r * H + c] = float_to_half_rne(y);
    } else {
      static_cast<float*>(output)[r * H + c] = y;
      norm_sq = __builtin_fmaf(y, y, norm_sq);
    }
  }
  if (row_norm != nullptr) {
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) norm_sq += __shfl_xor(norm_sq, m);
    if (lane == 0) row_norm[r] = __fsqrt_rn(norm_sq) * (1.0f + 0x1p-7f);
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
  const uint32_t* ids;
  uint32_t count;
  int status;  // 0 ok, 1 invalid row
};

// Fixed-width candidate table of the reference restricted head
// (greedy.cu:145-151): count 0 or above the maximum makes the row invalid.
__device__ RowList resolve_row(const HeadArgs& a, uint32_t r) {
  RowList l{nullptr, 0u, 0};
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
template <typename Y>
__device__ void fast_scores_generic(const HeadArgs& a, Y ys, HeadShared& sh, uint32_t n) {
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

template <int kH, int kG, typename Y>
__device__ void fast_scores(const HeadArgs& a, Y ys, HeadShared& sh, uint32_t n) {
  if constexpr (kH > 0) {
    fast_scores_vec<kH, kG, 2>(a, ys, sh, n);
  } else {
    fast_scores_generic(a, ys, sh, n);
  }
}

// Summarises one block of n candidates (scores in sh.sc / sh.bd, ids in
// sh.tk, list positions pos0 + c) into sh.rec.  All threads must call.
template <typename Y>
__device__ void summarize_block(const HeadArgs& a, Y ys, HeadShared& sh, uint32_t n,
                                uint32_t pos0, bool invalid) {
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

// Merges n records of one row (in sh.recs) into one: invalid when any is;
// otherwise the exact best (reference-order score) of the records whose
// window reaches the best lower bound L (fast records rescored), or "all
// NaN" when none has a finite score; the lowest id of all of them rides
// along.  Merging in stages gives the same record as merging all at once:
// L never exceeds the row's best exact score, so no stage drops the winner.
// All threads must call; every thread gets the record.
template <typename Y>
__device__ __forceinline__ Record merge_records(const HeadArgs& a, Y ys, HeadShared& sh, uint32_t n) {
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
  const float nan = __builtin_nanf("");
  if (invalid) return Record{nan, nan, nan, kInvalidToken, 0u, kRecInvalid, mt, mp};
  Best best = best_identity();
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
  best = block_best(sh, best);
  if (best.token == kInvalidToken) return Record{nan, nan, nan, kInvalidToken, 0u, kRecAllNan, mt, mp};
  return Record{best.score, best.score, best.score, best.token, best.pos, kRecExact, mt, mp};
}

// Merges the row's records (sh.recs[0, n)) and writes its outputs.
template <typename Y>
__device__ __forceinline__ void finalize_row(const HeadArgs& a, uint32_t r, Y ys, HeadShared& sh, uint32_t n) {
  const Record m = merge_records(a, ys, sh, n);
  if (threadIdx.x == 0) {
    uint32_t token = kInvalidToken;
    float score = __builtin_nanf("");
    if (m.kind & kRecExact) {
      token = m.token;
      score = m.value;
    } else if (m.kind & kRecAllNan) {
      // every score NaN: the lowest id (greedy.cu:205-207)
      token = m.min_token;
      score = canonical_dot_order(a.order, ys, a.emb + static_cast<uint64_t>(m.min_token) * a.H, a.H);
    }
    a.out_token[r] = token;
    if (a.out_score != nullptr) a.out_score[r] = score;
  }
}

// Loads the ids of candidates [begin, begin + n) into sh.tk; returns whether
// any id is outside the vocabulary (the reference marks the row invalid).
__device__ bool load_block_ids(const HeadArgs& a, const RowList& rl,
                               HeadShared& sh, uint32_t begin, uint32_t n) {
  uint32_t bad = 0u;
  for (uint32_t c = threadIdx.x; c < n; c += kThreads) {
    const uint32_t t = rl.ids[begin + c];
    bad |= t >= a.V ? 1u : 0u;
    sh.tk[c] = t < a.V ? t : 0u;
  }
  return block_sum(sh, bad) != 0u;
}

// One workgroup per row: the row's candidates in blocks of a.chunk, each
// block summarized into a record in LDS, then merged (finalize_row); when
// the records fill their LDS array, they are merged into its first entry
// and the row goes on (lists of any length).  kGlobalHidden: the hidden row
// is read from global memory in place of an FP32 copy in LDS (rows too wide
// for LDS).
template <int kH, int kG, bool kGlobalHidden>
__global__ __launch_bounds__(kThreads) void head_kernel(HeadArgs a) {
  extern __shared__ __align__(16) float ys_lds[];
  __shared__ HeadShared sh;
  const uint32_t r = blockIdx.x;
  const RowList rl = resolve_row(a, r);
  if (rl.status == 1) {
    if (threadIdx.x == 0) {
      a.out_token[r] = kInvalidToken;
      if (a.out_score != nullptr) a.out_score[r] = __builtin_nanf("");
    }
    return;
  }
  auto body = [&](auto ys) {
    const uint32_t nblocks = (rl.count + a.chunk - 1) / a.chunk;
    uint32_t nrec = 0;
    for (uint32_t blk = 0; blk < nblocks; ++blk) {
      const uint32_t begin = blk * a.chunk;
      const uint32_t n = rl.count - begin < a.chunk ? rl.count - begin : a.chunk;
      const bool invalid = load_block_ids(a, rl, sh, begin, n);
      if (!invalid) fast_scores<kH, kG>(a, ys, sh, n);
      __syncthreads();
      summarize_block(a, ys, sh, n, begin, invalid);
      if (threadIdx.x == 0) sh.recs[nrec] = sh.rec;
      __syncthreads();
      ++nrec;
      if (nrec == kHeadMaxRecords && blk + 1 < nblocks) {
        const Record m = merge_records(a, ys, sh, nrec);
        __syncthreads();
        if (threadIdx.x == 0) sh.recs[0] = m;
        __syncthreads();
        nrec = 1;
      }
    }
    finalize_row(a, r, ys, sh, nrec);
  };
  if constexpr (kGlobalHidden) {
    body(HalfRow{a.hidden16 + static_cast<uint64_t>(r) * a.H});
  } else {
    for (uint32_t f = threadIdx.x; f < a.H; f += kThreads) {
      ys_lds[f] = half_to_float(a.hidden16[static_cast<uint64_t>(r) * a.H + f]);
    }
    __syncthreads();
    body(static_cast<const float*>(ys_lds));
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

// Read floor: every 16 bytes of [p, p + 16 n16) read once, kReadBatch
// loads per thread issued before any is used, each workgroup on one
// contiguous chunk; the XOR of the words goes to *sink only if it equals a
// value that never occurs in practice (the loads must not be optimized away).
constexpr uint32_t kReadBatch = 8;
__global__ __launch_bounds__(kThreads) void read_floor_kernel(const uint4* p, uint64_t n16,
                                                              uint32_t* sink) {
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kReadBatch * kThreads + threadIdx.x;
  uint4 v[kReadBatch];
#pragma unroll
  for (uint32_t u = 0; u < kReadBatch; ++u) {
    const uint64_t q = base + u * kThreads;
    v[u] = q < n16 ? p[q] : uint4{0u, 0u, 0u, 0u};
  }
  uint32_t x = 0u;
#pragma unroll
  for (uint32_t u = 0; u < kReadBatch; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (x == 0x9E3779B9u && threadIdx.x == 0) *sink = x;
}

} // namespace

hipError_t launch_read_floor(const void* address, uint64_t bytes, uint32_t* sink,
                             hipStream_t stream) {
  const uint64_t n16 = bytes / 16;
  if (n16 == 0) return hipSuccess;
  const uint64_t blocks = (n16 + kReadBatch * kThreads - 1) / (kReadBatch * kThreads);
  if (blocks > 0xFFFFFFFFull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(read_floor_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                     stream, static_cast<const uint4*>(address), n16, sink);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const void* input, bool half_input, const void* weight,
                           bool half_weight, void* output, bool half_output,
                           float* row_norm, uint32_t rows, uint32_t hidden,
                           float epsilon, hipStream_t stream) {
  const dim3 grid(rows), block(kWave);
  if (hidden > kNormStagedMax) {
    if (row_norm != nullptr && hidden > 65536u) return hipErrorInvalidValue;  // bound's margin
    if (half_input && half_weight && half_output) {
      hipLaunchKernelGGL((rms_norm_wide_kernel<true, true, true>), grid, block, 0, stream,
                         input, weight, output, nullptr, hidden, epsilon);
    } else if (!half_input && !half_weight && !half_output) {
      hipLaunchKernelGGL((rms_norm_wide_kernel<false, false, false>), grid, block, 0, stream,
                         input, weight, output, row_norm, hidden, epsilon);
    } else {
      return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const size_t lds = (hidden <= kNormStagedWeightMax ? 3u : 2u) * static_cast<size_t>(hidden) *
                     sizeof(float);
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

hipError_t launch_head(const HeadArgs& args, hipStream_t stream) {
  const bool aligned = (reinterpret_cast<uintptr_t>(args.emb) & 15u) == 0;
  const size_t lds = static_cast<size_t>(args.H) * sizeof(float);
  if (args.H == 576 && aligned) {
    hipLaunchKernelGGL((head_kernel<576, 8, false>), dim3(args.rows), dim3(kThreads), lds, stream, args);
  } else if (args.H <= kHeadLdsHidden) {
    hipLaunchKernelGGL((head_kernel<0, 64, false>), dim3(args.rows), dim3(kThreads), lds, stream, args);
  } else {
    hipLaunchKernelGGL((head_kernel<0, 64, true>), dim3(args.rows), dim3(kThreads), 0, stream, args);
  }
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
