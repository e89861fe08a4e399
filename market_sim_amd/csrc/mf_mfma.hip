// gfx950 MFMA kernels: the dense full-vocabulary projection Y * E^T.
//
// Used for (1) the fallback head of unrestricted rows (windowed argmax
// epilogue + exact rescore, no logits written), (2) the full-output-projection
// comparator (FP32 scores), and (3) linear_f16 (FP16 logits).
//
// Tiling: a 256-thread workgroup owns 32 A rows (hidden vectors) x 128 tokens;
// each wave computes one 32x32 block with v_mfma_f32_32x32x16_f16.  FP32
// hidden values enter the MFMA as an exact-ish FP16 pair hi + lo
// (hi = rne(y), lo = rne(y - hi)), two MFMAs per step, so the fast score is
// accurate to ~2^-22 relative before the reference-order rescore.
//
// K permutation: a dot product does not depend on the order in which the
// hardware pairs features, only on A and B using the same pairing.  Lane
// group g (lanes 32g..32g+31) supplies, at step s, features
// g*H/2 + 8s .. +7, so every lane streams one contiguous half row of E.
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTileTokens = 128;
constexpr int kMTile = 32;
constexpr int kChunkSteps = 36; // A staging chunk: 36 steps of 16 features

struct ProjShared {
  union {
    half8_t a[2][2][kChunkSteps][kMTile]; // [hi|lo][group][step][row] 73,728 B
    struct {
      float g[kMTile][kTileTokens];
      float b[kMTile][kTileTokens];
    } epi;                                 // 32,768 B
  };
  Record rec[kMTile];
  uint32_t last;
};

__device__ __forceinline__ half8_t zero_half8() {
  half8_t z;
#pragma unroll
  for (int k = 0; k < 8; ++k) z[k] = static_cast<_Float16>(0.0f);
  return z;
}

// Stages A for steps [s0, s0 + sc) into LDS as hi/lo FP16 pairs (or the FP16
// input as hi with lo = 0).
template <bool kHalfA>
__device__ void stage_a(const ProjArgs& p, uint32_t m0, uint32_t s0, uint32_t sc,
                        ProjShared& sh) {
  const uint32_t items = 2u * sc * kMTile;
  const uint32_t half_h = p.H / 2;
  for (uint32_t q = threadIdx.x; q < items; q += kThreads) {
    const uint32_t i = q % kMTile;
    const uint32_t rest = q / kMTile;
    const uint32_t s = rest % sc;
    const uint32_t g = rest / sc;
    const uint32_t f0 = g * half_h + 8u * (s0 + s);
    half8_t hi = zero_half8();
    half8_t lo = zero_half8();
    const uint32_t row = m0 + i < p.m ? (p.row_index != nullptr ? p.row_index[m0 + i] : m0 + i)
                                      : 0xFFFFFFFFu;
    if (row < p.rows) {
      if constexpr (kHalfA) {
        hi = *reinterpret_cast<const half8_t*>(p.a16 + static_cast<uint64_t>(row) * p.H + f0);
      } else {
        const float4* src = reinterpret_cast<const float4*>(p.y + static_cast<uint64_t>(row) * p.H + f0);
        const float4 v0 = src[0];
        const float4 v1 = src[1];
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const _Float16 h = static_cast<_Float16>(v[k]);
          hi[k] = h;
          lo[k] = static_cast<_Float16>(v[k] - static_cast<float>(h));
        }
      }
    }
    sh.a[0][g][s][i] = hi;
    sh.a[1][g][s][i] = lo;
  }
}

// Main loop: one 32x32 block per wave.  Returns the accumulator and the
// lane's partial sum of squares of its B values (for ||e_t||).
template <bool kSplit, bool kHalfA>
__device__ floatx16 project_block(const ProjArgs& p, uint32_t m0, uint32_t token,
                                  ProjShared& sh, float& tok_sq) {
  const int lane = threadIdx.x % 64;
  const int g = lane / 32;
  const int i = lane % 32;
  const bool tok_ok = token < p.V;
  const uint16_t* brow = p.emb + static_cast<uint64_t>(tok_ok ? token : 0u) * p.H +
                         static_cast<uint64_t>(g) * (p.H / 2);
  floatx16 acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
  tok_sq = 0.0f;
  const uint32_t steps = p.H / 16;
  for (uint32_t s0 = 0; s0 < steps; s0 += kChunkSteps) {
    const uint32_t sc = steps - s0 < kChunkSteps ? steps - s0 : kChunkSteps;
    __syncthreads();
    stage_a<kHalfA>(p, m0, s0, sc, sh);
    __syncthreads();
#pragma unroll 4
    for (uint32_t s = 0; s < sc; ++s) {
      const half8_t b = tok_ok ? *reinterpret_cast<const half8_t*>(brow + 8u * (s0 + s))
                               : zero_half8();
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float e = static_cast<float>(b[k]);
        tok_sq = __builtin_fmaf(e, e, tok_sq);
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh.a[0][g][s][i], b, acc, 0, 0, 0);
      if constexpr (kSplit) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh.a[1][g][s][i], b, acc, 0, 0, 0);
      }
    }
  }
  __syncthreads();
  tok_sq += __shfl_xor(tok_sq, 32);
  return acc;
}

// Accumulator element v of lane l holds D[row][col] with col = l % 32 and
// row = 8 * (v / 4) + 4 * (l / 32) + v % 4 (the 32x32 MFMA output layout).
__device__ __forceinline__ int acc_row(int v, int lane) {
  return 8 * (v / 4) + 4 * (lane / 32) + (v % 4);
}

template <bool kSplit, bool kHalfA>
__global__ __launch_bounds__(kThreads) void projection_kernel(ProjArgs p) {
  __shared__ ProjShared sh;
  const uint32_t m0 = blockIdx.y * kMTile;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const uint32_t token = blockIdx.x * kTileTokens + wave * 32 + (lane % 32);
  float tok_sq;
  const floatx16 acc = project_block<kSplit, kHalfA>(p, m0, token, sh, tok_sq);
  if (token >= p.V) return;
  if (p.tok_norm != nullptr && blockIdx.y == 0 && lane < 32) {
    p.tok_norm[token] = __fsqrt_rn(tok_sq) * (1.0f + 0x1p-7f);
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const uint32_t row = m0 + acc_row(v, lane);
    if (row < p.m) {
      const uint64_t o = static_cast<uint64_t>(row) * p.V + token;
      if (p.out_f32 != nullptr) p.out_f32[o] = acc[v];
      if (p.out_f16 != nullptr) p.out_f16[o] = float_to_half_rne(acc[v]);
    }
  }
}

// Reference-order rescore with y read from global memory (the fallback keeps
// no per-row copy of y in LDS).
__device__ __forceinline__ float rescore(const FallbackArgs& f, uint32_t row,
                                         uint32_t token) {
  return canonical_dot_order(f.order, f.y + static_cast<uint64_t>(row) * f.H,
                             f.emb + static_cast<uint64_t>(token) * f.H, f.H);
}

// Reduction over the 8 consecutive lanes that share one row.
__device__ __forceinline__ float group8_max(float v) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, m, 8));
  return v;
}
__device__ __forceinline__ uint32_t group8_sum(uint32_t v) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) v += __shfl_xor(v, m, 8);
  return v;
}
__device__ __forceinline__ uint32_t group8_and(uint32_t v) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) v &= __shfl_xor(v, m, 8);
  return v;
}
__device__ __forceinline__ Best group8_best(Best b) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) {
    Best o{__shfl_xor(b.score, m, 8), __shfl_xor(b.token, m, 8), __shfl_xor(b.pos, m, 8)};
    b = best_of(b, o);
  }
  return b;
}
__device__ __forceinline__ void group8_min_token(uint32_t& t) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) {
    const uint32_t o = __shfl_xor(t, m, 8);
    t = o < t ? o : t;
  }
}

__global__ __launch_bounds__(kThreads) void fallback_kernel(FallbackArgs f) {
  __shared__ ProjShared sh;
  const uint32_t tile = blockIdx.x;
  const uint32_t mtile = blockIdx.y;
  const uint32_t m0 = mtile * kMTile;
  const uint32_t tiles = gridDim.x;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const uint32_t token = tile * kTileTokens + wave * 32 + (lane % 32);

  ProjArgs p{};
  p.y = f.y;
  p.row_index = f.row_index;
  p.m = f.m;
  p.rows = f.rows;
  p.emb = f.emb;
  p.H = f.H;
  p.V = f.V;
  float tok_sq;
  const floatx16 acc = project_block<true, false>(p, m0, token, sh, tok_sq);

  // scores and bounds of this tile into LDS (the A staging area is free now)
  const float tok_norm = __fsqrt_rn(tok_sq) * (1.0f + 0x1p-7f);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int i = acc_row(v, lane);
    const uint32_t row = m0 + i;
    float yn = 0.0f;
    if (row < f.m) {
      const uint32_t src = f.row_index[row];
      if (src < f.rows) yn = f.row_norm[src];
    }
    sh.epi.g[i][wave * 32 + (lane % 32)] = acc[v];
    sh.epi.b[i][wave * 32 + (lane % 32)] =
        __builtin_fmaf(tok_norm, __builtin_fmaf(f.coef, yn, f.coef2), f.slack);
  }
  __syncthreads();

  // per row: the tile's window, 8 lanes per row, 16 tokens per lane
  const uint32_t i = threadIdx.x / 8;
  const uint32_t sub = threadIdx.x % 8;
  const uint32_t tok0 = tile * kTileTokens;
  const uint32_t nt = f.V - tok0 < kTileTokens ? f.V - tok0 : kTileTokens;
  const bool row_ok = m0 + i < f.m && f.row_index[m0 + i] < f.rows;
  uint32_t fin = 1u;
  float lo = -__builtin_huge_valf();
  for (uint32_t c = sub; c < nt; c += 8) {
    const float g = sh.epi.g[i][c];
    const float b = sh.epi.b[i][c];
    fin &= (__builtin_isfinite(g) && __builtin_isfinite(b) && b < 0x1p100f) ? 1u : 0u;
    lo = __builtin_fmaxf(lo, g - b);
  }
  fin = group8_and(fin);
  const float L = group8_max(lo);
  uint32_t cnt = 0u;
  uint32_t member = 0u;
  for (uint32_t c = sub; c < nt; c += 8) {
    if (sh.epi.g[i][c] + sh.epi.b[i][c] >= L) {
      ++cnt;
      member = c;
    }
  }
  const uint32_t total = group8_sum(cnt);
  Record rec;
  rec.min_token = tok0;
  rec.min_pos = tok0;
  if (fin && total == 1u) {
    // the unique member: the lane that counted it publishes
    uint32_t who = cnt == 1u ? member : 0xFFFFFFFFu;
#pragma unroll
    for (int m = 4; m > 0; m >>= 1) {
      const uint32_t o = __shfl_xor(who, m, 8);
      who = o < who ? o : who;
    }
    const float g = sh.epi.g[i][who];
    const float b = sh.epi.b[i][who];
    rec.lower = g - b;
    rec.upper = g + b;
    rec.value = g;
    rec.token = tok0 + who;
    rec.pos = tok0 + who;
    rec.kind = kRecFast;
  } else {
    Best best = best_identity();
    if (row_ok) {
      const uint32_t row = f.row_index[m0 + i];
      for (uint32_t c = sub; c < nt; c += 8) {
        if (!fin || sh.epi.g[i][c] + sh.epi.b[i][c] >= L) {
          best = best_of(best, best_leaf(rescore(f, row, tok0 + c), tok0 + c, tok0 + c));
        }
      }
    }
    best = group8_best(best);
    if (best.token == kInvalidToken) {
      const float nan = __builtin_nanf("");
      rec.lower = rec.upper = rec.value = nan;
      rec.token = kInvalidToken;
      rec.pos = 0u;
      rec.kind = kRecAllNan;
    } else {
      rec.lower = rec.upper = rec.value = best.score;
      rec.token = best.token;
      rec.pos = best.pos;
      rec.kind = kRecExact;
    }
  }
  if (row_ok && sub == 0) {
    f.records[static_cast<uint64_t>(m0 + i) * tiles + tile] = rec;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t arrived = atomic_arrive(&f.counters[mtile]);
    sh.last = arrived == tiles - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (sh.last == 0u) return;
  acquire_agent();

  // last workgroup of this M-tile: merge every row's tile records
  if (threadIdx.x == 0) f.counters[mtile] = 0u;
  if (!row_ok) return;
  const Record* recs = f.records + static_cast<uint64_t>(m0 + i) * tiles;
  float lg = -__builtin_huge_valf();
  uint32_t mt = kInvalidToken;
  for (uint32_t t = sub; t < tiles; t += 8) {
    const Record q = recs[t];
    if (q.kind & (kRecFast | kRecExact)) lg = __builtin_fmaxf(lg, q.lower);
    mt = q.min_token < mt ? q.min_token : mt;
  }
  lg = group8_max(lg);
  group8_min_token(mt);
  const uint32_t row = f.row_index[m0 + i];
  Best best = best_identity();
  for (uint32_t t = sub; t < tiles; t += 8) {
    const Record q = recs[t];
    if ((q.kind & (kRecFast | kRecExact)) && q.upper >= lg) {
      const float s = (q.kind & kRecExact) ? q.value : rescore(f, row, q.token);
      best = best_of(best, best_leaf(s, q.token, q.pos));
    }
  }
  best = group8_best(best);
  if (sub == 0) {
    uint32_t tok = best.token;
    float score = best.score;
    if (tok == kInvalidToken) {
      tok = mt;
      score = rescore(f, row, mt);
    }
    f.out_token[row] = tok;
    if (f.out_score != nullptr) f.out_score[row] = score;
    if (f.out_next != nullptr) f.out_next[row] = kStateUnrestricted;
  }
}

} // namespace

uint32_t fallback_tiles(uint32_t vocab) {
  return (vocab + kTileTokens - 1) / kTileTokens;
}

hipError_t launch_projection(const ProjArgs& args, hipStream_t stream) {
  const dim3 grid(fallback_tiles(args.V), (args.m + kMTile - 1) / kMTile);
  if (args.a16 != nullptr) {
    hipLaunchKernelGGL((projection_kernel<false, true>), grid, dim3(kThreads), 0, stream, args);
  } else {
    hipLaunchKernelGGL((projection_kernel<true, false>), grid, dim3(kThreads), 0, stream, args);
  }
  return hipGetLastError();
}

hipError_t launch_fallback(const FallbackArgs& args, hipStream_t stream) {
  if (args.m == 0) return hipSuccess;
  const dim3 grid(fallback_tiles(args.V), (args.m + kMTile - 1) / kMTile);
  hipLaunchKernelGGL(fallback_kernel, grid, dim3(kThreads), 0, stream, args);
  return hipGetLastError();
}

} // namespace mf
