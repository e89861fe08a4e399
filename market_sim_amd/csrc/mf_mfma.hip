// gfx950 MFMA kernels: the dense full-vocabulary projection Y * E^T.
//
// Used for (1) the fallback head of unrestricted rows (windowed-argmax
// epilogue writing tile records; no logits written), (2) the
// full-output-projection comparator (FP32 scores), and (3) linear_f16 (FP16
// logits, the reference's cublasGemmEx call).
//
// Tiling: a 256-thread workgroup owns 32 A rows (hidden vectors) x 128
// tokens; each wave computes one 32x32 block with v_mfma_f32_32x32x16_f16.
// FP32 hidden values enter as the FP16 pair hi = rne(y), lo = rne(y - hi)
// (two MFMAs per step), so the fast score is accurate to ~2^-22 relative
// before the reference-order rescore.
//
// K permutation: a dot product does not depend on which features the
// hardware pairs in one step, only on A and B using the same pairing.  Lane
// group g (lanes 32g..32g+31) supplies at step s the features g*H/2 + 8s..+7,
// so each lane streams one contiguous half row of E.  A chunk of kChunk steps
// has all its B fragments loaded into registers before its MFMAs.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTileTokens = 128;
constexpr int kMTile = 32;
constexpr int kMaxChunk = 18;

struct ProjShared {
  union {
    half8_t a[2][2][kMaxChunk][kMTile];  // [hi|lo][group][step][row] 36,864 B
    struct {
      float g[kMTile][kTileTokens];
      float b[kMTile][kTileTokens];
    } epi;                                // 32,768 B
  };
};

enum class ASrc { kF32Split, kF16Pair, kF16 };

struct AView {
  const float* y;           // kF32Split
  const uint16_t* hi;       // kF16Pair, kF16
  const uint16_t* lo;       // kF16Pair
  const uint32_t* row_index;
  uint32_t m;
  uint32_t rows;
  uint32_t H;
};

__device__ __forceinline__ half8_t zero_half8() {
  half8_t z;
#pragma unroll
  for (int k = 0; k < 8; ++k) z[k] = static_cast<_Float16>(0.0f);
  return z;
}

template <ASrc kA, int kChunk>
__device__ void stage_a(const AView& A, uint32_t m0, uint32_t s0, ProjShared& sh) {
  constexpr uint32_t kItems = 2u * kChunk * kMTile;
  const uint32_t half_h = A.H / 2;
  for (uint32_t q = threadIdx.x; q < kItems; q += kThreads) {
    const uint32_t i = q % kMTile;
    const uint32_t rest = q / kMTile;
    const uint32_t s = rest % kChunk;
    const uint32_t g = rest / kChunk;
    const uint32_t f0 = g * half_h + 8u * (s0 + s);
    const uint32_t row = m0 + i < A.m ? (A.row_index != nullptr ? A.row_index[m0 + i] : m0 + i)
                                      : 0xFFFFFFFFu;
    half8_t hi = zero_half8();
    half8_t lo = zero_half8();
    if (row < A.rows) {
      const uint64_t o = static_cast<uint64_t>(row) * A.H + f0;
      if constexpr (kA == ASrc::kF32Split) {
        const float4* src = reinterpret_cast<const float4*>(A.y + o);
        const float4 v0 = src[0];
        const float4 v1 = src[1];
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const _Float16 h = static_cast<_Float16>(v[k]);
          hi[k] = h;
          lo[k] = static_cast<_Float16>(v[k] - static_cast<float>(h));
        }
      } else {
        hi = *reinterpret_cast<const half8_t*>(A.hi + o);
        if constexpr (kA == ASrc::kF16Pair) lo = *reinterpret_cast<const half8_t*>(A.lo + o);
      }
    }
    sh.a[0][g][s][i] = hi;
    sh.a[1][g][s][i] = lo;
  }
}

// One 32x32 block per wave; returns the accumulator and the lane's sum of
// squares of its B values (the token norm, combined across lane groups).
template <ASrc kA, int kChunk>
__device__ floatx16 project_block(const AView& A, const uint16_t* emb, uint32_t V,
                                  uint32_t m0, uint32_t token, ProjShared& sh,
                                  float& tok_sq) {
  const int lane = threadIdx.x % 64;
  const int g = lane / 32;
  const int i = lane % 32;
  const bool tok_ok = token < V;
  const uint32_t H = A.H;
  const uint16_t* brow = emb + static_cast<uint64_t>(tok_ok ? token : 0u) * H +
                         static_cast<uint64_t>(g) * (H / 2);
  floatx16 acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
  tok_sq = 0.0f;
  const uint32_t steps = H / 16;
  for (uint32_t s0 = 0; s0 < steps; s0 += kChunk) {
    half8_t b[kChunk];
#pragma unroll
    for (int s = 0; s < kChunk; ++s) {
      b[s] = tok_ok ? *reinterpret_cast<const half8_t*>(brow + 8u * (s0 + s)) : zero_half8();
    }
    __syncthreads();
    stage_a<kA, kChunk>(A, m0, s0, sh);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kChunk; ++s) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float e = static_cast<float>(b[s][k]);
        tok_sq = __builtin_fmaf(e, e, tok_sq);
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh.a[0][g][s][i], b[s], acc, 0, 0, 0);
      if constexpr (kA != ASrc::kF16) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh.a[1][g][s][i], b[s], acc, 0, 0, 0);
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

template <ASrc kA, int kChunk>
__global__ __launch_bounds__(kThreads) void projection_kernel(ProjArgs p) {
  __shared__ ProjShared sh;
  const uint32_t m0 = blockIdx.y * kMTile;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const uint32_t token = blockIdx.x * kTileTokens + wave * 32 + (lane % 32);
  const AView A{p.y, p.a16, nullptr, p.row_index, p.m, p.rows, p.H};
  float tok_sq;
  const floatx16 acc = project_block<kA, kChunk>(A, p.emb, p.V, m0, token, sh, tok_sq);
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

// Reductions over the 8 consecutive lanes that share one row.
__device__ __forceinline__ float group8_max(float v) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, m, 8));
  return v;
}
__device__ __forceinline__ uint32_t group8_and(uint32_t v) {
#pragma unroll
  for (int m = 4; m > 0; m >>= 1) v &= __shfl_xor(v, m, 8);
  return v;
}

template <int kChunk>
__global__ __launch_bounds__(kThreads) void fallback_kernel(FallbackArgs f) {
  __shared__ ProjShared sh;
  const uint32_t tile = blockIdx.x;
  const uint32_t m0 = blockIdx.y * kMTile;
  const uint32_t tiles = gridDim.x;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const uint32_t token = tile * kTileTokens + wave * 32 + (lane % 32);
  const AView A{nullptr, f.y_hi, f.y_lo, f.row_index, f.m, f.rows, f.H};
  float tok_sq;
  const floatx16 acc = project_block<ASrc::kF16Pair, kChunk>(A, f.emb, f.V, m0, token, sh, tok_sq);

  if (tile == 0 && threadIdx.x < kMTile && m0 + threadIdx.x < f.m) {
    const uint32_t row = f.row_index[m0 + threadIdx.x];
    if (row < f.rows) f.fb_map[row] = m0 + threadIdx.x;
  }

  // scores and bounds into LDS (the A staging area is free after the loop)
  const float tok_norm = __fsqrt_rn(tok_sq) * (1.0f + 0x1p-7f);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int i = acc_row(v, lane);
    float yn = 0.0f;
    if (m0 + i < f.m) {
      const uint32_t src = f.row_index[m0 + i];
      if (src < f.rows) yn = f.row_norm[src];
    }
    sh.epi.g[i][wave * 32 + (lane % 32)] = acc[v];
    sh.epi.b[i][wave * 32 + (lane % 32)] =
        __builtin_fmaf(tok_norm, __builtin_fmaf(f.coef, yn, f.coef2), f.slack);
  }
  __syncthreads();

  // per row (8 lanes, 16 tokens each): the tile's window record
  const uint32_t i = threadIdx.x / 8;
  const uint32_t sub = threadIdx.x % 8;
  const uint32_t tok0 = tile * kTileTokens;
  const uint32_t nt = f.V - tok0 < kTileTokens ? f.V - tok0 : kTileTokens;
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
  for (uint32_t c = sub; c < nt; c += 8) cnt += (sh.epi.g[i][c] + sh.epi.b[i][c] >= L) ? 1u : 0u;
  // exclusive prefix of the member counts across the row's 8 lanes
  uint32_t incl = cnt;
#pragma unroll
  for (int d = 1; d < 8; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d, 8);
    if (static_cast<int>(sub) >= d) incl += o;
  }
  const uint32_t total = __shfl(incl, 7, 8);
  const bool row_ok = m0 + i < f.m && f.row_index[m0 + i] < f.rows;
  if (!row_ok) return;
  TileRecord* rec = f.records + static_cast<uint64_t>(m0 + i) * tiles + tile;
  const bool ordinary = fin && total <= static_cast<uint32_t>(kTileMembers);
  if (ordinary) {
    uint32_t rank = incl - cnt;
    for (uint32_t c = sub; c < nt; c += 8) {
      const float g = sh.epi.g[i][c];
      const float b = sh.epi.b[i][c];
      if (g + b >= L) {
        rec->m[rank] = TileMember{tok0 + c, tok0 + c, g - b, g + b};
        ++rank;
      }
    }
  }
  if (sub == 0) {
    rec->best_lower = L;
    rec->flags = ordinary ? 0u : kTileRescoreAll;
    rec->min_token = tok0;
    rec->min_pos = tok0;
    rec->begin = tok0;
    rec->count = nt;
    rec->n_members = ordinary ? total : 0u;
  }
}

// Largest supported chunk that divides the step count.
template <typename F>
hipError_t with_chunk(uint32_t steps, F&& launch) {
  if (steps % 18 == 0) return launch(std::integral_constant<int, 18>{});
  if (steps % 16 == 0) return launch(std::integral_constant<int, 16>{});
  if (steps % 8 == 0) return launch(std::integral_constant<int, 8>{});
  if (steps % 4 == 0) return launch(std::integral_constant<int, 4>{});
  return launch(std::integral_constant<int, 1>{});
}

} // namespace

uint32_t fallback_tiles(uint32_t vocab) {
  return (vocab + kTileTokens - 1) / kTileTokens;
}

hipError_t launch_projection(const ProjArgs& args, hipStream_t stream) {
  const dim3 grid(fallback_tiles(args.V), (args.m + kMTile - 1) / kMTile);
  return with_chunk(args.H / 16, [&](auto chunk) {
    constexpr int C = decltype(chunk)::value;
    if (args.a16 != nullptr) {
      hipLaunchKernelGGL((projection_kernel<ASrc::kF16, C>), grid, dim3(kThreads), 0, stream, args);
    } else {
      hipLaunchKernelGGL((projection_kernel<ASrc::kF32Split, C>), grid, dim3(kThreads), 0, stream,
                         args);
    }
    return hipGetLastError();
  });
}

hipError_t launch_fallback(const FallbackArgs& args, hipStream_t stream) {
  if (args.m == 0) return hipSuccess;
  const dim3 grid(fallback_tiles(args.V), (args.m + kMTile - 1) / kMTile);
  return with_chunk(args.H / 16, [&](auto chunk) {
    constexpr int C = decltype(chunk)::value;
    hipLaunchKernelGGL((fallback_kernel<C>), grid, dim3(kThreads), 0, stream, args);
    return hipGetLastError();
  });
}

} // namespace mf
