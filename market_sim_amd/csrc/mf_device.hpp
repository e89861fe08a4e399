// Device-side building blocks shared by the gfx950 kernels.
//
// Exactness scheme used by every scoring kernel:
//   1. a fast pass computes each candidate score g in a parallel order
//      (lane-split FP32 FMA + cross-lane reduction, or MFMA) together with a
//      rigorous bound b >= |g - r|, where r is the score in the reference's
//      sequential order (greedy.cu:171-176 or operators.cpp:584-595);
//   2. only candidates whose interval [g - b, g + b] reaches the best lower
//      bound can be the reference winner; those are rescored in the
//      reference order (canonical_dot) and compared with the reference rule.
// The chosen token and its reported score are therefore the reference's
// bit for bit, while the bulk of the work runs in the fast order.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

// Phase timeline of a kernel (builds with -DMF_PASS_TIMELINE only): lane 0
// of each wave stores the real-time counter (100 MHz) at phase k into
// mf_timeline[(workgroup * 4 + wave) * 32 + k] (an array of the translation
// unit's own); MF_STAMP_VALUE records a value there instead.  Without the
// macro both are nothing.
#ifdef MF_PASS_TIMELINE
#define MF_STAMP(k)                                                                   \
  do {                                                                                \
    if (threadIdx.x % 64u == 0u)                                                      \
      mf_timeline[(blockIdx.x * 4u + threadIdx.x / 64u) * 32u + (k)] =                \
          __builtin_amdgcn_s_memrealtime();                                           \
  } while (0)
#define MF_STAMP_VALUE(k, v)                                                          \
  do {                                                                                \
    if (threadIdx.x % 64u == 0u)                                                      \
      mf_timeline[(blockIdx.x * 4u + threadIdx.x / 64u) * 32u + (k)] = (v);           \
  } while (0)
#else
#define MF_STAMP_VALUE(k, v) \
  do {                       \
  } while (0)
#define MF_STAMP(k) \
  do {              \
  } while (0)
#endif

namespace mf {

constexpr uint32_t kInvalidToken = 0xFFFFFFFFu;
constexpr uint32_t kStateUnrestricted = 0xFFFFFFFEu;
constexpr int kWave = 64;

__device__ __forceinline__ float half_to_float(uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

__device__ __forceinline__ uint16_t float_to_half_rne(float v) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// IEEE round-to-nearest square root and quotient of binary32 values.
//
// The hardware square root is faithful only (within one ulp), so the result
// is corrected exactly: for a positive finite candidate c with neighbours
// lo < c < hi, the midpoints (c + lo) / 2 and (c + hi) / 2 have at most 25
// significant bits, so their squares (and their products with a binary32
// divisor) are exact in binary64.  Comparing x against them decides the
// correctly rounded result; a square root or quotient of binary32 values is
// never exactly a midpoint, so no tie rule is needed.
__device__ __forceinline__ float next_up(float c) {
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, c) + 1u);
}
__device__ __forceinline__ float next_down(float c) {
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, c) - 1u);
}

__device__ __forceinline__ float sqrt_rn(float x) {
  float c = __builtin_sqrtf(x);
  if (!(x > 0.0f) || !__builtin_isfinite(x)) return c;  // 0, -0, <0, inf, NaN
  const double xd = x;
  for (int it = 0; it < 3; ++it) {
    const float lo = next_down(c);
    const float hi = next_up(c);
    const double mlo = (static_cast<double>(c) + lo) * 0.5;
    const double mhi = (static_cast<double>(c) + hi) * 0.5;
    if (xd < mlo * mlo) {
      c = lo;
    } else if (xd > mhi * mhi) {
      c = hi;
    } else {
      break;
    }
  }
  return c;
}

// a / b for positive finite a, b whose quotient is a positive normal float
// (the RMSNorm uses: sum / H and 1 / sqrt); other inputs take the compiler's
// IEEE division sequence.
__device__ __forceinline__ float div_rn(float a, float b) {
  float q = __fdiv_rn(a, b);
  if (!(a > 0.0f) || !(b > 0.0f) || !__builtin_isfinite(a) || !__builtin_isfinite(b) ||
      !(q >= 0x1p-126f) || !(q < 0x1p127f)) {
    return q;
  }
  const double ad = a;
  const double bd = b;
  for (int it = 0; it < 3; ++it) {
    const float lo = next_down(q);
    const float hi = next_up(q);
    const double mlo = (static_cast<double>(q) + lo) * 0.5;
    const double mhi = (static_cast<double>(q) + hi) * 0.5;
    if (ad < mlo * bd) {
      q = lo;
    } else if (ad > mhi * bd) {
      q = hi;
    } else {
      break;
    }
  }
  return q;
}

// One step of a reference summation order.  The file is compiled with
// -ffp-contract=off, so the MUL_ADD form keeps its two roundings.
template <bool kMulAdd>
__device__ __forceinline__ float order_step(float s, float h, float e) {
  if constexpr (kMulAdd) {
    const float p = h * e;
    return s + p;
  } else {
    return __builtin_fmaf(h, e, s);
  }
}

// A hidden row read as FP32 values from FP16 storage in global memory (for
// rows too wide to stage in LDS); y[f] as for a float pointer.
struct HalfRow {
  const uint16_t* h;
  __device__ __forceinline__ float operator[](uint32_t f) const { return half_to_float(h[f]); }
};

// Score of one embedding row in a reference order, f = 0..H-1 ascending.
// y: FP32 hidden (a float pointer to LDS or global, or a HalfRow); row: FP16
// embedding row (global).  When the row is 16-byte aligned and H % 8 == 0 the
// loads are 16-byte vectors; the arithmetic order is identical either way.
template <bool kMulAdd, typename Y = const float*>
__device__ float canonical_dot(Y y, const uint16_t* row, uint32_t H) {
  float s = 0.0f;
  uint32_t f = 0;
  if ((reinterpret_cast<uintptr_t>(row) & 15u) == 0 && (H & 7u) == 0) {
    const uint4* v = reinterpret_cast<const uint4*>(row);
#pragma unroll 4
    for (uint32_t i = 0; i < H / 8; ++i) {
      const uint4 q = v[i];
      const uint16_t* h = reinterpret_cast<const uint16_t*>(&q);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        s = order_step<kMulAdd>(s, y[i * 8 + k], half_to_float(h[k]));
      }
    }
    f = H;
  }
  for (; f < H; ++f) {
    s = order_step<kMulAdd>(s, y[f], half_to_float(row[f]));
  }
  return s;
}

template <typename Y = const float*>
__device__ __forceinline__ float canonical_dot_order(int order, Y y, const uint16_t* row,
                                                     uint32_t H) {
  return order == 1 ? canonical_dot<true, Y>(y, row, H)
                    : canonical_dot<false, Y>(y, row, H);
}

// The reference selection order (greedy.cu:96-100): higher score wins, equal
// scores go to the lower id, NaN never wins.  The identity element is
// (-inf, kInvalidToken); a NaN candidate is mapped to the identity before any
// reduction, so partial results are never NaN and the combine is a total
// order (associative and commutative).
struct Best {
  float score;
  uint32_t token;
  uint32_t pos;
};

__device__ __forceinline__ Best best_identity() {
  return Best{-__builtin_huge_valf(), kInvalidToken, 0u};
}

__device__ __forceinline__ bool better(float s1, uint32_t t1, float s2,
                                       uint32_t t2) {
  return s1 > s2 || (s1 == s2 && t1 < t2);
}

__device__ __forceinline__ Best best_of(Best a, Best b) {
  return better(b.score, b.token, a.score, a.token) ? b : a;
}

__device__ __forceinline__ Best best_leaf(float score, uint32_t token,
                                          uint32_t pos) {
  return score != score ? best_identity() : Best{score, token, pos};
}

// Cross-lane reductions without the LDS pipe (__shfl_xor compiles to
// ds_bpermute, an LDS round trip per step).  Within a DPP row (lanes 16 r ..
// 16 r + 15) rotations by 8, 4, 2 and 1 (row_ror) leave every lane of the
// row with the row's result; the four row results are then read with
// v_readlane.  The whole wave must be active, as for the shuffles.
template <int kN>
__device__ __forceinline__ uint32_t row_ror(uint32_t v, uint32_t identity) {
  static_assert(kN > 0 && kN < 16, "row_ror:1..15");
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      static_cast<int>(identity), static_cast<int>(v), 0x120 + kN, 0xF, 0xF, false));
}
__device__ __forceinline__ float as_float(uint32_t v) { return __builtin_bit_cast(float, v); }
__device__ __forceinline__ uint32_t as_u32(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ uint32_t lane_value(uint32_t v, int lane) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

__device__ __forceinline__ float row16_max(float v) {
  v = __builtin_fmaxf(v, as_float(row_ror<8>(as_u32(v), as_u32(v))));
  v = __builtin_fmaxf(v, as_float(row_ror<4>(as_u32(v), as_u32(v))));
  v = __builtin_fmaxf(v, as_float(row_ror<2>(as_u32(v), as_u32(v))));
  v = __builtin_fmaxf(v, as_float(row_ror<1>(as_u32(v), as_u32(v))));
  return v;
}
__device__ __forceinline__ uint32_t row16_and(uint32_t v) {
  v &= row_ror<8>(v, v);
  v &= row_ror<4>(v, v);
  v &= row_ror<2>(v, v);
  v &= row_ror<1>(v, v);
  return v;
}
__device__ __forceinline__ uint32_t row16_min(uint32_t v) {
  v = __builtin_elementwise_min(v, row_ror<8>(v, v));
  v = __builtin_elementwise_min(v, row_ror<4>(v, v));
  v = __builtin_elementwise_min(v, row_ror<2>(v, v));
  v = __builtin_elementwise_min(v, row_ror<1>(v, v));
  return v;
}
__device__ __forceinline__ uint32_t row16_sum(uint32_t v) {
  v += row_ror<8>(v, 0u);
  v += row_ror<4>(v, 0u);
  v += row_ror<2>(v, 0u);
  v += row_ror<1>(v, 0u);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  const uint32_t r = as_u32(row16_max(v));
  return __builtin_fmaxf(__builtin_fmaxf(as_float(lane_value(r, 0)), as_float(lane_value(r, 16))),
                         __builtin_fmaxf(as_float(lane_value(r, 32)), as_float(lane_value(r, 48))));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  const uint32_t r = row16_min(v);
  return __builtin_elementwise_min(
      __builtin_elementwise_min(lane_value(r, 0), lane_value(r, 16)),
      __builtin_elementwise_min(lane_value(r, 32), lane_value(r, 48)));
}

// A sum over the wave in an unspecified order (for bounds, not reference
// arithmetic).
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += as_float(row_ror<8>(as_u32(v), 0u));
  v += as_float(row_ror<4>(as_u32(v), 0u));
  v += as_float(row_ror<2>(as_u32(v), 0u));
  v += as_float(row_ror<1>(as_u32(v), 0u));
  const uint32_t r = as_u32(v);
  return (as_float(lane_value(r, 0)) + as_float(lane_value(r, 16))) +
         (as_float(lane_value(r, 32)) + as_float(lane_value(r, 48)));
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  const uint32_t r = row16_sum(v);
  return lane_value(r, 0) + lane_value(r, 16) + lane_value(r, 32) + lane_value(r, 48);
}

// The lowest token and, among its lanes, the lowest position (the first
// occurrence in list order: the all-NaN fallback rule).
__device__ __forceinline__ void wave_min_token(uint32_t& token, uint32_t& pos) {
  const uint32_t t = wave_min_u32(token);
  pos = wave_min_u32(token == t ? pos : 0xFFFFFFFFu);
  token = t;
}

__device__ __forceinline__ Best wave_best(Best b) {
  // within rows: each step takes the three fields from the same lane
#define MF_BEST_STEP(n)                                                   \
  {                                                                       \
    Best o;                                                               \
    o.score = as_float(row_ror<n>(as_u32(b.score), as_u32(b.score)));     \
    o.token = row_ror<n>(b.token, b.token);                               \
    o.pos = row_ror<n>(b.pos, b.pos);                                     \
    b = best_of(b, o);                                                    \
  }
  MF_BEST_STEP(8)
  MF_BEST_STEP(4)
  MF_BEST_STEP(2)
  MF_BEST_STEP(1)
#undef MF_BEST_STEP
  Best r{as_float(lane_value(as_u32(b.score), 0)), lane_value(b.token, 0), lane_value(b.pos, 0)};
#pragma unroll
  for (int row = 1; row < 4; ++row) {
    const Best o{as_float(lane_value(as_u32(b.score), 16 * row)), lane_value(b.token, 16 * row),
                 lane_value(b.pos, 16 * row)};
    r = best_of(r, o);
  }
  return r;
}

// Summary of one block of candidates, produced by one workgroup pass and
// merged per row (in LDS when one workgroup owns the row, otherwise through
// global memory by the last workgroup to finish the row).
enum : uint32_t {
  kRecFast = 1u,    // one window member: fast score value, interval [lower, upper]
  kRecExact = 2u,   // best reference-order score of the block: value
  kRecAllNan = 4u,  // every reference-order score was NaN
  kRecInvalid = 8u, // an id >= vocabulary was seen: the whole row is invalid
};

struct alignas(16) Record {
  float lower;
  float upper;
  float value;
  uint32_t token;
  uint32_t pos;
  uint32_t kind;
  uint32_t min_token;
  uint32_t min_pos;
};

// Window summary of one tile of candidates (a chunk of a row's list in the
// gather kernel, or 128 vocabulary ids of an unrestricted row in the MFMA
// kernel), merged per row by the finalize kernel.  best_lower is the tile's
// max over candidates of g - b; the members are the candidates with
// g + b >= best_lower.  kTileRescoreAll: non-finite values or more than
// kTileMembers members -- the finalize kernel rescores the whole tile.
constexpr int kTileMembers = 4;
enum : uint32_t {
  kTileInvalid = 1u,     // an id >= vocabulary: the whole row is invalid
  kTileRescoreAll = 2u,
  // with kTileRescoreAll: every bound finite, only the members overflowed;
  // best_lower is valid and upper_max is the tile's max of g + b, so the
  // finalize rescores the tile only if upper_max reaches the row's best
  // lower bound
  kTileCrowded = 4u,
};

struct alignas(16) TileMember {
  uint32_t token;
  uint32_t pos;
  float lower;
  float upper;
};

struct alignas(16) TileRecord {
  float best_lower;
  uint32_t flags;
  uint32_t min_token;
  uint32_t min_pos;
  uint32_t begin;     // list position of the tile's first candidate
  uint32_t count;     // candidates in the tile
  uint32_t n_members;
  float upper_max;    // max of g + b over the tile (kTileCrowded)
  TileMember m[kTileMembers];
};
// the header is written and read as two 16-byte words
static_assert(offsetof(TileRecord, best_lower) == 0 && offsetof(TileRecord, min_pos) == 12 &&
                  offsetof(TileRecord, begin) == 16 && offsetof(TileRecord, upper_max) == 28,
              "tile record header layout");

// Copies n 16-byte pieces from global memory to LDS with `lanes` threads
// (this one is `tid`), kBatch loads per thread in flight before their stores:
// a loop that stores each load before issuing the next pays a memory round
// trip per iteration.
template <uint32_t kBatch>
__device__ __forceinline__ void copy16_to_lds(uint4* dst, const uint4* src, uint32_t n,
                                              uint32_t tid, uint32_t lanes) {
  for (uint32_t base = tid; base < n; base += lanes * kBatch) {
    uint4 v[kBatch];
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t q = base + u * lanes;
      v[u] = q < n ? src[q] : uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t q = base + u * lanes;
      if (q < n) dst[q] = v[u];
    }
  }
}

// One 1 KiB burst from global memory straight into LDS (global_load_lds,
// 16 bytes per lane): lane l reads src_lane (its own 16 bytes) and the data
// lands at dst_wave + 16 l, without passing through registers.  The wave
// must wait for its vector memory count before the data is read, and a
// barrier must follow before other waves read it.
__device__ __forceinline__ void burst_to_lds(const void* src_lane, void* dst_wave) {
  __builtin_amdgcn_global_load_lds(
      (__attribute__((address_space(1))) void*)(const_cast<void*>(src_lane)),
      (__attribute__((address_space(3))) void*)(dst_wave), 16, 0, 0);
}
// Every vector memory operation of this wave has completed (loads landed,
// LDS bursts written).
__device__ __forceinline__ void wait_vector_memory() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The value of lane l - 1 in lane l (DPP wavefront shift right by one;
// lane 0 keeps its own).
__device__ __forceinline__ float lane_shift_right(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x138,
                                                    0xF, 0xF, false));
}

// LDS writes of this wave are visible to every lane of the wave afterwards.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-row metadata written by the decode-tail norm kernel.
// kRowDense (with kRowRestricted): the row's ascending list is scored by the
// dense head (mf_dense.hip), not by the gather; set by the norm launch.
enum : uint32_t { kRowRestricted = 1u, kRowUnrestricted = 2u, kRowInvalid = 4u, kRowDense = 8u };
struct alignas(16) RowMeta {
  uint32_t list_begin;
  uint32_t count;
  uint32_t state;
  uint32_t kind;
};

__device__ __forceinline__ uint32_t atomic_arrive(uint32_t* counter) {
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL,
                                __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void acquire_agent() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

__device__ __forceinline__ void release_agent() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}

} // namespace mf
