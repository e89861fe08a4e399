// The final RMSNorm in the reference's CPU order (src/cpu/operators.cpp:
// 523-535): every square rounded, an unfused sequential sum in column order,
// mean = sum / H, inv = 1 / sqrt(mean + eps) (IEEE division and square root),
// y = (x * inv) * w.  Used by the norm kernel and by the chain waves that run
// inside the gather launch.
#pragma once

#include <hip/hip_runtime.h>

#include "mf_device.hpp"

namespace mf {

// Sum of squares in the reference order: the squares are in sq[] (rounded),
// added in column order by one lane.  Blocks of 16 values alternate between
// two register sets: the LDS reads of block i + 1 are issued before the adds
// of block i (sched_barrier keeps the scheduler from sinking them to their
// use, which would pay an LDS round trip per block).
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
__device__ inline float sequential_sum(const float* sq, uint32_t H) {
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

// sequential_sum by the whole wave (every lane calls; every lane gets the
// sum).  When H is a multiple of 64 of at most 64 segments, lane k holds the
// squares [64 k, 64 k + 64) in registers and the sum runs segment by
// segment, handed one lane up between segments: the same additions in the
// same order, from registers instead of LDS reads.  Otherwise lane 0 runs
// sequential_sum.
__device__ inline float sequential_sum_wave(const float* sq, uint32_t H) {
  constexpr uint32_t kSeg = 64;
  const uint32_t lane = threadIdx.x % kWave;
  if (H % kSeg == 0u && H <= kSeg * kWave) {
    const uint32_t nseg = H / kSeg;
    const uint32_t k = lane < nseg ? lane : 0u;
    const float4* q = reinterpret_cast<const float4*>(sq + k * kSeg);
    float v[kSeg];
#pragma unroll
    for (uint32_t i = 0; i < kSeg / 4; ++i) {
      const float4 t = q[i];
      v[4 * i] = t.x;
      v[4 * i + 1] = t.y;
      v[4 * i + 2] = t.z;
      v[4 * i + 3] = t.w;
    }
    float s = 0.0f;
    for (uint32_t seg = 0; seg < nseg; ++seg) {
      if (lane == seg) {
#pragma unroll
        for (uint32_t i = 0; i < kSeg; ++i) s = s + v[i];
      }
      if (seg + 1 < nseg) s = lane_shift_right(s);
    }
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), nseg - 1u));
  }
  float s = 0.0f;
  if (lane == 0) s = sequential_sum(sq, H);
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(s)));
}

// inv of a row from its sum of squares (operators.cpp:531-533)
__device__ __forceinline__ float norm_inverse(float sum_squares, uint32_t H, float epsilon) {
  const float mean = div_rn(sum_squares, static_cast<float>(H));
  return div_rn(1.0f, sqrt_rn(mean + epsilon));
}

// One wave normalizes row r of x into y and stores inv: xs and sq are the
// wave's own H-float LDS buffers, w the weight already in LDS, inv_slot one
// float of the wave's own.  The caller guarantees H % 4 == 0.
__device__ inline void norm_chain_wave(const float* __restrict__ x, const float* w, float* y,
                                       float* row_inv, uint32_t r, uint32_t H, float epsilon,
                                       float* xs, float* sq, float* inv_slot) {
  const uint32_t lane = threadIdx.x % kWave;
  const float4* x4 = reinterpret_cast<const float4*>(x + static_cast<uint64_t>(r) * H);
  const uint32_t n = H / 4;
  constexpr uint32_t kBatch = 4;
  for (uint32_t base = lane; base < n; base += kWave * kBatch) {
    float4 v[kBatch];
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t q = base + u * kWave;
      v[u] = q < n ? x4[q] : float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t q = base + u * kWave;
      if (q < n) {
        reinterpret_cast<float4*>(xs)[q] = v[u];
        reinterpret_cast<float4*>(sq)[q] =
            float4{v[u].x * v[u].x, v[u].y * v[u].y, v[u].z * v[u].z, v[u].w * v[u].w};
      }
    }
  }
  // this wave's LDS writes are visible to its own lanes
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float sum_squares = sequential_sum_wave(sq, H);
  if (lane == 0) *inv_slot = norm_inverse(sum_squares, H, epsilon);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float inverse = *inv_slot;
  float4* y4 = reinterpret_cast<float4*>(y + static_cast<uint64_t>(r) * H);
  for (uint32_t q = lane; q < n; q += kWave) {
    const float4 v = reinterpret_cast<const float4*>(xs)[q];
    const float4 g = reinterpret_cast<const float4*>(w)[q];
    const float a0 = v.x * inverse, a1 = v.y * inverse, a2 = v.z * inverse, a3 = v.w * inverse;
    y4[q] = float4{a0 * g.x, a1 * g.y, a2 * g.z, a3 * g.w};
  }
  if (lane == 0) row_inv[r] = inverse;
}

}  // namespace mf
