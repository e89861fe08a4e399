// The full output projection on gfx950 MFMA: C[m, V] = A[m, H] . E[V, H]^T
// with FP16 A and E, FP32 accumulation, FP32 or FP16 (round to nearest
// even) output -- linear_f16 (the reference's cublasGemmEx call,
// src/cuda/linear.cu:92-102) and the full-vocabulary comparator's scores.
//
// Tiling.  A workgroup owns 256 A rows x 192 tokens, so at m <= 256 the 256
// token tiles of a 49152-token table are one workgroup per compute unit and
// E is read once; A (m x H, small) is read once per token tile, from L2.
// Four MFMA waves each compute 128 rows x 96 tokens as 4 x 3 blocks of
// v_mfma_f32_32x32x16_f16 (192 accumulator registers).
//
// K runs in chunks of 32 features.  A chunk's A and E rows (64 bytes each)
// go straight from memory into LDS by global_load_lds copies (16 bytes per
// lane, no registers); four chunk buffers, three chunks in flight.  The
// 16-byte pieces of a row are XOR-swizzled by the row's bits 2-3, so the 32
// rows of one MFMA operand read meet no LDS bank conflict.  The copies are
// issued by four copy waves of their own: a wave issuing copies stalls
// while the address unit is busy, and the MFMA waves would idle with it.
// One barrier per chunk hands chunk c to the MFMA waves: the copy waves
// arrive once chunk c has landed (their vector memory count), the MFMA
// waves once they are done reading chunk c - 1, whose buffer the copy waves
// then refill with chunk c + 3.
//
// Epilogue.  With V a multiple of 8 (and a 16-byte aligned output) the tile
// is staged in LDS and leaves as 16-byte pieces of whole rows, written
// through to memory (scope bits sc0 sc1, non-temporal: the scores are not
// read again by this kernel, and dirty lines left in L2 would be written
// back after the last wave, adding to the kernel's time); otherwise element
// by element from the accumulators.
//
// The comparator also needs ||e_t|| per token for its error bound: the MFMA
// waves of the first row half of M-tile 0 sum the squares of the E fragments
// they read (FP32, any order; the (1 + 2^-7) factor of the bound covers it).
#include <hip/hip_runtime.h>

#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace mf {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kMmaWaves = 4;
constexpr uint32_t kCopyWaves = 4;
constexpr int kThreads = static_cast<int>(64u * (kMmaWaves + kCopyWaves));
constexpr uint32_t kMT = 256;     // A rows per workgroup
constexpr uint32_t kNT = 192;     // tokens per workgroup
constexpr uint32_t kKC = 32;      // features per chunk
constexpr uint32_t kRowBytes = kKC * 2u;          // 64
constexpr uint32_t kABytes = kMT * kRowBytes;     // 16 KiB
constexpr uint32_t kBBytes = kNT * kRowBytes;     // 12 KiB
constexpr uint32_t kChunkBytes = kABytes + kBBytes;
constexpr uint32_t kBuffers = 4;
constexpr uint32_t kCopies = kChunkBytes / 1024u;            // 28
constexpr uint32_t kCopiesPerWave = kCopies / kCopyWaves;    // 7
static_assert(kCopies % kCopyWaves == 0, "every copy wave issues the same copies per chunk");
constexpr uint32_t kGemmLds = kBuffers * kChunkBytes;        // 112 KiB
// epilogue staging: F16 rows of 192 tokens padded to 400 bytes (rows R and
// R + 4, written by one store, land on other banks), F32 rows in two halves
// of 128 rows padded to 800 bytes
constexpr uint32_t kF16Stride = kNT * 2u + 16u;
constexpr uint32_t kF32Stride = kNT * 4u + 32u;
static_assert(kMT * kF16Stride <= kGemmLds && 128u * kF32Stride <= kGemmLds, "staging fits");

// LDS byte offset of the 16-byte piece p (0..3) of row r in a chunk region
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t p) {
  return (r * 4u + (p ^ ((r >> 2) & 3u))) * 16u;
}

// Copy i (0..27) of chunk c into buffer region `buf`: copies 0-15 hold A
// rows 16 i .. 16 i + 15, copies 16-27 E rows 16 (i - 16) ..; lane l takes
// row 16 i + l / 4 and LDS piece l % 4 (source piece (l % 4) ^ swizzle).
// Rows past m or V re-read the last one (their results are not stored).
__device__ __forceinline__ void chunk_copy(const ProjArgs& a, uint32_t m0, uint32_t n0, uint32_t c,
                                           uint32_t i, unsigned char* buf) {
  const uint32_t lane = threadIdx.x % 64u;
  const uint32_t pp = lane % 4u;
  const uint32_t k0 = c * kKC;
  if (i < kABytes / 1024u) {
    const uint32_t r = 16u * i + lane / 4u;
    const uint32_t p = pp ^ ((r >> 2) & 3u);
    const uint32_t row = m0 + r < a.m ? m0 + r : a.m - 1u;
    burst_to_lds(a.a16 + static_cast<uint64_t>(row) * a.H + k0 + p * 8u, buf + i * 1024u);
  } else {
    const uint32_t r = 16u * (i - kABytes / 1024u) + lane / 4u;
    const uint32_t p = pp ^ ((r >> 2) & 3u);
    const uint32_t tok = n0 + r < a.V ? n0 + r : a.V - 1u;
    burst_to_lds(a.emb + static_cast<uint64_t>(tok) * a.H + k0 + p * 8u, buf + i * 1024u);
  }
}

// Wait until at most `after` chunks of this copy wave's copies are in flight.
__device__ __forceinline__ void wait_chunks(uint32_t after) {
  static_assert(kCopiesPerWave == 7, "the wait counts below are multiples of 7");
  if (after >= 2u) {
    asm volatile("s_waitcnt vmcnt(14)" ::: "memory");
  } else if (after == 1u) {
    asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// A workgroup barrier without __syncthreads' release fence, which would
// wait for every copy in flight (vector memory count 0) and empty the
// pipeline.  The wave's own LDS operations are complete when it arrives.
__device__ __forceinline__ void chunk_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16 bytes to global memory, written through to memory (see the epilogue).
__device__ __forceinline__ void store_through(void* dst, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1 nt" ::"v"(dst), "v"(v) : "memory");
}

template <bool kF16Out>
__global__ __launch_bounds__(kThreads) void projection_kernel(ProjArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  const uint32_t lane = threadIdx.x % 64u;
  const uint32_t wave = threadIdx.x / 64u;
  const bool copier = wave >= kMmaWaves;
  const uint32_t wm = (wave % kMmaWaves) / 2u;  // MFMA wave's row half
  const uint32_t wn = wave % 2u;                // and token half
  const uint32_t m0 = blockIdx.y * kMT;
  const uint32_t n0 = blockIdx.x * kNT;
  const uint32_t chunks = a.H / kKC;
  const bool norms = a.tok_norm != nullptr && blockIdx.y == 0 && wm == 0u && !copier;

  floatx16 acc[4][3];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    }
  }
  float tok_sq[3] = {0.0f, 0.0f, 0.0f};
  // the MFMA lane's operand rows: A rows 128 wm + 32 i + lane % 32, E rows
  // 96 wn + 32 j + lane % 32; its K half of each 16-feature step is lane / 32
  const uint32_t r32 = lane % 32u;
  const uint32_t kh = lane / 32u;

  if (copier) {
    const uint32_t cw = wave - kMmaWaves;
    auto issue = [&](uint32_t c) {
      unsigned char* buf = lds + (c % kBuffers) * kChunkBytes;
#pragma unroll
      for (uint32_t u = 0; u < kCopiesPerWave; ++u) {
        chunk_copy(a, m0, n0, c, cw + kCopyWaves * u, buf);
      }
    };
    const uint32_t first = chunks < 3u ? chunks : 3u;
    for (uint32_t c = 0; c < first; ++c) issue(c);
    wait_chunks(first - 1u);
    chunk_barrier();  // chunk 0 in LDS
    for (uint32_t c = 0; c < chunks; ++c) {
      // the MFMA waves work on chunk c; chunk c - 1's buffer is free
      if (c + 3u < chunks) issue(c + 3u);
      if (c + 1u < chunks) {
        const uint32_t last = c + 3u < chunks ? c + 3u : chunks - 1u;
        wait_chunks(last - (c + 1u));
      }
      chunk_barrier();  // chunk c + 1 in LDS, chunk c read by every MFMA wave
    }
  } else {
    chunk_barrier();
    for (uint32_t c = 0; c < chunks; ++c) {
      const unsigned char* abuf = lds + (c % kBuffers) * kChunkBytes;
      const unsigned char* bbuf = abuf + kABytes;
      half8_t af[2][4];
      half8_t bf[2][3];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t p = 2u * s + kh;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          af[s][i] = *reinterpret_cast<const half8_t*>(abuf + swz(128u * wm + 32u * i + r32, p));
        }
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          bf[s][j] = *reinterpret_cast<const half8_t*>(bbuf + swz(96u * wn + 32u * j + r32, p));
        }
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int j = 0; j < 3; ++j) {
            acc[i][j] =
                __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s][i], bf[s][j], acc[i][j], 0, 0, 0);
          }
        }
        if (norms) {
#pragma unroll
          for (int j = 0; j < 3; ++j) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const float e = static_cast<float>(bf[s][j][k]);
              tok_sq[j] = __builtin_fmaf(e, e, tok_sq[j]);
            }
          }
        }
      }
      chunk_barrier();
    }
  }

  // token norm bounds (lanes l and l + 32 hold the two K halves of token l)
  if (norms) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const float sq = tok_sq[j] + __shfl_xor(tok_sq[j], 32);
      const uint32_t tok = n0 + 96u * wn + 32u * j + r32;
      if (kh == 0u && tok < a.V) a.tok_norm[tok] = __fsqrt_rn(sq) * (1.0f + 0x1p-7f);
    }
  }
  // D[row][col] of block (i, j): lane l holds rows 8 (v / 4) + 4 (l / 32) +
  // v % 4, column l % 32.  The last chunk barrier freed the LDS.
  const uintptr_t out_addr = kF16Out ? reinterpret_cast<uintptr_t>(a.out_f16)
                                     : reinterpret_cast<uintptr_t>(a.out_f32);
  if (a.V % 8u == 0u && out_addr % 16u == 0u) {
    if constexpr (kF16Out) {
      if (!copier) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const uint32_t r = 128u * wm + 32u * i + 8u * (v / 4) + 4u * kh + (v % 4);
              const uint32_t col = 96u * wn + 32u * j + r32;
              *reinterpret_cast<uint16_t*>(lds + r * kF16Stride + col * 2u) =
                  float_to_half_rne(acc[i][j][v]);
            }
          }
        }
      }
      chunk_barrier();
      constexpr uint32_t kPieces = kNT * 2u / 16u;  // 24 per row
      for (uint32_t q = threadIdx.x; q < kMT * kPieces; q += kThreads) {
        const uint32_t r = q / kPieces, piece = q % kPieces;
        const uint32_t row = m0 + r, tok = n0 + piece * 8u;  // 8 tokens, all < V or none
        if (row < a.m && tok < a.V) {
          store_through(a.out_f16 + static_cast<uint64_t>(row) * a.V + tok,
                        *reinterpret_cast<const u32x4*>(lds + r * kF16Stride + piece * 16u));
        }
      }
    } else {
      constexpr uint32_t kPieces = kNT * 4u / 16u;  // 48 per row
      for (uint32_t h = 0; h < 2u; ++h) {
        if (!copier && wm == h) {
#pragma unroll
          for (int j = 0; j < 3; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const uint32_t r = 32u * i + 8u * (v / 4) + 4u * kh + (v % 4);
                const uint32_t col = 96u * wn + 32u * j + r32;
                *reinterpret_cast<float*>(lds + r * kF32Stride + col * 4u) = acc[i][j][v];
              }
            }
          }
        }
        chunk_barrier();
        for (uint32_t q = threadIdx.x; q < 128u * kPieces; q += kThreads) {
          const uint32_t r = q / kPieces, piece = q % kPieces;
          const uint32_t row = m0 + 128u * h + r, tok = n0 + piece * 4u;
          if (row < a.m && tok < a.V) {
            store_through(a.out_f32 + static_cast<uint64_t>(row) * a.V + tok,
                          *reinterpret_cast<const u32x4*>(lds + r * kF32Stride + piece * 16u));
          }
        }
        chunk_barrier();  // the staging area is free for the second half
      }
    }
    return;
  }
  if (copier) return;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const uint32_t tok = n0 + 96u * wn + 32u * j + r32;
    if (tok >= a.V) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t row = m0 + 128u * wm + 32u * i + 8u * (v / 4) + 4u * kh + (v % 4);
        if (row < a.m) {
          const uint64_t o = static_cast<uint64_t>(row) * a.V + tok;
          if constexpr (kF16Out) {
            a.out_f16[o] = float_to_half_rne(acc[i][j][v]);
          } else {
            a.out_f32[o] = acc[i][j][v];
          }
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_projection(const ProjArgs& args, hipStream_t stream) {
  if (args.H % kKC != 0 || args.H == 0 || args.m == 0 || args.V == 0 || args.a16 == nullptr ||
      args.emb == nullptr || (args.out_f32 == nullptr) == (args.out_f16 == nullptr) ||
      reinterpret_cast<uintptr_t>(args.a16) % 16u != 0 ||
      reinterpret_cast<uintptr_t>(args.emb) % 16u != 0) {
    return hipErrorInvalidValue;
  }
  const dim3 grid((args.V + kNT - 1) / kNT, (args.m + kMT - 1) / kMT);
  if (args.out_f16 != nullptr) {
    hipLaunchKernelGGL((projection_kernel<true>), grid, dim3(kThreads), kGemmLds, stream, args);
  } else {
    hipLaunchKernelGGL((projection_kernel<false>), grid, dim3(kThreads), kGemmLds, stream, args);
  }
  return hipGetLastError();
}

}  // namespace mf
