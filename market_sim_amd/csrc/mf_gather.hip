// The restricted gather on the matrix cores (restricted stage of
// mf_decode_tail_f16 when H % 32 == 0).
//
// A wave owns one tile: up to a.tile consecutive candidates of one row's
// list (64; 32 or 16 for packs too small to give every SIMD a tile of 64),
// the granularity of the window records the finalize kernel merges.  It
// scores them 16 at a time with v_mfma_f32_16x16x32_f16:
//
//   scores  A = [z_hi; z_lo; 0 ...] (16 x 32)  x  B = 16 embedding rows
//           -> D[0][t] + D[1][t] = z . e_t with z = x * w (the normalized
//              row up to its positive factor inv) split into the FP16 pair
//              hi = rne(z), lo = rne(z - hi)
//   norms   A = B = the same 16 embedding rows
//           -> the Gram diagonal D[t][t] = ||e_t||^2 (FP16 products are exact
//              in FP32), which bounds the error of both the fast score and
//              the reference-order score (Cauchy-Schwarz)
//
// The operand registers are filled straight from HBM: in the 16x16x32 layout
// lane l holds 8 consecutive features of column l % 16 at k-block l / 16, so
// the four lanes of one token read 64 contiguous bytes per step and the next
// step the rest of the 128-byte line.  No LDS, no barriers after the plan:
// the loads of the next (block, chunk) unit are in flight while the current
// unit's MFMAs run, and waves never wait on one another.
#include <hip/hip_runtime.h>

#include <atomic>

#include "mf_device.hpp"
#include "mf_launch.hpp"
#include "mf_norm.hpp"
#include "mf_plan.hpp"

namespace mf {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr uint32_t kBlock = 16;  // tokens per MFMA block
constexpr uint32_t kStep = 32;   // features per MFMA step

// One unit: KC steps of the B operand (16 table rows) of one block.
template <int KC>
struct Operands {
  half8_t b[KC];
};

// Loads of one unit: straight-line (no predication, no branches) so the
// compiler can count the loads in flight and wait only for the unit about to
// be multiplied.
template <int KC>
__device__ __forceinline__ void load_unit(const uint16_t* brow, uint32_t f0, Operands<KC>& o) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    o.b[s] = *reinterpret_cast<const half8_t*>(brow + f0 + s * kStep);
  }
}

// MFMAs of one unit.  A comes from the wave's LDS stage of the row's FP16
// split: lanes of A row 0 read hi, all others lo; rows 2..15 are masked.
template <int KC>
__device__ __forceinline__ void mma_unit(const Operands<KC>& o, const uint16_t* a_lane,
                                         uint32_t f0, uint32_t amask, floatx4& sc,
                                         floatx4& gram) {
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    uint4 q = *reinterpret_cast<const uint4*>(a_lane + f0 + s * kStep);
    q.x &= amask;
    q.y &= amask;
    q.z &= amask;
    q.w &= amask;
    sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, q), o.b[s], sc, 0,
                                                0, 0);
    gram = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.b[s], o.b[s], gram, 0, 0, 0);
  }
}

// Block j done: lane 16 j + c takes column c's score and squared norm.  In
// the 16x16 output layout lane s holds D[4 (s / 16) + i][s % 16], i < 4: the
// score parts D[0][c], D[1][c] sit in lane c, the diagonal D[c][c] in lane
// c + 16 (c / 4), element c % 4.
__device__ __forceinline__ void finish_block(uint32_t j, uint32_t lane, floatx4& sc,
                                             floatx4& gram, float& g_mine, float& sq_mine) {
  const uint32_t col = lane % kBlock;
  const float g = sc[0] + sc[1];
  const uint32_t e = col % 4u;
  const float d = e == 0u ? gram[0] : (e == 1u ? gram[1] : (e == 2u ? gram[2] : gram[3]));
  const float gv = __shfl(g, static_cast<int>(col));
  const float dv = __shfl(d, static_cast<int>(col + kBlock * (col / 4u)));
  if (lane / kBlock == j) {
    g_mine = gv;
    sq_mine = dv;
  }
  sc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  gram = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
}

// Tile k of row r: candidates [64 k, 64 k + n) of the row's list.
// The wave's LDS stage holds row `staged`'s y_hi then y_lo (2 H halves).
template <int KC>
__device__ void mfma_tile(const GatherArgs& a, uint32_t r, uint32_t k, uint32_t list_begin,
                          uint32_t count, uint16_t* stage, uint32_t& staged) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t begin = k * a.tile;
  const uint32_t n = count - begin < a.tile ? count - begin : a.tile;
  const bool live = lane < n;
  const uint32_t id = a.tokens[list_begin + begin + (live ? lane : n - 1)];
  const uint32_t t = live ? id : 0u;
  const float yn = a.row_norm[r];
  const float row_slack = a.row_slack[r];
  TileRecord* rec = a.records + static_cast<uint64_t>(r) * a.max_tiles + k;
  if (__ballot(live && t >= a.V) != 0ull) {
    // an id outside the vocabulary: the row's result is the invalid sentinel
    if (lane == 0) {
      rec->best_lower = -__builtin_huge_valf();
      rec->flags = kTileInvalid;
      rec->min_token = kInvalidToken;
      rec->min_pos = begin;
      rec->begin = begin;
      rec->count = n;
      rec->n_members = 0u;
    }
    return;
  }

  const uint32_t H = a.H;
  const uint32_t chunks = H / (kStep * KC);
  const uint32_t nblocks = (n + kBlock - 1) / kBlock;
  const uint32_t units = nblocks * chunks;
  const uint32_t kb = lane / kBlock;   // k-block: features 8 kb .. 8 kb + 7 of a step
  const uint32_t col = lane % kBlock;  // B column (token) and A row of this lane
  const uint32_t unit_f = kStep * KC;
  // the B column's token of each block (lane col of block j holds candidate
  // 16 j + col), gathered once per tile
  uint32_t btok[4];
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    btok[j] = static_cast<uint32_t>(__shfl(static_cast<int>(t), static_cast<int>(j * kBlock + col)));
  }
  // unit q = (block q / chunks, chunk q % chunks); j is wave-uniform
  auto load_q = [&](uint32_t q, Operands<KC>& o) {
    const uint32_t j = q / chunks;
    const uint32_t bt = j == 0u ? btok[0] : (j == 1u ? btok[1] : (j == 2u ? btok[2] : btok[3]));
    load_unit<KC>(a.emb + static_cast<uint64_t>(bt) * H + kb * 8u, (q % chunks) * unit_f, o);
  };
  Operands<KC> o0, o1;
  // the first unit's table rows are in flight during the staging
  load_q(0, o0);
  if (staged != r) {
    // the row's FP16 split into the wave's stage (16 bytes per copy), four
    // loads per lane in flight before their stores
    constexpr uint32_t kBatch = 4;
    const uint32_t per = H / 8;
    const uint32_t n = 2u * per;
    for (uint32_t base = lane; base < n; base += kWave * kBatch) {
      uint4 v[kBatch];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t q = base + u * kWave;
        const uint16_t* src = (q < per ? a.y_hi : a.y_lo) + static_cast<uint64_t>(r) * H;
        v[u] = q < n ? *reinterpret_cast<const uint4*>(src + (q % per) * 8) : uint4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t q = base + u * kWave;
        if (q < n) *reinterpret_cast<uint4*>(stage + q * 8) = v[u];
      }
    }
    staged = r;
    // LDS writes of this wave complete before any lane reads them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // A rows 0 (hi) and 1 (lo); rows 2..15 read lo too and are masked
  const uint32_t amask = col < 2u ? 0xFFFFFFFFu : 0u;
  const uint16_t* a_lane = stage + (col == 0u ? 0u : H) + kb * 8u;

  floatx4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
  floatx4 gram = {0.0f, 0.0f, 0.0f, 0.0f};
  float g_mine = 0.0f;
  float sq_mine = 0.0f;
  // two units in flight; sched_barrier(0) keeps each unit's loads issued
  // before the previous unit's MFMAs, and no load sits under a branch in
  // the steady-state loop.
  auto mma_q = [&](uint32_t q, const Operands<KC>& o) {
    mma_unit<KC>(o, a_lane, (q % chunks) * unit_f, amask, sc, gram);
    if (q % chunks == chunks - 1u) finish_block(q / chunks, lane, sc, gram, g_mine, sq_mine);
  };
  uint32_t q = 0;
  for (; q + 2 < units; q += 2) {
    load_q(q + 1, o1);
    __builtin_amdgcn_sched_barrier(0);
    mma_q(q, o0);
    __builtin_amdgcn_sched_barrier(0);
    load_q(q + 2, o0);
    __builtin_amdgcn_sched_barrier(0);
    mma_q(q + 1, o1);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the last one or two units
  if (q + 1 < units) {
    load_q(q + 1, o1);
    __builtin_amdgcn_sched_barrier(0);
    mma_q(q, o0);
    mma_q(q + 1, o1);
  } else {
    mma_q(q, o0);
  }

  // window summary of the tile (the candidate of lane l is list position
  // begin + l); the bound is |g - r / inv| <= ||e|| (coef ||z|| + coef2) +
  // the row's slack, r the reference-order score
  const float tn = __fsqrt_rn(sq_mine) * (1.0f + 0x1p-7f);
  const float g = g_mine;
  const float b = __builtin_fmaf(tn, __builtin_fmaf(a.coef, yn, a.coef2), row_slack);
  const bool fin = !live || (__builtin_isfinite(g) && __builtin_isfinite(b) && b < 0x1p100f);
  const bool all_finite = __ballot(!fin) == 0ull;
  const float L = wave_max(live ? g - b : -__builtin_huge_valf());
  uint32_t mt = live ? t : kInvalidToken;
  uint32_t mp = begin + lane;
  wave_min_token(mt, mp);
  const float U = wave_max(live ? g + b : -__builtin_huge_valf());
  const bool member = all_finite && live && g + b >= L;
  const uint64_t mask = __ballot(member);
  const uint32_t total = static_cast<uint32_t>(__popcll(mask));
  const bool ordinary = all_finite && total <= static_cast<uint32_t>(kTileMembers);
  if (ordinary && member) {
    const uint32_t rank = static_cast<uint32_t>(__popcll(mask & ((1ull << lane) - 1ull)));
    rec->m[rank] = TileMember{t, begin + lane, g - b, g + b};
  }
  if (lane == 0) {
    rec->best_lower = L;
    rec->flags = ordinary ? 0u : (all_finite ? kTileRescoreAll | kTileCrowded : kTileRescoreAll);
    rec->min_token = mt;
    rec->min_pos = mp;
    rec->begin = begin;
    rec->count = n;
    rec->n_members = ordinary ? total : 0u;
    rec->upper_max = U;
  }
}

// LDS of a chain workgroup: the weight [H], one inv per wave (4 floats), then
// per wave x and its squares [2 H] (H % 4 == 0 keeps every part 16-byte
// aligned).
__host__ __device__ constexpr uint32_t chain_lds_bytes(uint32_t H) {
  return (H + 4u + static_cast<uint32_t>(kWaves) * 2u * H) * 4u;
}

// Chain workgroup b: its waves normalize rows kWaves b .. kWaves b + 3 in the
// reference order (the finalize's rescore needs y and inv; the fast scores
// of this launch do not).
__device__ void chain_block(const GatherArgs& a, float* lds) {
  const uint32_t H = a.H;
  float* w = lds;
  float* inv = lds + H;
  const uint32_t wave = threadIdx.x / kWave;
  float* xs = lds + H + 4u + wave * 2u * H;
  float* sq = xs + H;
  for (uint32_t q = threadIdx.x; q < H / 4u; q += kThreads) {
    reinterpret_cast<float4*>(w)[q] = reinterpret_cast<const float4*>(a.weight)[q];
  }
  __syncthreads();
  const uint32_t r = blockIdx.x * kWaves + wave;
  if (r < a.chain_rows) {
    norm_chain_wave(a.x, w, a.y_out, a.inv_out, r, H, a.epsilon, xs, sq, inv + wave);
  }
}

// Planned mode: the tile plan, then wave slot s of the grid's S slots walks
// tiles [W s / S, W (s + 1) / S).  The first chain workgroups of the grid run
// the norm's reference-order chains instead.
template <int KC>
__global__ __launch_bounds__(kThreads) void gather_mfma_kernel(GatherArgs a) {
  __shared__ TilePlan<kThreads> plan;
  extern __shared__ __align__(16) uint16_t stages[];  // [waves][2 H]
  const uint32_t chain_groups = (a.chain_rows + kWaves - 1) / kWaves;
  if (blockIdx.x < chain_groups) {
    chain_block(a, reinterpret_cast<float*>(stages));
    return;
  }
  uint16_t* stage = stages + static_cast<size_t>(threadIdx.x / kWave) * 2u * a.H;
  uint32_t staged = kInvalidToken;
  const uint64_t W = plan_tiles<kThreads>(a.row_meta, a.rows, a.tile, false, plan);
  const uint64_t slots = static_cast<uint64_t>(gridDim.x - chain_groups) * kWaves;
  const uint64_t me =
      static_cast<uint64_t>(blockIdx.x - chain_groups) * kWaves + threadIdx.x / kWave;
  const uint32_t w0 = static_cast<uint32_t>(W * me / slots);
  const uint32_t w1 = static_cast<uint32_t>(W * (me + 1) / slots);
  if (w0 >= w1) return;
  uint32_t r = plan_row_of<kThreads>(plan, a.rows, w0);
  for (uint32_t w = w0; w < w1; ++w) {
    while (plan.prefix[r + 1] <= w) ++r;
    mfma_tile<KC>(a, r, w - plan.prefix[r], plan.begin[r], plan.count[r], stage, staged);
  }
}

// Grid mode (rows above the plan's capacity): one wave per (row, tile),
// blockIdx.x = k * rows + r.
template <int KC>
__global__ __launch_bounds__(kWave) void gather_mfma_grid_kernel(GatherArgs a) {
  const uint32_t r = blockIdx.x % a.rows;
  const uint32_t k = blockIdx.x / a.rows;
  extern __shared__ __align__(16) uint16_t stages[];  // [2 H]
  const RowMeta meta = a.row_meta[r];
  if (!row_gathered(meta, false) || k * a.tile >= meta.count) return;
  uint32_t staged = kInvalidToken;
  mfma_tile<KC>(a, r, k, meta.list_begin, meta.count, stages, staged);
}

// Workgroups of gather_mfma_kernel<KC> one compute unit holds with `lds`
// bytes of dynamic LDS (cached per size: with and without chain waves).
template <int KC>
int resident_groups(uint32_t lds) {
  static std::atomic<uint64_t> cache[2];  // (lds << 8) | count
  for (auto& c : cache) {
    const uint64_t v = c.load(std::memory_order_relaxed);
    if (v != 0 && (v >> 8) == lds) return static_cast<int>(v & 0xFFu);
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &n, reinterpret_cast<const void*>(gather_mfma_kernel<KC>), kThreads, lds) != hipSuccess ||
      n <= 0) {
    n = 1;
  }
  if (n > 255) n = 255;
  const uint64_t v = (static_cast<uint64_t>(lds) << 8) | static_cast<uint64_t>(n);
  for (auto& c : cache) {
    uint64_t expected = 0;
    if (c.compare_exchange_strong(expected, v)) break;
  }
  return n;
}

template <int KC>
hipError_t launch_variant(const GatherArgs& a, hipStream_t stream) {
  if (a.rows <= kPlanRowsMax && a.groups > 0) {
    const uint32_t stage_lds = kWaves * 4u * a.H;
    const uint32_t chain_groups = (a.chain_rows + kWaves - 1) / kWaves;
    if (chain_groups > 0 && (a.H % 4u != 0 || a.x == nullptr || a.weight == nullptr ||
                             a.y_out == nullptr || a.inv_out == nullptr)) {
      return hipErrorInvalidValue;
    }
    const uint32_t lds =
        chain_groups > 0 && chain_lds_bytes(a.H) > stage_lds ? chain_lds_bytes(a.H) : stage_lds;
    // with chain workgroups the gather takes two workgroups per compute unit
    // so that every CU carries the same gather share (a CU's share is
    // bounded by what its memory pipeline moves) and the chain workgroups
    // find a free slot
    uint32_t per_cu = static_cast<uint32_t>(resident_groups<KC>(stage_lds));
    if (chain_groups > 0) {
      const uint32_t with_chain = static_cast<uint32_t>(resident_groups<KC>(lds));
      per_cu = with_chain > 2u ? 2u : (with_chain > 1u ? with_chain - 1u : 1u);
    }
    const uint32_t g = a.groups * per_cu;
    hipLaunchKernelGGL((gather_mfma_kernel<KC>), dim3(chain_groups + g), dim3(kThreads), lds,
                       stream, a);
    return hipGetLastError();
  }
  if (a.chain_rows > 0) return hipErrorInvalidValue;  // chains run in planned mode only
  const uint64_t slots = static_cast<uint64_t>(a.rows) * a.max_tiles;
  if (slots > 0x7FFFFFFFull) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gather_mfma_grid_kernel<KC>), dim3(static_cast<uint32_t>(slots)),
                     dim3(kWave), 4u * a.H, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gather_mfma(const GatherArgs& a, hipStream_t stream) {
  if (a.H == 0 || a.H % kStep != 0 ||
      (a.tile != 16u && a.tile != 32u && a.tile != kGatherWaveTile) || a.y_hi == nullptr ||
      a.y_lo == nullptr || a.row_norm == nullptr || a.row_slack == nullptr) {
    return hipErrorInvalidValue;
  }
  const uint32_t steps = a.H / kStep;
  if (steps % 9 == 0) return launch_variant<9>(a, stream);
  if (steps % 8 == 0) return launch_variant<8>(a, stream);
  if (steps % 6 == 0) return launch_variant<6>(a, stream);
  if (steps % 4 == 0) return launch_variant<4>(a, stream);
  if (steps % 2 == 0) return launch_variant<2>(a, stream);
  return launch_variant<1>(a, stream);
}

}  // namespace mf
