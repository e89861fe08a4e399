// C ABI of the gfx950 restricted head (include/marketforge_hip.h).
//
// Host-side validation mirrors the reference operators check for check and in
// the same order (src/cuda/greedy.cu:237-414, src/cuda/rms_norm.cu:104-182,
// src/cuda/linear.cu:40-81, src/cuda/device_buffer.cu:15-103), then launches.
// Nothing here allocates device memory except mf_device_alloc itself, and
// nothing synchronizes except mf_stream_synchronize.
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <limits>
#include <mutex>

#include <hip/hip_runtime.h>

#include "marketforge_hip.h"
#include "mf_device.hpp"
#include "mf_launch.hpp"

namespace {

using mf::HeadArgs;
using mf::ScoreSource;

constexpr uint64_t kU64Max = std::numeric_limits<uint64_t>::max();
constexpr uint64_t kU32Max = std::numeric_limits<uint32_t>::max();
constexpr uint64_t kIntMax = static_cast<uint64_t>(std::numeric_limits<int>::max());

mf_status status(int32_t code, uint32_t detail = 0) { return mf_status{code, detail}; }
mf_status ok() { return status(MF_OK); }

// src/cuda/cuda_internal.hpp:21-35
mf_status runtime_status(hipError_t e) {
  return e == hipSuccess ? ok() : status(MF_DEVICE_RUNTIME_FAILURE, static_cast<uint32_t>(e));
}
mf_status launch_status(hipError_t e) {
  return e == hipSuccess ? ok() : status(MF_DEVICE_BACKEND_FAILURE, static_cast<uint32_t>(e));
}

hipStream_t native(uintptr_t stream) { return reinterpret_cast<hipStream_t>(stream); }

template <typename T>
T* ptr(uintptr_t address) {
  return reinterpret_cast<T*>(address);
}

bool checked_mul(uint64_t a, uint64_t b, uint64_t& out) {
  if (a != 0 && b > kU64Max / a) return false;
  out = a * b;
  return true;
}

// Every address valid (non-zero) and pairwise distinct (greedy.cu:214-233).
bool distinct_valid(std::initializer_list<uintptr_t> addresses) {
  for (auto i = addresses.begin(); i != addresses.end(); ++i) {
    if (*i == 0) return false;
    for (auto j = i + 1; j != addresses.end(); ++j) {
      if (*i == *j) return false;
    }
  }
  return true;
}

uint64_t align256(uint64_t v) { return (v + 255u) & ~uint64_t{255u}; }

// gamma_n = n u / (1 - n u) (Higham): bound on the relative error of an
// n-term floating-point dot product in any evaluation order.
double gamma(double n, double u) { return n * u / (1.0 - n * u); }

// Fast FP32 dot vs reference order, both within gamma_H * sum|y e| of the
// exact value; the computed sum|y e| is at most (1 - gamma_H) low.  Factor 2
// of safety plus 16 u so the window test's own roundings stay inside.
float dot_bound_coef(uint64_t H) {
  const double g = gamma(static_cast<double>(H), std::ldexp(1.0, -24));
  return static_cast<float>(4.0 * g / (1.0 - g) + std::ldexp(1.0, -20));
}

// MFMA score g on z = x * w (hi + lo FP16 split, exact FP16 products, 2H FP32
// additions with up to one ulp each) against the reference-order score r on
// y = (x * inv) * w, in the scale of z (inv > 0 orders both alike):
//   |g - S_z|         <= (1.001 gamma'_2H + 2^-22) ||z|| ||e|| + 2^-25 sqrt(H) ||e||
//   |S_y / inv - S_z| <= 3.0001 u ||z|| ||e||   (y_f / inv and z_f differ by
//                                               three roundings, u = 2^-24)
//   |r - S_y| / inv   <= gamma_H (1 + 3.0001 u) ||z|| ||e||
// (S_v = the exact dot product of v with e; Sum |y e| / inv <= (1 + 3.0001 u)
// ||z|| ||e||), doubled for safety.  Without a norm weight z = y and inv = 1.
void mfma_bound_coefs(uint64_t H, float& coef, float& coef2) {
  const double h = static_cast<double>(H);
  const double u = std::ldexp(1.0, -24);
  const double c = gamma(h, u) * (1.0 + 4.0 * u) + 4.0 * u +
                   1.001 * gamma(2.0 * h, std::ldexp(1.0, -23)) + std::ldexp(1.0, -22);
  coef = static_cast<float>(2.0 * c + std::ldexp(1.0, -20));
  coef2 = static_cast<float>(2.0 * std::ldexp(1.0, -25) * std::sqrt(h));
}

// The table pass's candidate score g on hi = rne_f16(z) alone (exact FP16
// products, H FP32 additions): |hi_f - z_f| <= 2^-11 |z_f| + 2^-25 (FP16
// subnormals; |z_f| past the FP16 range makes g infinite and the candidate
// is rescored), so
//   |g - S_hi|   <= 1.001 gamma'_H (1 + 2^-10) ||z|| ||e||   (+ the 2^-25 term)
//   |S_hi - S_z| <= 2^-11 ||z|| ||e|| + 2^-25 sqrt(H) ||e||
// and the reference-order terms of mfma_bound_coefs, doubled for safety.
void pass_bound_coefs(uint64_t H, float& coef, float& coef2) {
  const double h = static_cast<double>(H);
  const double u = std::ldexp(1.0, -24);
  const double acc = 1.001 * gamma(h, std::ldexp(1.0, -23));
  const double c = gamma(h, u) * (1.0 + 4.0 * u) + 4.0 * u +
                   acc * (1.0 + std::ldexp(1.0, -10)) + std::ldexp(1.0, -11);
  coef = static_cast<float>(2.0 * c + std::ldexp(1.0, -20));
  coef2 = static_cast<float>(2.0 * std::ldexp(1.0, -25) * std::sqrt(h) * (1.0 + acc));
}

// Absolute term for underflow: each of up to 2H operations may lose 2^-126.
float underflow_slack(uint64_t H) {
  return static_cast<float>(4.0 * static_cast<double>(H) * std::ldexp(1.0, -126));
}

// The underflow of the reference score and of y, per unit of 1 / inv (the
// norm kernel multiplies it by its bound of 1 / inv): the chain's 2H
// operations, and two roundings of each y_f against |e_f| <= 65504.
float scaled_slack(uint64_t H) {
  const double h = static_cast<double>(H);
  return static_cast<float>(4.0 * h * std::ldexp(1.0, -126) + 2.0 * h * 65504.0 * std::ldexp(1.0, -148));
}

// Compute units of the current device (cached per device id).
uint32_t device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
      n = 256;
    }
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return static_cast<uint32_t>(n);
}


uint32_t head_chunk(uint64_t H, uint64_t max_count) {
  uint32_t c = H == 576 ? 128u : 64u;
  while (c < mf::kHeadChunkMax &&
         (max_count + c - 1) / c > mf::kHeadMaxRecords) {
    c *= 2;
  }
  return c;
}

}  // namespace

extern "C" {

uint32_t mf_abi_version(void) { return MF_ABI_VERSION; }

mf_status mf_device_count(int32_t* count) {
  if (count == nullptr) return status(MF_INVALID_ARGUMENT);
  int n = 0;
  const hipError_t e = hipGetDeviceCount(&n);
  *count = e == hipSuccess ? n : 0;
  return runtime_status(e);
}

// ---------------------------------------------------------------- plumbing --

mf_status mf_device_alloc(uint64_t bytes, uintptr_t* address) {
  if (address == nullptr) return status(MF_INVALID_ARGUMENT);
  *address = 0;
  if (bytes == 0) return ok();
  if (bytes > std::numeric_limits<size_t>::max()) return status(MF_ARITHMETIC_OVERFLOW);
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, static_cast<size_t>(bytes));
  if (e != hipSuccess) return runtime_status(e);
  *address = reinterpret_cast<uintptr_t>(p);
  return ok();
}

mf_status mf_device_free(uintptr_t address) {
  if (address == 0) return ok();
  return runtime_status(hipFree(ptr<void>(address)));
}

// src/cuda/device_buffer.cu:15-33 (validate_copy)
static mf_status validate_copy(const void* host, uint64_t bytes, uint64_t offset,
                               uint64_t size, uintptr_t stream) {
  if (stream == 0 || (bytes != 0 && host == nullptr)) return status(MF_INVALID_ARGUMENT);
  if (offset > kU64Max - bytes) return status(MF_ARITHMETIC_OVERFLOW);
  if (offset + bytes > size) return status(MF_INVALID_ARGUMENT);
  if (bytes > std::numeric_limits<size_t>::max()) return status(MF_ARITHMETIC_OVERFLOW);
  return ok();
}

mf_status mf_copy_to_device_async(mf_buffer destination, uint64_t offset, const void* source,
                                  uint64_t bytes, uintptr_t stream) {
  const mf_status v = validate_copy(source, bytes, offset, destination.bytes, stream);
  if (v.code != MF_OK || bytes == 0) return v;
  return runtime_status(hipMemcpyAsync(ptr<char>(destination.address) + offset, source,
                                       static_cast<size_t>(bytes), hipMemcpyHostToDevice,
                                       native(stream)));
}

mf_status mf_copy_to_host_async(void* destination, mf_buffer source, uint64_t offset,
                                uint64_t bytes, uintptr_t stream) {
  const mf_status v = validate_copy(destination, bytes, offset, source.bytes, stream);
  if (v.code != MF_OK || bytes == 0) return v;
  return runtime_status(hipMemcpyAsync(destination, ptr<const char>(source.address) + offset,
                                       static_cast<size_t>(bytes), hipMemcpyDeviceToHost,
                                       native(stream)));
}

mf_status mf_stream_create(uintptr_t* stream) {
  if (stream == nullptr) return status(MF_INVALID_ARGUMENT);
  *stream = 0;
  hipStream_t s = nullptr;
  const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return runtime_status(e);
  *stream = reinterpret_cast<uintptr_t>(s);
  return ok();
}

mf_status mf_stream_destroy(uintptr_t stream) {
  if (stream == 0) return ok();
  return runtime_status(hipStreamDestroy(native(stream)));
}

mf_status mf_stream_synchronize(uintptr_t stream) {
  if (stream == 0) return status(MF_INVALID_ARGUMENT);
  return runtime_status(hipStreamSynchronize(native(stream)));
}

// --------------------------------------------------------------- RMSNorm ----

// src/cuda/rms_norm.cu:104-141 (FP32) and :143-182 (FP16) check order.
static mf_status rms_norm(mf_buffer input, mf_buffer weight, mf_buffer output, uint64_t rows,
                          uint64_t hidden, float epsilon, uintptr_t stream, bool half) {
  if (rows == 0 || hidden == 0 || !std::isfinite(epsilon) || epsilon <= 0.0f || stream == 0) {
    return status(MF_INVALID_ARGUMENT);
  }
  const uint64_t esize = half ? 2u : 4u;
  uint64_t elements = 0, tensor_bytes = 0, weight_bytes = 0;
  if (!checked_mul(rows, hidden, elements) || !checked_mul(elements, esize, tensor_bytes) ||
      !checked_mul(hidden, esize, weight_bytes)) {
    return status(MF_ARITHMETIC_OVERFLOW);
  }
  if (input.bytes != tensor_bytes || output.bytes != tensor_bytes ||
      weight.bytes != weight_bytes || input.address == 0 || output.address == 0 ||
      weight.address == 0 || weight.address == input.address ||
      weight.address == output.address) {
    return status(MF_INVALID_ARGUMENT);
  }
  if (rows > kIntMax) return status(MF_RESOURCE_LIMIT);
  if (hidden > kU32Max) return status(MF_RESOURCE_LIMIT);
  return launch_status(mf::launch_rms_norm(
      ptr<const void>(input.address), half, ptr<const void>(weight.address), half,
      ptr<void>(output.address), half, nullptr, static_cast<uint32_t>(rows),
      static_cast<uint32_t>(hidden), epsilon, native(stream)));
}

mf_status mf_rms_norm_f32(mf_buffer input, mf_buffer weight, mf_buffer output, uint64_t rows,
                          uint64_t hidden_size, float epsilon, uintptr_t stream) {
  return rms_norm(input, weight, output, rows, hidden_size, epsilon, stream, false);
}

mf_status mf_rms_norm_f16(mf_buffer input, mf_buffer weight, mf_buffer output, uint64_t rows,
                          uint64_t hidden_size, float epsilon, uintptr_t stream) {
  return rms_norm(input, weight, output, rows, hidden_size, epsilon, stream, true);
}

// ---------------------------------------------------------------- greedy ----

// src/cuda/greedy.cu:237-279
static mf_status greedy(mf_buffer logits, mf_buffer token_ids, uint64_t rows, uint64_t vocab,
                        uintptr_t stream, bool half) {
  if (rows == 0 || vocab == 0 || stream == 0) return status(MF_INVALID_ARGUMENT);
  if (vocab > kU32Max) return status(MF_RESOURCE_LIMIT);
  if (rows > kIntMax) return status(MF_RESOURCE_LIMIT);
  if (rows > kU64Max / vocab) return status(MF_ARITHMETIC_OVERFLOW);
  const uint64_t elements = rows * vocab;
  const uint64_t esize = half ? 2u : 4u;
  if (elements > kU64Max / esize || rows > kU64Max / 4u) return status(MF_ARITHMETIC_OVERFLOW);
  if (logits.bytes != elements * esize || token_ids.bytes != rows * 4u || logits.address == 0 ||
      token_ids.address == 0 || logits.address == token_ids.address) {
    return status(MF_INVALID_ARGUMENT);
  }
  return launch_status(mf::launch_greedy(ptr<const void>(logits.address), half,
                                         ptr<uint32_t>(token_ids.address),
                                         static_cast<uint32_t>(rows),
                                         static_cast<uint32_t>(vocab), native(stream)));
}

mf_status mf_greedy_select_f16(mf_buffer logits, mf_buffer token_ids, uint64_t rows,
                               uint64_t vocabulary_size, uintptr_t stream) {
  return greedy(logits, token_ids, rows, vocabulary_size, stream, true);
}

mf_status mf_greedy_select_f32(mf_buffer logits, mf_buffer token_ids, uint64_t rows,
                               uint64_t vocabulary_size, uintptr_t stream) {
  return greedy(logits, token_ids, rows, vocabulary_size, stream, false);
}

// src/cuda/greedy.cu:281-347
static mf_status restricted_greedy(mf_buffer logits, mf_buffer allowed, mf_buffer counts,
                                   mf_buffer token_ids, uint64_t rows, uint64_t vocab,
                                   uint64_t max_allowed, uintptr_t stream, bool half) {
  if (rows == 0 || vocab == 0 || max_allowed == 0 || stream == 0) {
    return status(MF_INVALID_ARGUMENT);
  }
  if (vocab > kU32Max || max_allowed > kU32Max || rows > kIntMax) {
    return status(MF_RESOURCE_LIMIT);
  }
  if (rows > kU64Max / vocab || rows > kU64Max / max_allowed) {
    return status(MF_ARITHMETIC_OVERFLOW);
  }
  const uint64_t logit_elements = rows * vocab;
  const uint64_t allowed_elements = rows * max_allowed;
  const uint64_t esize = half ? 2u : 4u;
  if (logit_elements > kU64Max / esize || allowed_elements > kU64Max / 4u ||
      rows > kU64Max / 4u) {
    return status(MF_ARITHMETIC_OVERFLOW);
  }
  if (logits.bytes != logit_elements * esize || allowed.bytes != allowed_elements * 4u ||
      counts.bytes != rows * 4u || token_ids.bytes != rows * 4u ||
      !distinct_valid({logits.address, allowed.address, counts.address, token_ids.address})) {
    return status(MF_INVALID_ARGUMENT);
  }
  return launch_status(mf::launch_restricted_greedy(
      ptr<const void>(logits.address), half, ptr<const uint32_t>(allowed.address),
      ptr<const uint32_t>(counts.address), ptr<uint32_t>(token_ids.address),
      static_cast<uint32_t>(rows), static_cast<uint32_t>(vocab),
      static_cast<uint32_t>(max_allowed), native(stream)));
}

mf_status mf_restricted_greedy_select_f16(mf_buffer logits, mf_buffer allowed_token_ids,
                                          mf_buffer allowed_token_counts, mf_buffer token_ids,
                                          uint64_t rows, uint64_t vocabulary_size,
                                          uint64_t maximum_allowed_tokens, uintptr_t stream) {
  return restricted_greedy(logits, allowed_token_ids, allowed_token_counts, token_ids, rows,
                           vocabulary_size, maximum_allowed_tokens, stream, true);
}

mf_status mf_restricted_greedy_select_f32(mf_buffer logits, mf_buffer allowed_token_ids,
                                          mf_buffer allowed_token_counts, mf_buffer token_ids,
                                          uint64_t rows, uint64_t vocabulary_size,
                                          uint64_t maximum_allowed_tokens, uintptr_t stream) {
  return restricted_greedy(logits, allowed_token_ids, allowed_token_counts, token_ids, rows,
                           vocabulary_size, maximum_allowed_tokens, stream, false);
}

// ------------------------------------------------------- restricted head ----

// src/cuda/greedy.cu:349-414
mf_status mf_restricted_output_head_f16(mf_buffer hidden, mf_buffer embedding,
                                        mf_buffer allowed_token_ids,
                                        mf_buffer allowed_token_counts, mf_buffer token_ids,
                                        uint64_t rows, uint64_t hidden_size,
                                        uint64_t vocabulary_size,
                                        uint64_t maximum_allowed_tokens, uintptr_t stream) {
  if (rows == 0 || hidden_size == 0 || vocabulary_size == 0 || maximum_allowed_tokens == 0 ||
      stream == 0) {
    return status(MF_INVALID_ARGUMENT);
  }
  if (vocabulary_size > kU32Max || maximum_allowed_tokens > kU32Max || rows > kIntMax) {
    return status(MF_RESOURCE_LIMIT);
  }
  if (rows > kU64Max / hidden_size || vocabulary_size > kU64Max / hidden_size ||
      rows > kU64Max / maximum_allowed_tokens) {
    return status(MF_ARITHMETIC_OVERFLOW);
  }
  const uint64_t hidden_elements = rows * hidden_size;
  const uint64_t embedding_elements = vocabulary_size * hidden_size;
  const uint64_t allowed_elements = rows * maximum_allowed_tokens;
  if (hidden_elements > kU64Max / 2u || embedding_elements > kU64Max / 2u ||
      allowed_elements > kU64Max / 4u || rows > kU64Max / 4u) {
    return status(MF_ARITHMETIC_OVERFLOW);
  }
  if (hidden.bytes != hidden_elements * 2u || embedding.bytes != embedding_elements * 2u ||
      allowed_token_ids.bytes != allowed_elements * 4u ||
      allowed_token_counts.bytes != rows * 4u || token_ids.bytes != rows * 4u ||
      !distinct_valid({hidden.address, embedding.address, allowed_token_ids.address,
                       allowed_token_counts.address, token_ids.address})) {
    return status(MF_INVALID_ARGUMENT);
  }
  HeadArgs a{};
  a.hidden16 = ptr<const uint16_t>(hidden.address);
  a.emb = ptr<const uint16_t>(embedding.address);
  a.fixed_ids = ptr<const uint32_t>(allowed_token_ids.address);
  a.fixed_counts = ptr<const uint32_t>(allowed_token_counts.address);
  a.out_token = ptr<uint32_t>(token_ids.address);
  a.rows = static_cast<uint32_t>(rows);
  a.H = static_cast<uint32_t>(hidden_size);
  a.V = static_cast<uint32_t>(vocabulary_size);
  a.max_allowed = static_cast<uint32_t>(maximum_allowed_tokens);
  a.chunk = head_chunk(hidden_size, maximum_allowed_tokens);
  a.coef = dot_bound_coef(hidden_size);
  a.slack = underflow_slack(hidden_size);
  a.order = MF_ORDER_FMA_CHAIN;  // greedy.cu:171-176
  return launch_status(mf::launch_head(a, native(stream)));
}

// ------------------------------------------------------------------ linear ---

// src/cuda/linear.cu:40-81 (the handle check has no counterpart here)
mf_status mf_linear_f16(mf_buffer input, mf_buffer weight, mf_buffer output, uint64_t rows,
                        uint64_t input_features, uint64_t output_features, uintptr_t stream) {
  if (stream == 0) return status(MF_INVALID_ARGUMENT);
  auto matrix_bytes = [](uint64_t r, uint64_t c, uint64_t& bytes) -> mf_status {
    if (r == 0 || c == 0) return status(MF_INVALID_ARGUMENT);
    if (r > kU64Max / c) return status(MF_ARITHMETIC_OVERFLOW);
    const uint64_t e = r * c;
    if (e > kU64Max / 2u) return status(MF_ARITHMETIC_OVERFLOW);
    bytes = e * 2u;
    return ok();
  };
  uint64_t ib = 0, wb = 0, ob = 0;
  mf_status s = matrix_bytes(rows, input_features, ib);
  if (s.code != MF_OK) return s;
  s = matrix_bytes(output_features, input_features, wb);
  if (s.code != MF_OK) return s;
  s = matrix_bytes(rows, output_features, ob);
  if (s.code != MF_OK) return s;
  if (rows > kIntMax || input_features > kIntMax || output_features > kIntMax) {
    return status(MF_RESOURCE_LIMIT);
  }
  if (input.bytes != ib || weight.bytes != wb || output.bytes != ob || input.address == 0 ||
      weight.address == 0 || output.address == 0 || input.address == weight.address ||
      input.address == output.address || weight.address == output.address) {
    return status(MF_INVALID_ARGUMENT);
  }
  const bool mfma_shape = (input_features % 32u) == 0 && (input.address % 16u) == 0 &&
                          (weight.address % 16u) == 0 && output_features <= kU32Max &&
                          rows <= kU32Max;
  if (mfma_shape) {
    mf::ProjArgs p{};
    p.a16 = ptr<const uint16_t>(input.address);
    p.m = static_cast<uint32_t>(rows);
    p.emb = ptr<const uint16_t>(weight.address);
    p.H = static_cast<uint32_t>(input_features);
    p.V = static_cast<uint32_t>(output_features);
    p.out_f16 = ptr<uint16_t>(output.address);
    return launch_status(mf::launch_projection(p, native(stream)));
  }
  return launch_status(mf::launch_linear_f16_simple(
      ptr<const uint16_t>(input.address), ptr<const uint16_t>(weight.address),
      ptr<uint16_t>(output.address), static_cast<uint32_t>(rows),
      static_cast<uint32_t>(input_features), static_cast<uint32_t>(output_features),
      native(stream)));
}

// ------------------------------------------------------------ decode tail ----

namespace {

constexpr uint32_t kFullTile = 256;  // selection over projected scores

struct TailLayout {
  uint64_t y, row_inv, row_norm, row_slack, row_meta, y_hi, y_lo, fb_map, records, fb_records,
      fb_panel, fb_slot_row, fb_slot_norm, fb_slot_slack, scores, tok_norm, range_index,
      row_tiles, dense_spans, dense_flag, total;
  uint32_t tile, max_tiles, fb_tiles, fb_rows;
  uint64_t short_counts, short_records;
  uint32_t short_per_part, short_parts;
  bool pass;   // the table pass serves both kinds of rows
  bool fused;  // the one-kernel tail (short lists)
  bool dense;  // the dense head serves unrestricted rows and long ascending lists
};

bool buffer_is(const mf_buffer& b, uint64_t bytes) { return b.address != 0 && b.bytes == bytes; }
bool optional_is(const mf_buffer& b, uint64_t bytes) {
  return b.address == 0 || b.bytes == bytes;
}

// The restricted gather runs on MFMA when H is a multiple of the 32-feature
// MFMA step (64-candidate wave tiles); otherwise on the VALU dot.
bool mfma_gather(uint64_t H) { return H % 32u == 0; }
// Candidates per gather tile (one wave each on the MFMA gather).  Tiles of
// 64 unless the pack is small: when even the upper bound of its 64-candidate
// tiles (every row as long as the longest list) stays under four per
// compute unit of an MI355X (256 CUs), a wave would stream 64 rows through
// eight dependent load units while most SIMDs idle, so the tiles shrink to
// 32 or 16 candidates (more waves, one or two units each; the finalize
// merges the extra records).
constexpr uint64_t kGatherSmallPack = 4u * 256u;
uint32_t gather_tile(uint64_t H, uint64_t rows, uint64_t max_count) {
  if (!mfma_gather(H)) return H == 2048 ? 128u : 64u;
  const uint64_t lists = max_count == 0 ? 1 : max_count;
  const uint64_t t64 = rows * ((lists + mf::kGatherWaveTile - 1) / mf::kGatherWaveTile);
  if (t64 >= kGatherSmallPack) return mf::kGatherWaveTile;
  const uint64_t t32 = rows * ((lists + 31) / 32);
  return t32 >= kGatherSmallPack ? 32u : 16u;
}

// The table pass (one launch for restricted and unrestricted rows): lists
// declared ascending, the whole table read anyway (unrestricted rows) or the
// pass asked for, a panel tile that fits LDS, the row plan in LDS.
bool table_pass(const mf_decode_tail_args* a) {
  return (a->flags & MF_TAIL_SORTED_LISTS) &&
         (a->unrestricted_count > 0 || (a->flags & MF_TAIL_TABLE_PASS)) && a->hidden % 64u == 0 &&
         mf::panel_tile_bytes(a->hidden) <= mf::kPanelLdsMaxBytes && a->rows <= mf::kPassRowsMax;
}

// The one-kernel tail: no unrestricted rows, not switched off, and every
// list within kShortPartsMax parts of a workgroup's stage of candidate rows
// (at most kShortListMax); a pack whose rows need more than one part each
// must fit two workgroups per compute unit of an MI355X (256 CUs), beyond
// which the gather's MFMA scores cost less than rescoring every candidate.
// The parts then shrink (to no fewer than 32 candidates) while the pack
// stays within two workgroups per compute unit: a compute unit moves only
// so many bytes per microsecond, and smaller parts spread the staging.  Fixed numbers, not the device's: the
// workspace layout must not depend on where it is sized.
constexpr uint64_t kShortPlanCUs = 256;
bool short_plan(const mf_decode_tail_args* a, uint32_t& per_part, uint32_t& parts) {
  if ((a->flags & MF_TAIL_NO_FUSED) || a->unrestricted_count > 0 || a->hidden % 8u != 0 ||
      a->hidden > 65535u) {
    return false;
  }
  const uint32_t cap = mf::short_stage_rows(static_cast<uint32_t>(a->hidden), mf::kShortListMax);
  if (cap == 0) return false;
  const uint64_t lists = a->max_count == 0 ? 1u : a->max_count;
  auto parts_of = [lists](uint64_t per) { return (lists + per - 1u) / per; };
  if (parts_of(cap) > mf::kShortPartsMax) return false;
  if (parts_of(cap) > 1u &&
      (a->rows * parts_of(cap) > 2u * kShortPlanCUs || a->rows > mf::kShortCountRows)) {
    return false;
  }
  uint64_t per = cap;
  while (per >= 64u && a->rows * parts_of(per / 2u) <= 2u * kShortPlanCUs &&
         parts_of(per / 2u) <= mf::kShortPartsMax) {
    per /= 2u;
  }
  per_part = static_cast<uint32_t>(per);
  parts = static_cast<uint32_t>(parts_of(per));
  return true;
}

// The dense head (mf_dense.hip): lists declared ascending, a hidden size of
// whole 32-feature steps wide enough that gathering a long list costs more
// than scoring its row against every token, and every row fitting the
// launch's panels (the compute units of each XCD, 256 slots each) and the
// row ranking's 32-bit keys.  Which
// rows it takes is decided on the device (dense_min_ids, dense_total_ids).
constexpr uint64_t kDenseMinHidden = 1024;
bool dense_head(const mf_decode_tail_args* a) {
  if (!(a->flags & MF_TAIL_SORTED_LISTS) || (a->flags & MF_TAIL_NO_DENSE) ||
      a->hidden % 32u != 0 || a->hidden < kDenseMinHidden) {
    return false;
  }
  // the row ranking packs (count, row) into 32 bits: rows < 2^13, lists < 2^19
  const uint64_t panels = device_cus() / 8u;
  return a->rows + a->unrestricted_count <= panels * mf::kDensePanelSlots && a->rows <= 8191u &&
         a->vocab < (1u << 19);
}
// A list the dense head may take: at least 1/256 of the vocabulary (and 64
// ids).  A panel of the dense head is added when its lists hold at least
// 5/2 of the vocabulary's ids: one panel's pass over the table and the
// gather of that many candidate rows take about the same time (both are
// bound by what each compute unit's memory pipeline moves, and both scale
// with the hidden size; measured at V = 128256, H = 2048: a panel pass
// 190 us, the gather 7.2 TB/s of candidate rows).
uint32_t dense_min_ids(uint64_t vocab) {
  const uint64_t m = vocab / 256u;
  return static_cast<uint32_t>(m > 64u ? m : 64u);
}
uint64_t dense_panel_ids(uint64_t vocab) { return vocab * 5u / 2u; }

// Validation common to both decode-tail entry points; fills the layout.
mf_status validate_tail(const mf_decode_tail_args* a, bool full, TailLayout& L) {
  if (a == nullptr) return status(MF_INVALID_ARGUMENT);
  if (a->rows == 0 || a->hidden == 0 || a->vocab == 0 || a->states == 0 ||
      (a->order != MF_ORDER_FMA_CHAIN && a->order != MF_ORDER_MUL_ADD_CHAIN) ||
      (a->norm_weight.address != 0 && (!std::isfinite(a->epsilon) || a->epsilon <= 0.0f))) {
    return status(MF_INVALID_ARGUMENT);
  }
  if (a->vocab > kU32Max || a->states >= kU32Max - 1 || a->nnz > kU32Max ||
      a->rows > kIntMax || a->unrestricted_count > a->rows) {
    return status(MF_RESOURCE_LIMIT);
  }
  // limits of this build: the hidden row is staged in LDS (H <= 8192), the
  // MFMA heads take K in chunks of 64 features, lists are at most the
  // vocabulary
  if (a->hidden > mf::kHeadMaxHidden || a->max_count > a->vocab ||
      ((a->unrestricted_count > 0 || full) && (a->hidden % 64u) != 0)) {
    return status(MF_RESOURCE_LIMIT);
  }
  uint64_t xe = 0, ee = 0, te = 0;
  if (!checked_mul(a->rows, a->hidden, xe) || !checked_mul(a->vocab, a->hidden, ee) ||
      !checked_mul(a->states, a->vocab, te) || xe > kU64Max / 4u || ee > kU64Max / 2u ||
      te > kU64Max / 4u) {
    return status(MF_ARITHMETIC_OVERFLOW);
  }
  // the state buffers: one entry per row, or a sequence table of any
  // capacity that row_sequence indexes
  const bool table = a->row_sequence.address != 0;
  if ((a->flags & ~static_cast<uint64_t>(MF_TAIL_HOLD_FINISHED | MF_TAIL_SORTED_LISTS |
                                         MF_TAIL_TABLE_PASS | MF_TAIL_NO_FUSED |
                                         MF_TAIL_NO_DENSE)) != 0) {
    return status(MF_INVALID_ARGUMENT);
  }
  if (table && (a->row_state.bytes / 4u > kU32Max || a->row_state.bytes == 0 ||
                (a->row_state.bytes % 4u) != 0 || !buffer_is(a->row_sequence, a->rows * 4u))) {
    return status(a->row_state.bytes / 4u > kU32Max ? MF_RESOURCE_LIMIT : MF_INVALID_ARGUMENT);
  }
  const uint64_t state_bytes = table ? a->row_state.bytes : a->rows * 4u;
  if (!buffer_is(a->x, xe * 4u) || !buffer_is(a->embedding, ee * 2u) ||
      !optional_is(a->norm_weight, a->hidden * 4u) || !buffer_is(a->row_state, state_bytes) ||
      !buffer_is(a->state_offsets, (a->states + 1) * 4u) ||
      !(a->nnz == 0 || buffer_is(a->state_tokens, a->nnz * 4u)) ||
      !optional_is(a->state_next, a->nnz * 4u) || !optional_is(a->next_table, te * 4u) ||
      (a->state_next.address != 0 && a->next_table.address != 0) ||
      !buffer_is(a->out_token, a->rows * 4u) || !optional_is(a->out_score, a->rows * 4u) ||
      !optional_is(a->out_next_state, state_bytes) ||
      (a->unrestricted_count > 0 &&
       !buffer_is(a->unrestricted_rows, a->unrestricted_count * 4u))) {
    return status(MF_INVALID_ARGUMENT);
  }
  // outputs must not alias each other or any input; with a sequence table the
  // next states may update the table in place
  const uintptr_t outs[3] = {a->out_token.address, a->out_score.address,
                             a->out_next_state.address};
  const uintptr_t ins[11] = {a->x.address, a->embedding.address, a->norm_weight.address,
                             a->row_state.address, a->state_offsets.address,
                             a->state_tokens.address, a->state_next.address,
                             a->next_table.address, a->unrestricted_rows.address,
                             a->workspace.address, a->row_sequence.address};
  for (int i = 0; i < 3; ++i) {
    if (outs[i] == 0) continue;
    for (int j = 0; j < 3; ++j) {
      if (j != i && outs[j] == outs[i]) return status(MF_INVALID_ARGUMENT);
    }
    for (uintptr_t in : ins) {
      const bool in_place = table && i == 2 && in == a->row_state.address &&
                            a->out_next_state.bytes == a->row_state.bytes;
      if (in != 0 && in == outs[i] && !in_place) return status(MF_INVALID_ARGUMENT);
    }
  }
  if ((a->embedding.address % 16u) != 0 || (a->x.address % 16u) != 0 ||
      (a->norm_weight.address % 16u) != 0) {
    return status(MF_INVALID_ARGUMENT);
  }
  const uint64_t rows = a->rows;
  if (full) {
    // unrestricted rows take the whole vocabulary as their list
    const uint64_t longest = a->max_count > a->vocab ? a->max_count : a->vocab;
    L.tile = kFullTile;
    L.max_tiles = static_cast<uint32_t>((longest + L.tile - 1) / L.tile);
  } else {
    L.tile = gather_tile(a->hidden, a->rows, a->max_count);
    L.max_tiles = static_cast<uint32_t>(a->max_count == 0 ? 1 : (a->max_count + L.tile - 1) / L.tile);
  }
  L.fb_tiles = mf::fallback_tiles(static_cast<uint32_t>(a->vocab));
  // table pass: one record per (row, 192-token range) holding its ids
  L.pass = !full && table_pass(a);
  L.fused = !full && !L.pass && short_plan(a, L.short_per_part, L.short_parts);
  L.dense = !full && !L.pass && !L.fused && dense_head(a);
  if (L.pass) {
    const uint64_t longest = a->max_count == 0 ? 1 : a->max_count;
    L.max_tiles = static_cast<uint32_t>(longest < L.fb_tiles ? longest : L.fb_tiles);
  }
  // the unplanned gather launches one workgroup per (row, tile)
  if (rows * L.max_tiles > kU32Max) return status(MF_RESOURCE_LIMIT);
  const uint64_t fb_rows = full ? 0 : a->unrestricted_count;
  L.fb_rows = static_cast<uint32_t>(fb_rows);
  // the dense head's slots: the unrestricted rows, then any row
  const uint64_t fb_slots = L.dense ? fb_rows + rows : fb_rows;
  const uint64_t panel_rows = L.dense ? 0u : fb_rows;
  uint64_t off = 0;
  auto take = [&off](uint64_t bytes) {
    const uint64_t at = off;
    off = align256(off + bytes);
    return at;
  };
  // the one-kernel tail's arrival counters: at the start of every layout,
  // which no other path writes, so they stay zero between calls whatever
  // the calls' shapes
  L.short_counts = take(mf::kShortCountRows * 4u);
  L.short_records = take(L.fused && L.short_parts > 1u
                             ? rows * L.short_parts * sizeof(mf::ShortPartRecord)
                             : 0u);
  L.y = take(xe * 4u);
  L.row_inv = take(rows * 4u);
  L.row_norm = take(rows * 4u);
  L.row_slack = take(rows * 4u);
  L.row_meta = take(rows * sizeof(mf::RowMeta));
  const bool split = full || mfma_gather(a->hidden);
  L.y_hi = take(split ? xe * 2u : 0u);
  L.y_lo = take(split ? xe * 2u : 0u);
  L.fb_map = take(rows * 4u);
  L.records = take(rows * L.max_tiles * sizeof(mf::TileRecord));
  L.fb_records = take(fb_slots * L.fb_tiles * sizeof(mf::TileRecord));
  L.fb_panel = take(mf::panel_tiles(static_cast<uint32_t>(panel_rows)) *
                    mf::panel_tile_bytes(a->hidden));
  L.fb_slot_row = take(panel_rows * 4u);
  L.fb_slot_norm = take(panel_rows * 4u);
  L.fb_slot_slack = take(panel_rows * 4u);
  L.scores = take(full ? rows * a->vocab * 4u : 0u);
  L.tok_norm = take(full ? a->vocab * 4u : 0u);
  L.range_index = take(L.pass ? L.fb_tiles * rows * 16u : 0u);
  L.row_tiles = take(L.pass ? rows * 4u : 0u);
  L.dense_spans = take(L.dense ? static_cast<uint64_t>(L.fb_tiles) * rows * 32u : 0u);
  L.dense_flag = take(L.dense ? rows * 4u : 0u);
  L.total = off;
  return ok();
}

mf_status check_workspace(const mf_decode_tail_args* a, const TailLayout& L) {
  if (a->workspace.address == 0 || a->workspace.bytes < L.total ||
      (a->workspace.address % 256u) != 0) {
    return status(MF_INVALID_ARGUMENT);
  }
  return ok();
}

enum class Stage { kPrepare, kRestricted, kUnrestricted, kFinalize };

// The norm's reference-order chains run in the gather launch (next to the
// MFMA gather, which scores z and does not need y) when the gather plans its
// tiles; otherwise in the norm kernel.
bool defer_chain(const mf_decode_tail_args* a) {
  return mfma_gather(a->hidden) && a->rows <= mf::kPlanRowsMax && a->norm_weight.address != 0 &&
         (a->hidden % 4u) == 0;
}

mf::TailNormArgs norm_args(const mf_decode_tail_args* a, const TailLayout& L, char* ws,
                           bool split, bool chain) {
  mf::TailNormArgs n{};
  n.rows = static_cast<uint32_t>(a->rows);
  n.x = ptr<const float>(a->x.address);
  n.weight = ptr<const float>(a->norm_weight.address);
  n.epsilon = a->epsilon;
  n.y = reinterpret_cast<float*>(ws + L.y);
  n.row_inv = reinterpret_cast<float*>(ws + L.row_inv);
  n.row_norm = reinterpret_cast<float*>(ws + L.row_norm);
  n.row_slack = reinterpret_cast<float*>(ws + L.row_slack);
  n.slack = underflow_slack(a->hidden);
  n.slack_scaled = scaled_slack(a->hidden);
  n.chain = chain ? 1u : 0u;
  n.y_hi = split ? reinterpret_cast<uint16_t*>(ws + L.y_hi) : nullptr;
  n.y_lo = split ? reinterpret_cast<uint16_t*>(ws + L.y_lo) : nullptr;
  n.row_state = ptr<const uint32_t>(a->row_state.address);
  n.offsets = ptr<const uint32_t>(a->state_offsets.address);
  n.states = static_cast<uint32_t>(a->states);
  n.nnz = static_cast<uint32_t>(a->nnz);
  n.max_count = static_cast<uint32_t>(a->max_count);
  n.V = static_cast<uint32_t>(a->vocab);
  n.H = static_cast<uint32_t>(a->hidden);
  n.row_meta = reinterpret_cast<mf::RowMeta*>(ws + L.row_meta);
  n.fb_map = reinterpret_cast<uint32_t*>(ws + L.fb_map);
  n.out_token = ptr<uint32_t>(a->out_token.address);
  n.out_score = ptr<float>(a->out_score.address);
  n.out_next = ptr<uint32_t>(a->out_next_state.address);
  n.row_sequence = ptr<const uint32_t>(a->row_sequence.address);
  n.capacity = static_cast<uint32_t>(n.row_sequence != nullptr ? a->row_state.bytes / 4u : a->rows);
  n.hold = (a->flags & MF_TAIL_HOLD_FINISHED) ? 1u : 0u;
  if (L.fb_rows > 0 && !L.dense) {  // the MFMA head's panel
    n.fb_rows = ptr<const uint32_t>(a->unrestricted_rows.address);
    n.fb_m = static_cast<uint32_t>(a->unrestricted_count);
    n.fb_panel = reinterpret_cast<uint16_t*>(ws + L.fb_panel);
    n.fb_slot_row = reinterpret_cast<uint32_t*>(ws + L.fb_slot_row);
    n.fb_slot_norm = reinterpret_cast<float*>(ws + L.fb_slot_norm);
    n.fb_slot_slack = reinterpret_cast<float*>(ws + L.fb_slot_slack);
  }
  if (L.pass) {  // the range index of the table pass
    n.tokens = ptr<const uint32_t>(a->state_tokens.address);
    n.range_index = reinterpret_cast<uint4*>(ws + L.range_index);
    n.row_tiles = reinterpret_cast<uint32_t*>(ws + L.row_tiles);
    n.ranges = L.fb_tiles;
    n.records = reinterpret_cast<mf::TileRecord*>(ws + L.records);
    n.max_recs = L.max_tiles;
  }
  if (L.dense) {  // the dense head's span index and row choice
    n.tokens = ptr<const uint32_t>(a->state_tokens.address);
    n.ranges = L.fb_tiles;
    n.dense_spans = reinterpret_cast<uint4*>(ws + L.dense_spans);
    n.dense_flag = reinterpret_cast<uint32_t*>(ws + L.dense_flag);
    n.dense_min = dense_min_ids(a->vocab);
    n.dense_fb = static_cast<uint32_t>(a->unrestricted_count);
    n.dense_sort = 1u;
    while (n.dense_sort < a->rows) n.dense_sort <<= 1;
    n.dense_panel_ids = dense_panel_ids(a->vocab);
  }
  return n;
}

mf::GatherArgs gather_args(const mf_decode_tail_args* a, const TailLayout& L, char* ws) {
  mf::GatherArgs g{};
  g.y = reinterpret_cast<const float*>(ws + L.y);
  g.emb = ptr<const uint16_t>(a->embedding.address);
  g.tokens = ptr<const uint32_t>(a->state_tokens.address);
  g.row_meta = reinterpret_cast<const mf::RowMeta*>(ws + L.row_meta);
  g.records = reinterpret_cast<mf::TileRecord*>(ws + L.records);
  g.rows = static_cast<uint32_t>(a->rows);
  g.H = static_cast<uint32_t>(a->hidden);
  g.V = static_cast<uint32_t>(a->vocab);
  g.tile = L.tile;
  g.max_tiles = L.max_tiles;
  g.slack = underflow_slack(a->hidden);
  // the MFMA gather and the comparator's lookup bound scores on z per row
  g.row_slack = reinterpret_cast<const float*>(ws + L.row_slack);
  // persistent workgroups: the launcher multiplies by the resident count
  g.groups = device_cus();
  return g;
}

mf::FinalizeArgs finalize_args(const mf_decode_tail_args* a, const TailLayout& L, char* ws,
                               bool full) {
  mf::FinalizeArgs f{};
  f.y = reinterpret_cast<const float*>(ws + L.y);
  // the MFMA gather, the MFMA head and the comparator's GEMMs score z
  f.row_inv = (full || mfma_gather(a->hidden)) ? reinterpret_cast<const float*>(ws + L.row_inv)
                                              : nullptr;
  f.emb = ptr<const uint16_t>(a->embedding.address);
  f.tokens = ptr<const uint32_t>(a->state_tokens.address);
  f.row_meta = reinterpret_cast<const mf::RowMeta*>(ws + L.row_meta);
  f.records = reinterpret_cast<const mf::TileRecord*>(ws + L.records);
  f.max_tiles = L.max_tiles;
  f.tile = L.tile;
  f.row_tiles = L.pass ? reinterpret_cast<const uint32_t*>(ws + L.row_tiles) : nullptr;
  if (!full && (a->unrestricted_count > 0 || L.dense)) {
    f.fb_records = reinterpret_cast<const mf::TileRecord*>(ws + L.fb_records);
    f.fb_map = reinterpret_cast<const uint32_t*>(ws + L.fb_map);
    f.fb_tiles = L.fb_tiles;
  }
  f.lookup_unrestricted = full ? 1 : 0;
  f.state_next = ptr<const uint32_t>(a->state_next.address);
  f.next_table = ptr<const int32_t>(a->next_table.address);
  f.out_token = ptr<uint32_t>(a->out_token.address);
  f.out_score = ptr<float>(a->out_score.address);
  f.out_next = ptr<uint32_t>(a->out_next_state.address);
  f.row_sequence = ptr<const uint32_t>(a->row_sequence.address);
  f.capacity = static_cast<uint32_t>(f.row_sequence != nullptr ? a->row_state.bytes / 4u : a->rows);
  f.rows = static_cast<uint32_t>(a->rows);
  f.H = static_cast<uint32_t>(a->hidden);
  f.V = static_cast<uint32_t>(a->vocab);
  f.order = a->order;
  return f;
}

mf::FallbackArgs fallback_args(const mf_decode_tail_args* a, const TailLayout& L, char* ws) {
  mf::FallbackArgs f{};
  f.panel = reinterpret_cast<const uint16_t*>(ws + L.fb_panel);
  f.slot_row = reinterpret_cast<const uint32_t*>(ws + L.fb_slot_row);
  f.slot_norm = reinterpret_cast<const float*>(ws + L.fb_slot_norm);
  f.slot_slack = reinterpret_cast<const float*>(ws + L.fb_slot_slack);
  f.m = static_cast<uint32_t>(a->unrestricted_count);
  f.emb = ptr<const uint16_t>(a->embedding.address);
  f.H = static_cast<uint32_t>(a->hidden);
  f.V = static_cast<uint32_t>(a->vocab);
  f.records = reinterpret_cast<mf::TileRecord*>(ws + L.fb_records);
  f.fb_map = reinterpret_cast<uint32_t*>(ws + L.fb_map);
  mfma_bound_coefs(a->hidden, f.coef, f.coef2);
  f.groups = device_cus();
  return f;
}

mf::DenseArgs dense_args(const mf_decode_tail_args* a, const TailLayout& L, char* ws) {
  mf::DenseArgs d{};
  d.emb = ptr<const uint16_t>(a->embedding.address);
  d.z_hi = reinterpret_cast<const uint16_t*>(ws + L.y_hi);
  d.row_norm = reinterpret_cast<const float*>(ws + L.row_norm);
  d.row_slack = reinterpret_cast<const float*>(ws + L.row_slack);
  d.row_meta = reinterpret_cast<const mf::RowMeta*>(ws + L.row_meta);
  d.spans = reinterpret_cast<const uint4*>(ws + L.dense_spans);
  d.fb_rows = ptr<const uint32_t>(a->unrestricted_rows.address);
  d.fb_m = static_cast<uint32_t>(a->unrestricted_count);
  d.rows = static_cast<uint32_t>(a->rows);
  d.H = static_cast<uint32_t>(a->hidden);
  d.V = static_cast<uint32_t>(a->vocab);
  d.ranges = L.fb_tiles;
  d.records = reinterpret_cast<mf::TileRecord*>(ws + L.fb_records);
  d.fb_map = reinterpret_cast<uint32_t*>(ws + L.fb_map);
  pass_bound_coefs(a->hidden, d.coef, d.coef2);
  d.groups = device_cus() / 8u * 8u;
  return d;
}

mf::PassArgs pass_args(const mf_decode_tail_args* a, const TailLayout& L, char* ws) {
  mf::PassArgs p{};
  p.head = fallback_args(a, L, ws);
  p.row_meta = reinterpret_cast<const mf::RowMeta*>(ws + L.row_meta);
  p.row_tiles = reinterpret_cast<const uint32_t*>(ws + L.row_tiles);
  p.range_index = reinterpret_cast<const uint4*>(ws + L.range_index);
  // the pass reads list entry 0 when a tile has no candidates; without lists
  // (nnz == 0) that read goes to a word of the workspace instead
  p.tokens = a->state_tokens.address != 0 ? ptr<const uint32_t>(a->state_tokens.address)
                                          : reinterpret_cast<const uint32_t*>(ws + L.row_tiles);
  p.z_hi = reinterpret_cast<const uint16_t*>(ws + L.y_hi);
  p.row_norm = reinterpret_cast<const float*>(ws + L.row_norm);
  p.row_slack = reinterpret_cast<const float*>(ws + L.row_slack);
  p.records = reinterpret_cast<mf::TileRecord*>(ws + L.records);
  p.max_recs = L.max_tiles;
  p.rows = static_cast<uint32_t>(a->rows);
  p.ranges = L.fb_tiles;
  pass_bound_coefs(a->hidden, p.coef, p.coef2);
  // the pass scores the unrestricted rows on the FP16 hi of z alone too, so
  // their windows take the hi-only coefficients (|z - hi| <= 2^-11 |z|), not
  // the hi + lo ones of the separate MFMA head
  p.head.coef = p.coef;
  p.head.coef2 = p.coef2;
  return p;
}

mf_status decode_tail_stage(const mf_decode_tail_args* args, uintptr_t stream, Stage stage) {
  if (stream == 0) return status(MF_INVALID_ARGUMENT);
  TailLayout L{};
  mf_status v = validate_tail(args, false, L);
  if (v.code != MF_OK) return v;
  v = check_workspace(args, L);
  if (v.code != MF_OK) return v;
  const mf_decode_tail_args* a = args;
  char* ws = ptr<char>(a->workspace.address);
  const hipStream_t s = native(stream);
  hipError_t e = hipSuccess;
  switch (stage) {
    case Stage::kPrepare:
      if (L.fused) {
        mf::ShortSplit sp{};
        sp.records = reinterpret_cast<mf::ShortPartRecord*>(ws + L.short_records);
        sp.counts = reinterpret_cast<uint32_t*>(ws + L.short_counts);
        sp.per_part = L.short_per_part;
        sp.parts = L.short_parts;
        e = mf::launch_short(norm_args(a, L, ws, false, true), finalize_args(a, L, ws, false), sp,
                             s);
        break;
      }
      e = mf::launch_tail_norm(
          norm_args(a, L, ws, mfma_gather(a->hidden), L.pass || !defer_chain(a)), s);
      break;
    case Stage::kRestricted: {
      if (L.fused) break;
      if (L.pass) {
        e = mf::launch_pass(pass_args(a, L, ws), s);
        break;
      }
      mf::GatherArgs g = gather_args(a, L, ws);
      if (mfma_gather(a->hidden)) {
        g.y_hi = reinterpret_cast<const uint16_t*>(ws + L.y_hi);
        g.y_lo = reinterpret_cast<const uint16_t*>(ws + L.y_lo);
        g.row_norm = reinterpret_cast<const float*>(ws + L.row_norm);
        mfma_bound_coefs(a->hidden, g.coef, g.coef2);
        if (defer_chain(a)) {
          g.x = ptr<const float>(a->x.address);
          g.weight = ptr<const float>(a->norm_weight.address);
          g.epsilon = a->epsilon;
          g.y_out = reinterpret_cast<float*>(ws + L.y);
          g.inv_out = reinterpret_cast<float*>(ws + L.row_inv);
          g.chain_rows = static_cast<uint32_t>(a->rows);
        }
        e = mf::launch_gather_mfma(g, s);
      } else {
        g.coef = dot_bound_coef(a->hidden);
        e = mf::launch_gather(ScoreSource::kDotF32, g, s);
      }
      break;
    }
    case Stage::kUnrestricted: {
      if (L.dense) {
        e = mf::launch_dense(dense_args(a, L, ws), s);
        break;
      }
      if (a->unrestricted_count == 0 || L.pass || L.fused) break;
      e = mf::launch_fallback(fallback_args(a, L, ws), s);
      break;
    }
    case Stage::kFinalize:
      if (L.fused) break;
      e = mf::launch_finalize(finalize_args(a, L, ws, false), s);
      break;
  }
  return launch_status(e);
}

}  // namespace

mf_status mf_decode_tail_workspace_bytes(const mf_decode_tail_args* args, uint64_t* bytes) {
  if (bytes == nullptr) return status(MF_INVALID_ARGUMENT);
  TailLayout L{};
  const mf_status v = validate_tail(args, false, L);
  if (v.code != MF_OK) return v;
  *bytes = L.total;
  return ok();
}

mf_status mf_decode_tail_path(const mf_decode_tail_args* args, uint32_t* path) {
  if (path == nullptr) return status(MF_INVALID_ARGUMENT);
  TailLayout L{};
  const mf_status v = validate_tail(args, false, L);
  if (v.code != MF_OK) return v;
  *path = L.pass    ? MF_TAIL_PATH_TABLE_PASS
          : L.fused ? MF_TAIL_PATH_FUSED
          : L.dense ? MF_TAIL_PATH_DENSE
                    : MF_TAIL_PATH_GATHER;
  return ok();
}

mf_status mf_decode_tail_full_workspace_bytes(const mf_decode_tail_args* args, uint64_t* bytes) {
  if (bytes == nullptr) return status(MF_INVALID_ARGUMENT);
  TailLayout L{};
  const mf_status v = validate_tail(args, true, L);
  if (v.code != MF_OK) return v;
  *bytes = L.total;
  return ok();
}

mf_status mf_workspace_init(mf_buffer workspace, uintptr_t stream) {
  if (workspace.address == 0 || stream == 0 || (workspace.address % 16u) != 0) {
    return status(MF_INVALID_ARGUMENT);
  }
  return launch_status(mf::launch_fill_zero(ptr<void>(workspace.address),
                                            workspace.bytes & ~uint64_t{15u}, native(stream)));
}

mf_status mf_read_floor(mf_buffer data, mf_buffer sink, uintptr_t stream) {
  if (data.address == 0 || stream == 0 || (data.address % 16u) != 0 || sink.address == 0 ||
      sink.bytes < 4u || (sink.address % 4u) != 0) {
    return status(MF_INVALID_ARGUMENT);
  }
  return launch_status(mf::launch_read_floor(ptr<const void>(data.address), data.bytes & ~uint64_t{15u},
                                             ptr<uint32_t>(sink.address), native(stream)));
}

mf_status mf_decode_tail_prepare(const mf_decode_tail_args* args, uintptr_t stream) {
  return decode_tail_stage(args, stream, Stage::kPrepare);
}

mf_status mf_decode_tail_restricted(const mf_decode_tail_args* args, uintptr_t stream) {
  return decode_tail_stage(args, stream, Stage::kRestricted);
}

mf_status mf_decode_tail_unrestricted(const mf_decode_tail_args* args, uintptr_t stream) {
  return decode_tail_stage(args, stream, Stage::kUnrestricted);
}

mf_status mf_decode_tail_finalize(const mf_decode_tail_args* args, uintptr_t stream) {
  return decode_tail_stage(args, stream, Stage::kFinalize);
}

// The MFMA head runs before the gather: it streams the whole table in
// order, and the gather's row lookups then find most rows in the
// last-level cache.
mf_status mf_decode_tail_f16(const mf_decode_tail_args* args, uintptr_t stream) {
  for (Stage st : {Stage::kPrepare, Stage::kUnrestricted, Stage::kRestricted, Stage::kFinalize}) {
    const mf_status v = decode_tail_stage(args, stream, st);
    if (v.code != MF_OK) return v;
  }
  return ok();
}

}  // extern "C"

// ------------------------------------------- decode tail without allocation --

namespace {

// The workspace of mf_decode_tail_f16_noalloc: one array per GPU, held from
// module load to process end.  Host code never passes the array's name to a
// kernel or a copy (on the host it is a stand-in, not a device address): it
// takes the device address from hipGetSymbolAddress, once per device.
constexpr uint64_t kScratchBytes = 16ull << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct ScratchSlot {
  std::mutex lock;
  bool ready = false;
  void* address = nullptr;
};
ScratchSlot g_scratch[64];

// The current device's array: its address, looked up with that device
// current on the first successful call there, when the array is also
// zero-filled on the caller's stream (the state every workspace starts
// from).  Only success is latched: a call that fails here (a bad stream, a
// failed lookup) leaves the next call to try again.  A stream under graph
// capture cannot carry that first fill (it would become a graph node that
// eager calls made before a replay never see), so a first call under
// capture is refused with hipErrorStreamCaptureUnsupported.
hipError_t scratch_address(hipStream_t stream, void** out) {
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  ScratchSlot& slot = g_scratch[dev];
  std::lock_guard<std::mutex> guard(slot.lock);
  if (!slot.ready) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &capture);
    if (e != hipSuccess) return e;
    if (capture != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p == nullptr) e = hipErrorInvalidSymbol;
    if (e == hipSuccess) e = mf::launch_fill_zero(p, kScratchBytes, stream);
    if (e != hipSuccess) return e;
    slot.address = p;
    slot.ready = true;
  }
  *out = slot.address;
  return hipSuccess;
}

}  // namespace

extern "C" {

uint64_t mf_decode_tail_noalloc_max_bytes(void) { return kScratchBytes; }

mf_status mf_decode_tail_f16_noalloc(const mf_decode_tail_args* args, uintptr_t stream) {
  if (args == nullptr || stream == 0) return status(MF_INVALID_ARGUMENT);
  mf_decode_tail_args a = *args;
  a.workspace = mf_buffer{0, 0};  // the caller's workspace field is not used
  TailLayout L{};
  mf_status v = validate_tail(&a, false, L);
  if (v.code != MF_OK) return v;
  if (L.total > kScratchBytes) return status(MF_RESOURCE_LIMIT);
  void* base = nullptr;
  const hipError_t e = scratch_address(native(stream), &base);
  if (e != hipSuccess) return runtime_status(e);
  a.workspace = mf_buffer{reinterpret_cast<uintptr_t>(base), kScratchBytes};
  for (Stage st : {Stage::kPrepare, Stage::kUnrestricted, Stage::kRestricted, Stage::kFinalize}) {
    v = decode_tail_stage(&a, stream, st);
    if (v.code != MF_OK) return v;
  }
  return ok();
}

mf_status mf_decode_tail_full_f16(const mf_decode_tail_args* args, uintptr_t stream) {
  if (stream == 0) return status(MF_INVALID_ARGUMENT);
  TailLayout L{};
  mf_status v = validate_tail(args, true, L);
  if (v.code != MF_OK) return v;
  v = check_workspace(args, L);
  if (v.code != MF_OK) return v;
  const mf_decode_tail_args* a = args;
  char* ws = ptr<char>(a->workspace.address);
  const hipStream_t s = native(stream);
  float* scores = reinterpret_cast<float*>(ws + L.scores);
  float* tok_norm = reinterpret_cast<float*>(ws + L.tok_norm);

  // 1. final RMSNorm (and its FP16 split for the MFMA projection)
  hipError_t e = mf::launch_tail_norm(norm_args(a, L, ws, true, true), s);
  if (e != hipSuccess) return launch_status(e);
  // 2. full output projection of every row: FP32 scores [rows, V] of z's
  // FP16 hi on the MFMA projection kernel (the hand-written replacement of
  // the reference's library GEMM, linear.cu:92-102), and the token norm
  // bounds the exact selection needs
  {
    mf::ProjArgs pj{};
    pj.a16 = reinterpret_cast<const uint16_t*>(ws + L.y_hi);
    pj.m = static_cast<uint32_t>(a->rows);
    pj.emb = ptr<const uint16_t>(a->embedding.address);
    pj.H = static_cast<uint32_t>(a->hidden);
    pj.V = static_cast<uint32_t>(a->vocab);
    pj.out_f32 = scores;
    pj.tok_norm = tok_norm;
    e = mf::launch_projection(pj, s);
    if (e != hipSuccess) return launch_status(e);
  }
  // 3. restricted selection over the scores (unrestricted rows: every id),
  // windows from the bound of a score on the FP16 hi alone
  mf::GatherArgs g = gather_args(a, L, ws);
  g.scores = scores;
  g.row_norm = reinterpret_cast<const float*>(ws + L.row_norm);
  g.tok_norm = tok_norm;
  pass_bound_coefs(a->hidden, g.coef, g.coef2);
  g.groups = device_cus();
  e = mf::launch_gather(ScoreSource::kLookup, g, s);
  if (e != hipSuccess) return launch_status(e);
  // 4. merge, reference-order rescore, DFA advance
  e = mf::launch_finalize(finalize_args(a, L, ws, true), s);
  return launch_status(e);
}

}  // extern "C"
