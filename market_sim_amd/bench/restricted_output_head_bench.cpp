// restricted_output_head_bench -- the reference's restricted output-head
// benchmark (src/tools/cuda_restricted_output_head_bench.cu), run on MI355X
// through the C++ operator layer (include/marketforge_gpu.hpp).
//
// Kept identical to the reference so the numbers compare cell by cell with
// its published L4 table (BENCHMARKS.md:33-44):
//   * shape H = 576, V = 49,152 (SmolLM2-135M);
//   * the 12 cases rows x allowed in {1, 16, 256} x {2, 8, 32, 128} with
//     500 / 300 / 100 timed iterations (bench.cu:278-291);
//   * inputs: table E[t][f] = fp16((t % 101) / 64 + (f % 7) / 256)
//     (bench.cu:250-258), hidden fp16(0.5 + (i % 13) / 32) (:129-132),
//     allowed id (row * 131 + j * 977 + 17) % V with every count = allowed
//     (:133-140);
//   * "full" = linear_f16 (FP16 logits) + restricted_greedy_select_f16,
//     "restricted" = restricted_output_head_f16 (:181-198), token parity
//     checked before timing (:199-213);
//   * timing: 10 untimed launches, a stream sync, then one event pair
//     around `iterations` back-to-back launches (:61-109);
//   * output: one JSON line in the reference schema (:300-330), validated by
//     tools/modal/vllm_modal_app.py:459-516 apart from the GPU identity.
//
// Usage: restricted_output_head_bench [--iterations-divisor N]
// (N > 1 shortens every case, for tests; the published protocol is N = 1).
#include <hip/hip_runtime_api.h>

#include <array>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "marketforge_gpu.hpp"

namespace {

namespace mg = marketforge::gpu;

constexpr std::uint64_t kHidden = 576;
constexpr std::uint64_t kVocab = 49'152;

struct Case {
  std::uint64_t rows;
  std::uint64_t allowed;
  std::uint32_t iterations;
};

struct Cell {
  Case c;
  double full_us = 0.0;
  double restricted_us = 0.0;
  bool parity = false;
};

// float -> binary16, round to nearest even (IEEE 754 conversion; values here
// are normal and far inside the half range, but the general case is kept).
std::uint16_t to_half(float value) {
  std::uint32_t x;
  std::memcpy(&x, &value, 4);
  const std::uint32_t sign = (x >> 16) & 0x8000u;
  const std::uint32_t mag = x & 0x7FFFFFFFu;
  if (mag >= 0x7F800000u) {  // inf / nan
    return static_cast<std::uint16_t>(sign | 0x7C00u | (mag > 0x7F800000u ? 0x200u : 0u));
  }
  if (mag >= 0x477FF000u) return static_cast<std::uint16_t>(sign | 0x7C00u);  // rounds to inf
  if (mag < 0x38800000u) {  // half subnormal or zero: scale by 2^24 and round
    const float scaled = std::fabs(value) * 16777216.0f;  // exact (power of two)
    const float r = std::nearbyint(scaled);                // ties to even
    return static_cast<std::uint16_t>(sign | static_cast<std::uint32_t>(r));
  }
  const std::uint32_t exp = (mag >> 23) - 112u;  // rebias 127 -> 15
  std::uint32_t m = mag & 0x7FFFFFu;
  std::uint32_t h = (exp << 10) | (m >> 13);
  const std::uint32_t rest = m & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;  // carries into the exponent
  return static_cast<std::uint16_t>(sign | h);
}

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return false;
}

bool status_ok(const mg::Status& s, const char* what) {
  if (s.ok()) return true;
  std::fprintf(stderr, "%s: error code %u detail %u\n", what,
               static_cast<unsigned>(s.code), s.detail);
  return false;
}

// 10 warm-up launches, sync, then events around `iterations` launches;
// returns the average microseconds per launch (negative on failure).
template <typename Launch>
double time_launches(const mg::GpuStream& stream, std::uint32_t iterations, Launch launch) {
  for (int i = 0; i < 10; ++i)
    if (!launch()) return -1.0;
  if (!status_ok(stream.synchronize(), "synchronize")) return -1.0;
  hipEvent_t start = nullptr, stop = nullptr;
  if (!hip_ok(hipEventCreate(&start), "hipEventCreate") ||
      !hip_ok(hipEventCreate(&stop), "hipEventCreate"))
    return -1.0;
  const auto s = reinterpret_cast<hipStream_t>(stream.handle().value);
  bool ok = hip_ok(hipEventRecord(start, s), "hipEventRecord");
  for (std::uint32_t i = 0; ok && i < iterations; ++i) ok = launch();
  ok = ok && hip_ok(hipEventRecord(stop, s), "hipEventRecord") &&
       hip_ok(hipEventSynchronize(stop), "hipEventSynchronize");
  float ms = 0.0f;
  ok = ok && hip_ok(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
  (void)hipEventDestroy(start);
  (void)hipEventDestroy(stop);
  if (!ok || ms <= 0.0f) return -1.0;
  return static_cast<double>(ms) * 1000.0 / static_cast<double>(iterations);
}

template <typename T>
mg::Result<mg::DeviceBuffer> upload(const std::vector<T>& host, const mg::GpuStream& stream) {
  auto b = mg::DeviceBuffer::allocate(host.size() * sizeof(T));
  if (!b) return b;
  const auto s = b.value().copy_from_host_async(host.data(), host.size() * sizeof(T), 0,
                                                stream.handle());
  if (!s.ok()) return mg::Result<mg::DeviceBuffer>::failure(s);
  return b;
}

bool run_cell(Cell& cell, const mg::GpuStream& stream, mg::BlasHandle& blas,
              const mg::DeviceBuffer& table) {
  const Case c = cell.c;
  std::vector<std::uint16_t> hidden(c.rows * kHidden);
  for (std::size_t i = 0; i < hidden.size(); ++i)
    hidden[i] = to_half(0.5f + static_cast<float>(i % 13u) / 32.0f);
  std::vector<std::uint32_t> allowed(c.rows * c.allowed);
  for (std::uint64_t r = 0; r < c.rows; ++r)
    for (std::uint64_t j = 0; j < c.allowed; ++j)
      allowed[r * c.allowed + j] = static_cast<std::uint32_t>((r * 131u + j * 977u + 17u) % kVocab);
  const std::vector<std::uint32_t> counts(c.rows, static_cast<std::uint32_t>(c.allowed));

  auto hid = upload(hidden, stream);
  auto ids = upload(allowed, stream);
  auto cnt = upload(counts, stream);
  auto logits = mg::DeviceBuffer::allocate(c.rows * kVocab * 2);
  auto full_tok = mg::DeviceBuffer::allocate(c.rows * 4);
  auto head_tok = mg::DeviceBuffer::allocate(c.rows * 4);
  if (!hid || !ids || !cnt || !logits || !full_tok || !head_tok) {
    std::fprintf(stderr, "allocation or upload failed\n");
    return false;
  }
  auto full = [&]() {
    return status_ok(mg::linear_f16(hid.value(), table, logits.value(), c.rows, kHidden, kVocab,
                                    blas, stream.handle()),
                     "linear_f16") &&
           status_ok(mg::restricted_greedy_select_f16(logits.value(), ids.value(), cnt.value(),
                                                      full_tok.value(), c.rows, kVocab, c.allowed,
                                                      stream.handle()),
                     "restricted_greedy_select_f16");
  };
  auto restricted = [&]() {
    return status_ok(mg::restricted_output_head_f16(hid.value(), table, ids.value(), cnt.value(),
                                                    head_tok.value(), c.rows, kHidden, kVocab,
                                                    c.allowed, stream.handle()),
                     "restricted_output_head_f16");
  };
  std::vector<std::uint32_t> a(c.rows), b(c.rows);
  if (!full() || !restricted() ||
      !status_ok(full_tok.value().copy_to_host_async(a.data(), c.rows * 4, 0, stream.handle()),
                 "copy") ||
      !status_ok(head_tok.value().copy_to_host_async(b.data(), c.rows * 4, 0, stream.handle()),
                 "copy") ||
      !status_ok(stream.synchronize(), "synchronize"))
    return false;
  cell.parity = (a == b);
  if (!cell.parity) {
    std::fprintf(stderr, "token mismatch: rows %llu allowed %llu\n",
                 static_cast<unsigned long long>(c.rows),
                 static_cast<unsigned long long>(c.allowed));
    return false;
  }
  cell.full_us = time_launches(stream, c.iterations, full);
  cell.restricted_us = time_launches(stream, c.iterations, restricted);
  return cell.full_us > 0.0 && cell.restricted_us > 0.0;
}

}  // namespace

int main(int argc, char** argv) {
  std::uint32_t divisor = 1;
  for (int i = 1; i < argc; ++i) {
    if (std::strcmp(argv[i], "--iterations-divisor") == 0 && i + 1 < argc) {
      divisor = static_cast<std::uint32_t>(std::strtoul(argv[++i], nullptr, 10));
    } else {
      std::fprintf(stderr, "usage: %s [--iterations-divisor N]\n", argv[0]);
      return 2;
    }
  }
  if (divisor == 0) divisor = 1;
  int devices = 0;
  if (!hip_ok(hipGetDeviceCount(&devices), "hipGetDeviceCount") || devices < 1) return 1;
  hipDeviceProp_t prop{};
  if (!hip_ok(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties")) return 1;

  std::vector<std::uint16_t> host_table(kVocab * kHidden);
  for (std::uint64_t t = 0; t < kVocab; ++t) {
    const float base = static_cast<float>(t % 101u) / 64.0f;
    for (std::uint64_t f = 0; f < kHidden; ++f)
      host_table[t * kHidden + f] = to_half(base + static_cast<float>(f % 7u) / 256.0f);
  }
  auto stream = mg::GpuStream::create();
  auto blas = mg::BlasHandle::create();
  if (!stream || !blas) return 1;
  auto table = upload(host_table, stream.value());
  if (!table || !status_ok(stream.value().synchronize(), "synchronize")) return 1;

  const std::array<Case, 12> cases{{{1, 2, 500},   {1, 8, 500},    {1, 32, 500},  {1, 128, 500},
                                    {16, 2, 300},  {16, 8, 300},   {16, 32, 300}, {16, 128, 300},
                                    {256, 2, 100}, {256, 8, 100}, {256, 32, 100}, {256, 128, 100}}};
  std::vector<Cell> cells;
  for (Case c : cases) {
    c.iterations = c.iterations / divisor > 0 ? c.iterations / divisor : 1;
    Cell cell{c};
    if (!run_cell(cell, stream.value(), blas.value(), table.value())) return 1;
    cells.push_back(cell);
  }

  // the marketing name can be empty (no device-id table on the host); the
  // architecture name then identifies the GPU
  std::string name = prop.name;
  if (name.empty()) {
    std::string arch = prop.gcnArchName;
    name = "AMD " + arch.substr(0, arch.find(':'));
  }

  std::string out;
  char buf[512];
  std::snprintf(buf, sizeof buf,
                "{\"schema_version\":1,\"result\":\"pass\",\"operator\":\"restricted_output_head_f16\","
                "\"model_shape\":\"SmolLM2-135M\",\"hidden_size\":%llu,\"vocabulary_size\":%llu,"
                "\"gpu\":{\"name\":\"%s\",\"compute_capability\":\"%d.%d\"},\"measurements\":[",
                static_cast<unsigned long long>(kHidden), static_cast<unsigned long long>(kVocab),
                name.c_str(), prop.major, prop.minor);
  out += buf;
  for (std::size_t i = 0; i < cells.size(); ++i) {
    const Cell& m = cells[i];
    std::snprintf(buf, sizeof buf,
                  "%s{\"rows\":%llu,\"allowed_tokens_per_row\":%llu,\"iterations\":%u,"
                  "\"full_average_microseconds\":%.3f,\"restricted_average_microseconds\":%.3f,"
                  "\"speedup\":%.3f,\"full_scores\":%llu,\"restricted_scores\":%llu,"
                  "\"materialized_logit_bytes_avoided\":%llu,\"exact_token_parity\":%s}",
                  i ? "," : "", static_cast<unsigned long long>(m.c.rows),
                  static_cast<unsigned long long>(m.c.allowed), m.c.iterations, m.full_us,
                  m.restricted_us, m.full_us / m.restricted_us,
                  static_cast<unsigned long long>(m.c.rows * kVocab),
                  static_cast<unsigned long long>(m.c.rows * m.c.allowed),
                  static_cast<unsigned long long>(m.c.rows * kVocab * 2),
                  m.parity ? "true" : "false");
    out += buf;
  }
  out += "]}";
  std::printf("%s\n", out.c_str());
  return 0;
}
