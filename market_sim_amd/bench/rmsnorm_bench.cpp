// rmsnorm_bench -- the reference's RMSNorm benchmark
// (src/tools/cuda_rmsnorm_bench.cu), run on MI355X through the C++ operator
// layer (include/marketforge_gpu.hpp).
//
// Kept like the reference so the figures compare with it:
//   * rms_norm_f32 at hidden 576 (SmolLM2-135M), epsilon 1e-5 (bench.cu:84-89);
//   * input[i] = ((i % 29) - 14) / 16, weight[i] = 0.75 + (i % 13) / 32
//     (:55-63);
//   * the cases rows in {1, 16, 256, 1024} with 2000 / 1000 / 500 / 200
//     timed iterations (:141-146), 20 untimed launches and a sync before one
//     event pair (:84-127);
//   * logical bytes = 2 * rows * hidden * 4 + hidden * 4 (:129-131), as GiB/s;
//   * one JSON line in the reference's fields (:155-175).
// Added: each case's output is checked bit for bit against the reference's
// CPU order on the host (src/cpu/operators.cpp:523-535: squares summed in
// order, 1 / sqrt(sum / H + eps), then (x * inv) * w); a mismatch is
// reported on stderr and the program exits with status 3 (the document
// keeps exactly the reference's fields, tools/modal/vllm_modal_app.py:311-318).
//
// Usage: rmsnorm_bench [--iterations-divisor N] (N > 1 shortens every case).
#include <array>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "bench_util.hpp"

namespace {

namespace mg = marketforge::gpu;
using bench::status_ok;

constexpr std::uint64_t kHidden = 576;

struct Case {
  std::uint64_t rows;
  std::uint32_t iterations;
};

struct Result {
  std::uint64_t rows = 0;
  std::uint32_t iterations = 0;
  double average_us = 0.0;
  double gib_per_second = 0.0;
  bool parity = false;
};

// the reference CPU order (compiled without FMA contraction: every product
// and sum rounds on its own)
void host_norm(const std::vector<float>& x, const std::vector<float>& w, std::uint64_t rows,
               std::vector<float>& y) {
  for (std::uint64_t r = 0; r < rows; ++r) {
    volatile float sum = 0.0f;
    for (std::uint64_t c = 0; c < kHidden; ++c) {
      const volatile float v = x[r * kHidden + c];
      const volatile float sq = v * v;
      sum = sum + sq;
    }
    const volatile float mean = sum / static_cast<float>(kHidden);
    const volatile float inv = 1.0f / std::sqrt(mean + 1.0e-5f);
    for (std::uint64_t c = 0; c < kHidden; ++c) {
      const volatile float scaled = x[r * kHidden + c] * inv;
      y[r * kHidden + c] = scaled * w[c];
    }
  }
}

bool run_case(const Case c, Result& out) {
  const std::uint64_t n = c.rows * kHidden;
  std::vector<float> x(n), w(kHidden), y(n), want(n);
  for (std::uint64_t i = 0; i < n; ++i) {
    x[i] = static_cast<float>(static_cast<std::int32_t>(i % 29) - 14) * 0.0625f;
  }
  for (std::uint64_t i = 0; i < kHidden; ++i) w[i] = 0.75f + static_cast<float>(i % 13) * 0.03125f;
  host_norm(x, w, c.rows, want);
  auto stream_r = mg::GpuStream::create();
  if (!stream_r) return false;
  mg::GpuStream stream = std::move(stream_r).value();
  auto d_x = bench::upload(x, stream);
  auto d_w = bench::upload(w, stream);
  auto d_y = mg::DeviceBuffer::allocate(n * 4);
  if (!d_x || !d_w || !d_y) return false;
  auto launch = [&]() {
    return status_ok(mg::rms_norm_f32(d_x.value(), d_w.value(), d_y.value(), c.rows, kHidden,
                                      1.0e-5f, stream.handle()),
                     "rms_norm_f32");
  };
  if (!launch()) return false;
  if (!bench::download(y, d_y.value(), stream)) return false;
  const double us = bench::time_launches(stream, 20, c.iterations, launch);
  if (us <= 0.0) return false;
  const double logical = static_cast<double>(n * 4u * 2u + kHidden * 4u);
  out.rows = c.rows;
  out.iterations = c.iterations;
  out.average_us = us;
  out.gib_per_second = logical / (us * 1e-6) / static_cast<double>(1ull << 30);
  out.parity = std::memcmp(y.data(), want.data(), n * 4) == 0;
  return true;
}

}  // namespace

int main(int argc, char** argv) {
  std::uint32_t divisor = 1;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--iterations-divisor" && i + 1 < argc) {
      divisor = static_cast<std::uint32_t>(std::strtoul(argv[++i], nullptr, 10));
    } else {
      std::fprintf(stderr, "usage: %s [--iterations-divisor N]\n", argv[0]);
      return 2;
    }
  }
  if (divisor == 0) return 2;
  constexpr std::array<Case, 4> cases{{{1, 2'000}, {16, 1'000}, {256, 500}, {1'024, 200}}};
  std::array<Result, cases.size()> res{};
  for (std::size_t i = 0; i < cases.size(); ++i) {
    Case c = cases[i];
    c.iterations = c.iterations / divisor > 0 ? c.iterations / divisor : 1;
    if (!run_case(c, res[i])) return 1;
  }
  std::printf("{\"schema_version\":1,\"result\":\"pass\",\"operator\":\"rms_norm_f32\","
              "\"model_shape\":\"SmolLM2-135M hidden_size=576\",");
  bench::print_gpu(stdout);
  std::printf(",\"measurements\":[");
  for (std::size_t i = 0; i < res.size(); ++i) {
    std::printf("%s{\"rows\":%llu,\"hidden_size\":%llu,\"iterations\":%u,"
                "\"average_microseconds\":%.3f,\"logical_gib_per_second\":%.3f}",
                i ? "," : "", static_cast<unsigned long long>(res[i].rows),
                static_cast<unsigned long long>(kHidden), res[i].iterations, res[i].average_us,
                res[i].gib_per_second);
  }
  std::printf("]}\n");
  for (const auto& r : res) {
    if (!r.parity) {
      std::fprintf(stderr, "output differs from the reference order at %llu rows\n",
                   static_cast<unsigned long long>(r.rows));
      return 3;
    }
  }
  return 0;
}
