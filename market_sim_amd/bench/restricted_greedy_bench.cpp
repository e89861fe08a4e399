// restricted_greedy_bench -- the reference's restricted-greedy benchmark
// (src/tools/cuda_restricted_greedy_bench.cu), run on MI355X through the C++
// operator layer (include/marketforge_gpu.hpp).
//
// Kept like the reference so the figures compare with it:
//   * the allowed sets are the SmolLM2 market-action grammar's non-empty
//     states in state order (bench.cu:108-131), row r taking state
//     r * states / rows (:147-149), as a fixed-width table of the longest
//     set padded with MF_INVALID_TOKEN (:141-144);
//   * FP16 logits [rows, 49152] at -4, the allowed tokens at
//     (token * 13 + row) % 41 (:141-156);
//   * the cases rows in {1, 16, 256} with 2000 / 1000 / 500 timed
//     iterations (:253-257), 20 untimed launches and a sync before one event
//     pair (:62-104);
//   * logical bytes = allowed * (2 + 4) + rows * 8 (:208-214), reported as
//     GiB/s, and sequences per second;
//   * one JSON line in the reference's fields (:262-296).
// Added: each case's tokens are checked against the host selection (lowest
// id among the maximal logits of the row's set) before timing; a mismatch
// is reported on stderr and the program exits with status 3 (the document
// keeps exactly the reference's fields, which its validator requires,
// tools/modal/vllm_modal_app.py:359-420).
//
// Usage: restricted_greedy_bench --dfa FILE [--iterations-divisor N]
// FILE is the DFA table of market_sim_amd.dfa.write_tables (the market
// grammar: tests/golden/market_dfa.npz); N > 1 shortens every case.
#include <algorithm>
#include <array>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "bench_util.hpp"

namespace {

namespace mg = marketforge::gpu;
using bench::status_ok;

constexpr std::uint64_t kVocab = 49'152;

struct Case {
  std::uint64_t rows;
  std::uint32_t iterations;
};

struct Measurement {
  std::uint64_t rows = 0;
  std::uint64_t total_allowed = 0;
  std::uint32_t iterations = 0;
  double average_us = 0.0;
  double sequences_per_second = 0.0;
  double candidate_gib_per_second = 0.0;
  bool parity = false;
};

bool run_case(const Case c, const std::vector<std::vector<std::uint32_t>>& sets,
              std::size_t max_allowed, Measurement& out) {
  const std::uint64_t rows = c.rows;
  std::vector<std::uint16_t> logits(rows * kVocab, bench::to_half(-4.0f));
  std::vector<std::uint32_t> allowed(rows * max_allowed, mg::restricted_greedy_invalid_token_id);
  std::vector<std::uint32_t> counts(rows);
  std::vector<std::uint32_t> expect(rows);
  std::uint64_t total = 0;
  for (std::uint64_t r = 0; r < rows; ++r) {
    const auto& set = sets[r * sets.size() / rows];
    counts[r] = static_cast<std::uint32_t>(set.size());
    total += set.size();
    std::uint32_t best = mg::restricted_greedy_invalid_token_id;
    float best_v = 0.0f;
    for (std::size_t i = 0; i < set.size(); ++i) {
      const std::uint32_t t = set[i];
      allowed[r * max_allowed + i] = t;
      const float v = static_cast<float>((t * 13u + static_cast<std::uint32_t>(r)) % 41u);
      logits[r * kVocab + t] = bench::to_half(v);
      if (best == mg::restricted_greedy_invalid_token_id || v > best_v || (v == best_v && t < best)) {
        best = t;
        best_v = v;
      }
    }
    expect[r] = best;
  }
  auto stream_r = mg::GpuStream::create();
  if (!stream_r) return false;
  mg::GpuStream stream = std::move(stream_r).value();
  auto d_logits = bench::upload(logits, stream);
  auto d_allowed = bench::upload(allowed, stream);
  auto d_counts = bench::upload(counts, stream);
  auto d_out = mg::DeviceBuffer::allocate(rows * 4);
  if (!d_logits || !d_allowed || !d_counts || !d_out) return false;
  auto launch = [&]() {
    return status_ok(mg::restricted_greedy_select_f16(d_logits.value(), d_allowed.value(),
                                                      d_counts.value(), d_out.value(), rows,
                                                      kVocab, max_allowed, stream.handle()),
                     "restricted_greedy_select_f16");
  };
  if (!launch()) return false;
  std::vector<std::uint32_t> got(rows);
  if (!bench::download(got, d_out.value(), stream)) return false;
  const double us = bench::time_launches(stream, 20, c.iterations, launch);
  if (us <= 0.0) return false;
  const double seconds = us * 1e-6;
  const double logical = static_cast<double>(total * (2u + 4u) + rows * 8u);
  out.rows = rows;
  out.total_allowed = total;
  out.iterations = c.iterations;
  out.average_us = us;
  out.sequences_per_second = static_cast<double>(rows) / seconds;
  out.candidate_gib_per_second = logical / seconds / static_cast<double>(1ull << 30);
  out.parity = got == expect;
  return true;
}

}  // namespace

int main(int argc, char** argv) {
  const char* dfa_path = nullptr;
  std::uint32_t divisor = 1;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--dfa" && i + 1 < argc) dfa_path = argv[++i];
    else if (a == "--iterations-divisor" && i + 1 < argc) divisor = static_cast<std::uint32_t>(std::strtoul(argv[++i], nullptr, 10));
    else {
      std::fprintf(stderr, "usage: %s --dfa FILE [--iterations-divisor N]\n", argv[0]);
      return 2;
    }
  }
  if (dfa_path == nullptr || divisor == 0) {
    std::fprintf(stderr, "usage: %s --dfa FILE [--iterations-divisor N]\n", argv[0]);
    return 2;
  }
  mg::DfaTables t;
  if (!bench::read_tables(dfa_path, t, kVocab)) {
    std::fprintf(stderr, "%s: not a DFA table file\n", dfa_path);
    return 1;
  }
  // the non-empty states' allowed sets, in state order
  std::vector<std::vector<std::uint32_t>> sets;
  std::size_t max_allowed = 0;
  for (std::uint64_t s = 0; s < t.states(); ++s) {
    const std::uint32_t b = t.offsets[s], e = t.offsets[s + 1];
    if (b == e) continue;
    sets.emplace_back(t.tokens.begin() + b, t.tokens.begin() + e);
    max_allowed = std::max<std::size_t>(max_allowed, e - b);
  }
  if (sets.empty()) return 1;
  constexpr std::array<Case, 3> cases{{{1, 2'000}, {16, 1'000}, {256, 500}}};
  std::array<Measurement, cases.size()> m{};
  for (std::size_t i = 0; i < cases.size(); ++i) {
    Case c = cases[i];
    c.iterations = std::max<std::uint32_t>(1, c.iterations / divisor);
    if (!run_case(c, sets, max_allowed, m[i])) return 1;
  }
  std::printf("{\"schema_version\":1,\"result\":\"pass\",\"operator\":\"restricted_greedy_f16\","
              "\"grammar\":\"smollm2_market_action_v1\",\"vocabulary_size\":%llu,"
              "\"grammar_states\":%llu,\"grammar_arcs\":%llu,\"maximum_allowed_tokens\":%zu,",
              static_cast<unsigned long long>(kVocab),
              static_cast<unsigned long long>(t.states()),
              static_cast<unsigned long long>(t.tokens.size()), max_allowed);
  bench::print_gpu(stdout);
  std::printf(",\"measurements\":[");
  for (std::size_t i = 0; i < m.size(); ++i) {
    std::printf("%s{\"rows\":%llu,\"total_allowed_candidates\":%llu,\"iterations\":%u,"
                "\"average_microseconds\":%.3f,\"sequences_per_second\":%.3f,"
                "\"candidate_gib_per_second\":%.3f}",
                i ? "," : "", static_cast<unsigned long long>(m[i].rows),
                static_cast<unsigned long long>(m[i].total_allowed), m[i].iterations,
                m[i].average_us, m[i].sequences_per_second, m[i].candidate_gib_per_second);
  }
  std::printf("]}\n");
  for (const auto& x : m) {
    if (!x.parity) {
      std::fprintf(stderr, "token parity failed at %llu rows\n", static_cast<unsigned long long>(x.rows));
      return 3;
    }
  }
  return 0;
}
