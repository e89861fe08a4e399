// decode_loop_bench -- restricted generation over a token DFA, on MI355X,
// through the C++ operator layer (include/marketforge_gpu.hpp).
//
// B sequences generate one grammar choice each (the SmolLM2 market-action
// DFA when given its table file), greedy and restricted, from the DFA root
// until every sequence is terminal.  Hidden rows are synthetic N(0, 1) per
// step (the model layers are not part of this path); the tied FP16 table is
// N(0, 0.02); the final norm weight is 1 + N(0, 0.02).
//
// Four loops over the same inputs, each timed with HIP events around R whole
// generations (after warm-up):
//   resident         RestrictedDecoder: one mf_decode_tail_f16 per step, DFA
//                    state on the device, no host round trip until the end;
//   graph            the same steps captured once into a HIP graph and
//                    replayed (the per-generation start copy stays eager);
//   round_trip       the reference's loop structure on the same kernels: per
//                    step the states go up, the tail runs, the tokens come
//                    back, the stream synchronizes and the host advances the
//                    DFA (CudaSmolLm2::decode_restricted, smollm2.cu:336-366,
//                    :386-405, :494-501, with token_dfa.cpp:111-128 on the host);
//   reference_ops    the reference's own operators in that loop: per step the
//                    allowed lists go up as a fixed-width table, then
//                    rms_norm_f16 and restricted_output_head_f16 on FP16
//                    hidden rows (smollm2.cu:473-493), tokens back, sync, host
//                    advance.
// resident, graph and round_trip must produce identical tokens (checked);
// reference_ops rounds the hidden rows to FP16 first, so its tokens may
// differ (reported, not required).
//
// Usage: decode_loop_bench --dfa FILE [--rows B] [--repeats R] [--hidden H] [--no-fused]
// FILE is the binary table written by market_sim_amd.dfa.write_tables.
#include <hip/hip_runtime_api.h>

#include <chrono>
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

constexpr std::uint64_t kVocab = 49'152;

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return false;
}

bool ok(const mg::Status& s, const char* what) {
  if (s.ok()) return true;
  std::fprintf(stderr, "%s: error code %u detail %u\n", what, static_cast<unsigned>(s.code),
               s.detail);
  return false;
}

// xoshiro256** with a splitmix64 seed, Box-Muller normals in double
struct Rng {
  std::uint64_t s[4];
  explicit Rng(std::uint64_t seed) {
    for (auto& v : s) {
      seed += 0x9E3779B97F4A7C15ull;
      std::uint64_t z = seed;
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
      v = z ^ (z >> 31);
    }
  }
  static std::uint64_t rotl(std::uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
  std::uint64_t next() {
    const std::uint64_t r = rotl(s[1] * 5, 7) * 9;
    const std::uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
  }
  double uniform() { return (static_cast<double>(next() >> 11) + 0.5) * 0x1p-53; }
  float normal() {
    const double u = uniform(), v = uniform();
    return static_cast<float>(std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v));
  }
};

std::uint16_t to_half(float value) {
  // IEEE binary16, round to nearest even
  std::uint32_t x;
  std::memcpy(&x, &value, 4);
  const std::uint32_t sign = (x >> 16) & 0x8000u, mag = x & 0x7FFFFFFFu;
  if (mag >= 0x7F800000u) return static_cast<std::uint16_t>(sign | 0x7C00u | (mag > 0x7F800000u ? 0x200u : 0u));
  if (mag >= 0x477FF000u) return static_cast<std::uint16_t>(sign | 0x7C00u);
  if (mag < 0x38800000u) {
    const float r = std::nearbyint(std::fabs(value) * 16777216.0f);
    return static_cast<std::uint16_t>(sign | static_cast<std::uint32_t>(r));
  }
  std::uint32_t h = (((mag >> 23) - 112u) << 10) | ((mag & 0x7FFFFFu) >> 13);
  const std::uint32_t rest = mag & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
  return static_cast<std::uint16_t>(sign | h);
}

bool read_tables(const char* path, mg::DfaTables& t) {
  FILE* f = std::fopen(path, "rb");
  if (f == nullptr) return false;
  std::uint32_t head[3];
  bool good = std::fread(head, 4, 3, f) == 3 && head[0] == 0x3144464Du;
  if (good) {
    t.offsets.resize(head[1] + 1);
    t.tokens.resize(head[2]);
    t.next.resize(head[2]);
    t.choice.resize(head[1]);
    good = std::fread(t.offsets.data(), 4, t.offsets.size(), f) == t.offsets.size() &&
           std::fread(t.tokens.data(), 4, t.tokens.size(), f) == t.tokens.size() &&
           std::fread(t.next.data(), 4, t.next.size(), f) == t.next.size() &&
           std::fread(t.choice.data(), 4, t.choice.size(), f) == t.choice.size();
  }
  std::fclose(f);
  return good && t.finish(kVocab).ok();
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

// host-side advance with finished rows held (token_dfa.cpp:111-128)
std::uint32_t host_advance(const mg::DfaTables& t, std::uint32_t state, std::uint32_t token) {
  if (state >= t.states()) return mg::state_invalid;
  const std::uint32_t b = t.offsets[state], e = t.offsets[state + 1];
  if (b == e) return state;
  std::uint32_t lo = b, hi = e;
  while (lo < hi) {
    const std::uint32_t mid = (lo + hi) / 2;
    if (t.tokens[mid] < token) lo = mid + 1; else hi = mid;
  }
  return (lo < e && t.tokens[lo] == token) ? t.next[lo] : mg::state_invalid;
}

struct Timer {
  hipEvent_t a = nullptr, b = nullptr;
  Timer() {
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
  }
  ~Timer() {
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
  }
  void start(hipStream_t s) { (void)hipEventRecord(a, s); }
  double stop_ms(hipStream_t s) {
    float ms = 0.0f;
    (void)hipEventRecord(b, s);
    (void)hipEventSynchronize(b);
    (void)hipEventElapsedTime(&ms, a, b);
    return ms;
  }
};

}  // namespace

int main(int argc, char** argv) {
  const char* dfa_path = nullptr;
  std::uint64_t rows = 256, repeats = 50, hidden = 576;
  bool fused = true;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--dfa" && i + 1 < argc) dfa_path = argv[++i];
    else if (a == "--rows" && i + 1 < argc) rows = std::strtoull(argv[++i], nullptr, 10);
    else if (a == "--repeats" && i + 1 < argc) repeats = std::strtoull(argv[++i], nullptr, 10);
    else if (a == "--hidden" && i + 1 < argc) hidden = std::strtoull(argv[++i], nullptr, 10);
    else if (a == "--no-fused") fused = false;
    else {
      std::fprintf(stderr, "usage: %s --dfa FILE [--rows B] [--repeats R] [--hidden H] [--no-fused]\n",
                   argv[0]);
      return 2;
    }
  }
  mg::DfaTables tables;
  if (dfa_path == nullptr || !read_tables(dfa_path, tables)) {
    std::fprintf(stderr, "cannot read a DFA table from %s\n", dfa_path ? dfa_path : "(none)");
    return 2;
  }
  if (rows == 0 || rows > 65535 || repeats == 0 || hidden == 0 || hidden % 64 != 0) return 2;
  const std::uint64_t steps = tables.depth;  // every sequence is terminal after this many

  // inputs
  Rng rng(2024);
  std::vector<std::uint16_t> table(kVocab * hidden);
  for (auto& v : table) v = to_half(0.02f * rng.normal());
  std::vector<float> weight(hidden), x(steps * rows * hidden);
  for (auto& v : weight) v = 1.0f + 0.02f * rng.normal();
  for (auto& v : x) v = rng.normal();
  std::vector<std::uint16_t> x16(x.size()), w16(hidden);
  for (std::size_t i = 0; i < x.size(); ++i) x16[i] = to_half(x[i]);
  for (std::size_t i = 0; i < hidden; ++i) w16[i] = to_half(weight[i]);

  auto stream_r = mg::GpuStream::create();
  if (!stream_r) return 1;
  mg::GpuStream& stream = stream_r.value();
  const mg::StreamHandle h = stream.handle();
  const auto hs = reinterpret_cast<hipStream_t>(h.value);
  auto d_table = upload(table, stream);
  auto d_w = upload(weight, stream);
  auto d_x = upload(x, stream);
  auto d_x16 = upload(x16, stream);
  auto d_w16 = upload(w16, stream);
  auto dfa = mg::DeviceDfa::upload(tables, h);
  if (!d_table || !d_w || !d_x || !d_x16 || !d_w16 || !dfa) return 1;
  mg::RestrictedDecoder::Config cfg;
  cfg.rows = rows;
  cfg.hidden = hidden;
  cfg.vocab = kVocab;
  cfg.max_steps = steps;
  cfg.fused = fused;
  auto dec_r = mg::RestrictedDecoder::create(d_table.value(), &d_w.value(), dfa.value(), cfg, h);
  if (!dec_r) return 1;
  mg::RestrictedDecoder& dec = dec_r.value();
  const std::uint64_t step_bytes = rows * hidden * 4;
  auto step_view = [&](std::uint64_t k) {
    return mf_buffer{d_x.value().address().value + k * step_bytes, step_bytes};
  };
  auto generate = [&]() {
    if (!ok(dec.start(nullptr, h), "start")) return false;
    for (std::uint64_t k = 0; k < steps; ++k)
      if (!ok(dec.step(step_view(k), h), "step")) return false;
    return true;
  };

  // ---- resident ------------------------------------------------------------
  if (!generate()) return 1;
  auto ref_out = dec.finish(h);
  if (!ref_out) return 1;
  const mg::DecodeOutput resident_out = ref_out.value();
  std::uint64_t finished = 0, emitted = 0;
  for (std::uint64_t r = 0; r < rows; ++r) finished += resident_out.choice[r] != mg::no_choice;
  for (const std::uint32_t t : resident_out.tokens) emitted += t != mg::restricted_greedy_invalid_token_id;
  for (int i = 0; i < 3; ++i)
    if (!generate()) return 1;
  Timer timer;
  timer.start(hs);
  for (std::uint64_t i = 0; i < repeats; ++i)
    if (!generate()) return 1;
  const double resident_ms = timer.stop_ms(hs) / static_cast<double>(repeats);
  auto again = dec.finish(h);
  bool resident_stable = again && again.value().tokens == resident_out.tokens;

  // ---- graph ---------------------------------------------------------------
  bool graph_ok = true, graph_match = true;
  double graph_ms = 0.0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  if (!ok(dec.start(nullptr, h), "start") || !ok(stream.synchronize(), "sync")) return 1;
  graph_ok = hip_ok(hipStreamBeginCapture(hs, hipStreamCaptureModeRelaxed), "begin capture");
  for (std::uint64_t k = 0; graph_ok && k < steps; ++k) graph_ok = ok(dec.step(step_view(k), h), "captured step");
  if (graph_ok) graph_ok = hip_ok(hipStreamEndCapture(hs, &graph), "end capture");
  if (graph_ok) graph_ok = hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate");
  auto replay = [&]() {
    if (!ok(dec.start(nullptr, h), "start") || !hip_ok(hipGraphLaunch(exec, hs), "graph launch"))
      return false;
    dec.assume_steps(steps);  // the graph ran the captured steps
    return true;
  };
  if (graph_ok) {
    // each replay checked against the eager tokens, with eager work between
    for (int i = 0; i < 3 && graph_ok; ++i) {
      graph_ok = replay();
      auto out = graph_ok ? dec.finish(h) : mg::Result<mg::DecodeOutput>::failure({});
      graph_match = graph_match && out && out.value().tokens == resident_out.tokens &&
                    out.value().states == resident_out.states;
      graph_ok = graph_ok && generate() && static_cast<bool>(dec.finish(h));
    }
    timer.start(hs);
    for (std::uint64_t i = 0; graph_ok && i < repeats; ++i) graph_ok = replay();
    graph_ms = timer.stop_ms(hs) / static_cast<double>(repeats);
    auto out = dec.finish(h);
    graph_match = graph_match && out && out.value().tokens == resident_out.tokens;
  }
  if (exec != nullptr) (void)hipGraphExecDestroy(exec);
  if (graph != nullptr) (void)hipGraphDestroy(graph);

  // ---- round trip on the same kernels -----------------------------------------
  auto d_state = mg::DeviceBuffer::allocate(rows * 4);
  auto d_tok = mg::DeviceBuffer::allocate(rows * 4);
  auto d_sc = mg::DeviceBuffer::allocate(rows * 4);
  if (!d_state || !d_tok || !d_sc) return 1;
  mg::DecodeTailArgs ta;
  ta.norm_weight = &d_w.value();
  ta.embedding = &d_table.value();
  ta.row_state = &d_state.value();
  ta.state_offsets = &dfa.value().offsets();
  ta.state_tokens = &dfa.value().tokens();
  ta.out_token = &d_tok.value();
  ta.out_score = &d_sc.value();
  ta.rows = rows;
  ta.hidden = hidden;
  ta.vocab = kVocab;
  ta.states = tables.states();
  ta.nnz = tables.arcs();
  ta.max_count = tables.max_count;
  // one x buffer per step: DecodeTailArgs takes whole buffers
  std::vector<mg::DeviceBuffer> xs;
  for (std::uint64_t k = 0; k < steps; ++k) {
    std::vector<float> part(x.begin() + k * rows * hidden, x.begin() + (k + 1) * rows * hidden);
    auto b = upload(part, stream);
    if (!b) return 1;
    xs.push_back(std::move(b).value());
  }
  ta.x = &xs[0];
  auto ws_bytes = mg::decode_tail_workspace_bytes(ta);
  if (!ws_bytes) return 1;
  auto ws = mg::DeviceBuffer::allocate(ws_bytes.value());
  if (!ws || !ok(mg::workspace_init(ws.value(), h), "workspace")) return 1;
  std::vector<std::uint32_t> state(rows), tok(rows);
  std::vector<std::uint32_t> rt_tokens(steps * rows);
  auto round_trip = [&](bool record) {
    std::fill(state.begin(), state.end(), 0u);
    for (std::uint64_t k = 0; k < steps; ++k) {
      ta.x = &xs[k];
      if (!ok(d_state.value().copy_from_host_async(state.data(), rows * 4, 0, h), "h2d") ||
          !ok(mg::decode_tail_f16(ta, ws.value(), h), "tail") ||
          !ok(d_tok.value().copy_to_host_async(tok.data(), rows * 4, 0, h), "d2h") ||
          !ok(stream.synchronize(), "sync"))
        return false;
      for (std::uint64_t r = 0; r < rows; ++r) {
        const std::uint32_t s = state[r];
        const bool done = s < tables.states() && tables.offsets[s] == tables.offsets[s + 1];
        if (record) rt_tokens[k * rows + r] = tok[r];
        state[r] = done ? s : host_advance(tables, s, tok[r]);
      }
    }
    return true;
  };
  if (!round_trip(true)) return 1;
  const bool rt_match = rt_tokens == resident_out.tokens;
  for (int i = 0; i < 2; ++i)
    if (!round_trip(false)) return 1;
  auto t0 = std::chrono::steady_clock::now();
  for (std::uint64_t i = 0; i < repeats; ++i)
    if (!round_trip(false)) return 1;
  const double rt_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() /
                       static_cast<double>(repeats);

  // ---- the reference's operators in the same loop ----------------------------
  const std::uint64_t width = tables.max_count;
  auto d_ids = mg::DeviceBuffer::allocate(rows * width * 4);
  auto d_cnt = mg::DeviceBuffer::allocate(rows * 4);
  auto d_norm16 = mg::DeviceBuffer::allocate(rows * hidden * 2);
  if (!d_ids || !d_cnt || !d_norm16) return 1;
  std::vector<mg::DeviceBuffer> x16s;
  for (std::uint64_t k = 0; k < steps; ++k) {
    std::vector<std::uint16_t> part(x16.begin() + k * rows * hidden, x16.begin() + (k + 1) * rows * hidden);
    auto b = upload(part, stream);
    if (!b) return 1;
    x16s.push_back(std::move(b).value());
  }
  std::vector<std::uint32_t> ids(rows * width), cnt(rows);
  std::uint64_t ref_diff = 0;
  auto reference_ops = [&](bool record) {
    std::fill(state.begin(), state.end(), 0u);
    for (std::uint64_t k = 0; k < steps; ++k) {
      std::uint64_t live = 0;
      for (std::uint64_t r = 0; r < rows; ++r) {
        const std::uint32_t s = state[r];
        const std::uint32_t b = tables.offsets[s], e = tables.offsets[s + 1];
        // finished rows still take a slot (count 0 is the invalid sentinel)
        cnt[r] = e - b;
        live += e > b;
        for (std::uint32_t j = b; j < e; ++j) ids[r * width + (j - b)] = tables.tokens[j];
      }
      if (live == 0) break;
      if (!ok(d_ids.value().copy_from_host_async(ids.data(), rows * width * 4, 0, h), "h2d ids") ||
          !ok(d_cnt.value().copy_from_host_async(cnt.data(), rows * 4, 0, h), "h2d counts") ||
          !ok(mg::rms_norm_f16(x16s[k], d_w16.value(), d_norm16.value(), rows, hidden, 1e-5f, h), "norm") ||
          !ok(mg::restricted_output_head_f16(d_norm16.value(), d_table.value(), d_ids.value(),
                                             d_cnt.value(), d_tok.value(), rows, hidden, kVocab,
                                             width, h), "head") ||
          !ok(d_tok.value().copy_to_host_async(tok.data(), rows * 4, 0, h), "d2h") ||
          !ok(stream.synchronize(), "sync"))
        return false;
      for (std::uint64_t r = 0; r < rows; ++r) {
        const std::uint32_t s = state[r];
        const bool done = tables.offsets[s] == tables.offsets[s + 1];
        if (record && !done && tok[r] != resident_out.tokens[k * rows + r]) ++ref_diff;
        state[r] = done ? s : host_advance(tables, s, tok[r]);
      }
    }
    return true;
  };
  if (!reference_ops(true)) return 1;
  for (int i = 0; i < 2; ++i)
    if (!reference_ops(false)) return 1;
  t0 = std::chrono::steady_clock::now();
  for (std::uint64_t i = 0; i < repeats; ++i)
    if (!reference_ops(false)) return 1;
  const double ref_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() /
                        static_cast<double>(repeats);

  auto rates = [&](double ms) {
    char b[256];
    std::snprintf(b, sizeof b,
                  "{\"ms_per_generation\":%.5f,\"us_per_step\":%.3f,\"tokens_per_s\":%.1f,"
                  "\"actions_per_s\":%.1f}",
                  ms, ms * 1000.0 / static_cast<double>(steps),
                  static_cast<double>(emitted) / (ms * 1e-3),
                  static_cast<double>(finished) / (ms * 1e-3));
    return std::string(b);
  };
  std::printf(
      "{\"tool\":\"decode_loop_bench\",\"states\":%llu,\"arcs\":%llu,\"rows\":%llu,"
      "\"hidden\":%llu,\"vocab\":%llu,\"steps\":%llu,\"repeats\":%llu,\"fused\":%s,\"finished_rows\":%llu,"
      "\"emitted_tokens\":%llu,\"resident\":%s,\"resident_repeatable\":%s,\"graph\":%s,"
      "\"graph_ok\":%s,\"graph_token_parity\":%s,\"round_trip\":%s,\"round_trip_token_parity\":%s,"
      "\"reference_ops\":%s,\"reference_ops_token_differences\":%llu}\n",
      static_cast<unsigned long long>(tables.states()), static_cast<unsigned long long>(tables.arcs()),
      static_cast<unsigned long long>(rows), static_cast<unsigned long long>(hidden),
      static_cast<unsigned long long>(kVocab), static_cast<unsigned long long>(steps),
      static_cast<unsigned long long>(repeats), fused ? "true" : "false",
      static_cast<unsigned long long>(finished),
      static_cast<unsigned long long>(emitted), rates(resident_ms).c_str(),
      resident_stable ? "true" : "false", rates(graph_ms > 0 ? graph_ms : 1e9).c_str(),
      graph_ok ? "true" : "false", graph_match ? "true" : "false", rates(rt_ms).c_str(),
      rt_match ? "true" : "false", rates(ref_ms).c_str(),
      static_cast<unsigned long long>(ref_diff));
  return (resident_stable && rt_match && finished == rows) ? 0 : 3;
}
