// Tests of the C++ operator layer (include/marketforge_gpu.hpp), written the
// way the reference's own operator tests are (tests/cuda/cuda_tests.cu):
// build inputs on the host, upload through DeviceBuffer, run the op on an
// explicit stream, download and compare.
//
//   host_api_test --cpu   type semantics and argument validation; needs no
//                         GPU (validation precedes every device call)
//   host_api_test --gpu   the reference known answers on the device, and a
//                         decode-tail pack against the CPU oracle
//                         (oracle/liboracle.so, bit-exact)
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <span>
#include <string>
#include <vector>

#include "marketforge_gpu.hpp"

extern "C" {
// oracle/oracle.c (test infrastructure)
uint16_t orc_float_to_half(float f);
void orc_rms_norm_f32(const float* input, const float* weight, float epsilon, float* output,
                      uint64_t rows, uint64_t hidden);
int orc_decode_tail(const float* x, const float* norm_weight, float epsilon,
                    const uint16_t* embedding, const float* embedding_f32, uint64_t vocab,
                    uint64_t hidden, const uint32_t* row_state, uint64_t rows,
                    const uint32_t* state_offsets, const uint32_t* state_tokens,
                    uint64_t states, const uint32_t* state_next, const int32_t* next_table,
                    int order, uint32_t* out_token, float* out_score, uint32_t* out_next,
                    int threads);
}

namespace mg = marketforge::gpu;

namespace {

int failures = 0;
int checks = 0;

#define CHECK(cond)                                                          \
  do {                                                                       \
    ++checks;                                                                \
    if (!(cond)) {                                                           \
      ++failures;                                                            \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, \
                   #cond);                                                   \
    }                                                                        \
  } while (0)

#define REQUIRE_OK(expr)                                                          \
  do {                                                                            \
    const mg::Status s_ = (expr);                                                 \
    if (!s_.ok()) {                                                               \
      std::fprintf(stderr, "%s:%d: %s -> code %d detail %u\n", __FILE__, __LINE__, \
                   #expr, static_cast<int>(s_.code), s_.detail);                  \
      ++failures;                                                                 \
      return;                                                                     \
    }                                                                             \
  } while (0)

// ---- CPU: types and validation ---------------------------------------------

static_assert(static_cast<int>(mg::ErrorCode::invalid_argument) == MF_INVALID_ARGUMENT);
static_assert(static_cast<int>(mg::ErrorCode::arithmetic_overflow) == MF_ARITHMETIC_OVERFLOW);
static_assert(static_cast<int>(mg::ErrorCode::allocation_failed) == MF_ALLOCATION_FAILED);
static_assert(static_cast<int>(mg::ErrorCode::resource_limit) == MF_RESOURCE_LIMIT);
static_assert(static_cast<int>(mg::ErrorCode::cuda_backend_failure) == MF_DEVICE_BACKEND_FAILURE);
static_assert(static_cast<int>(mg::ErrorCode::cuda_runtime_failure) == MF_DEVICE_RUNTIME_FAILURE);
static_assert(mg::restricted_greedy_invalid_token_id == UINT32_MAX);

void test_status_and_result() {
  CHECK(mg::Status::success().ok());
  const mg::Status f = mg::Status::failure(mg::ErrorCode::resource_limit, 7);
  CHECK(!f.ok() && f.detail == 7u);
  CHECK(f == mg::Status::failure(mg::ErrorCode::resource_limit, 7));
  auto r = mg::Result<int>::success(5);
  CHECK(r.has_value() && r.value() == 5 && r.status().ok());
  auto e = mg::Result<int>::failure(f);
  CHECK(!e && e.status() == f);
}

void test_buffers_without_device() {
  mg::DeviceBuffer empty;
  CHECK(empty.size_bytes() == 0 && !empty.address().valid());
  // a zero-byte allocation owns nothing and touches no device
  auto zero = mg::DeviceBuffer::allocate(0);
  CHECK(zero.has_value() && !zero.value().address().valid());
  mg::DeviceBuffer moved(std::move(zero).value());
  CHECK(moved.size_bytes() == 0);
  // copies validate before any device call: null stream, then bounds
  char host[4] = {};
  CHECK(empty.copy_from_host_async(host, 4, 0, mg::StreamHandle{}).code ==
        mg::ErrorCode::invalid_argument);
  CHECK(empty.copy_from_host_async(host, 4, 0, mg::StreamHandle{0x1000}).code ==
        mg::ErrorCode::invalid_argument);
  CHECK(empty.copy_to_host_async(host, 1, UINT64_MAX, mg::StreamHandle{0x1000}).code ==
        mg::ErrorCode::arithmetic_overflow);
}

void test_validation_order() {
  const mg::StreamHandle fake{0x1000};
  mg::DeviceBuffer a, b, c, d, e;
  // zero dimensions and a missing stream come first (greedy.cu:245-252)
  CHECK(mg::greedy_select_f16(a, b, 0, 8, fake).code == mg::ErrorCode::invalid_argument);
  CHECK(mg::greedy_select_f16(a, b, 1, 8, mg::StreamHandle{}).code ==
        mg::ErrorCode::invalid_argument);
  // mismatched sizes (empty buffers) are invalid arguments
  CHECK(mg::greedy_select_f16(a, b, 1, 8, fake).code == mg::ErrorCode::invalid_argument);
  // limits before sizes: a vocabulary beyond uint32 ids (greedy.cu:361-364)
  CHECK(mg::restricted_output_head_f16(a, b, c, d, e, 1, 8, (1ull << 32) + 1, 1, fake).code ==
        mg::ErrorCode::resource_limit);
  // a negative epsilon is an invalid argument (rms_norm.cu:112-118)
  CHECK(mg::rms_norm_f32(a, b, c, 1, 8, -1.0f, fake).code == mg::ErrorCode::invalid_argument);
  mg::BlasHandle h;
  CHECK(mg::linear_f16(a, b, c, 0, 8, 8, h, fake).code == mg::ErrorCode::invalid_argument);
  // decode tail: a missing x is an invalid argument, found before any launch
  mg::DecodeTailArgs t;
  t.rows = 4;
  t.hidden = 64;
  t.vocab = 128;
  t.states = 2;
  t.nnz = 4;
  t.max_count = 2;
  CHECK(mg::decode_tail_workspace_bytes(t).status().code == mg::ErrorCode::invalid_argument);
  t.unrestricted_count = 5;  // more unrestricted rows than rows
  CHECK(mg::decode_tail_workspace_bytes(t).status().code == mg::ErrorCode::resource_limit);
}

// ---- GPU: reference known answers and an oracle-checked pack ----------------

// Upload and wait: the host vector may be a temporary, and an asynchronous
// copy reads it until the stream reaches the copy.
template <typename T>
mg::Result<mg::DeviceBuffer> upload(const std::vector<T>& host, const mg::GpuStream& stream) {
  auto buf = mg::DeviceBuffer::allocate(host.size() * sizeof(T));
  if (!buf) return buf;
  mg::Status s = buf.value().copy_from_host_async(host.data(), host.size() * sizeof(T), 0,
                                                  stream.handle());
  if (s.ok()) s = stream.synchronize();
  if (!s.ok()) return mg::Result<mg::DeviceBuffer>::failure(s);
  return buf;
}

template <typename T>
std::vector<T> download(const mg::DeviceBuffer& buf, const mg::GpuStream& stream) {
  std::vector<T> out(buf.size_bytes() / sizeof(T));
  if (!buf.copy_to_host_async(out.data(), buf.size_bytes(), 0, stream.handle()).ok() ||
      !stream.synchronize().ok()) {
    ++failures;
  }
  return out;
}

std::vector<uint16_t> to_half(const std::vector<float>& v) {
  std::vector<uint16_t> h(v.size());
  for (size_t i = 0; i < v.size(); ++i) h[i] = orc_float_to_half(v[i]);
  return h;
}

// tests/cuda/cuda_tests.cu:699-800: tokens [14, 8, 1] (row 1 ties tokens 4
// and 6 -> 4 loses to 8 on score; row 2 is all NaN -> lowest id 1).
void test_tiny_head(const mg::GpuStream& stream) {
  const uint64_t rows = 3, hidden = 8, vocab = 17, max_allowed = 5;
  std::vector<float> h(rows * hidden), e(vocab * hidden);
  for (uint64_t i = 0; i < h.size(); ++i) h[i] = static_cast<float>(static_cast<int>(i % 11) - 5) / 8.0f;
  for (uint64_t i = 0; i < e.size(); ++i) {
    e[i] = static_cast<float>(static_cast<int>((i * 7) % 19) - 9) / 16.0f;
  }
  for (uint64_t f = 0; f < hidden; ++f) e[6 * hidden + f] = e[4 * hidden + f];
  for (uint64_t f = 0; f < hidden; ++f) h[2 * hidden + f] = NAN;
  const std::vector<uint32_t> allowed = {9, 3, 14, 0, 0, 6, 4, 8, 0, 0, 7, 1, 0, 0, 0};
  const std::vector<uint32_t> counts = {3, 3, 2};
  auto dh = upload(to_half(h), stream);
  auto de = upload(to_half(e), stream);
  auto da = upload(allowed, stream);
  auto dc = upload(counts, stream);
  auto dout = mg::DeviceBuffer::allocate(rows * 4);
  if (!dh || !de || !da || !dc || !dout) {
    ++failures;
    return;
  }
  REQUIRE_OK(mg::restricted_output_head_f16(dh.value(), de.value(), da.value(), dc.value(),
                                            dout.value(), rows, hidden, vocab, max_allowed,
                                            stream.handle()));
  const auto tok = download<uint32_t>(dout.value(), stream);
  CHECK(tok.size() == 3 && tok[0] == 14u && tok[1] == 8u && tok[2] == 1u);
}

// tests/cuda/cuda_tests.cu:508-531: winner (7 r + 3) % V; row 1 ties 9 with
// its winner -> 9; row 2 all -inf with NaN at 0 -> 1.
void test_greedy(const mg::GpuStream& stream) {
  const uint64_t rows = 4, vocab = 17;
  std::vector<float> logits(rows * vocab, -4.0f);
  std::vector<uint32_t> expect(rows);
  for (uint64_t r = 0; r < rows; ++r) {
    expect[r] = static_cast<uint32_t>((r * 7 + 3) % vocab);
    logits[r * vocab + expect[r]] = 8.0f;
  }
  logits[1 * vocab + 9] = 8.0f;
  expect[1] = 9;
  for (uint64_t v = 0; v < vocab; ++v) logits[2 * vocab + v] = -INFINITY;
  logits[2 * vocab + 0] = NAN;
  expect[2] = 1;
  auto dl = upload(to_half(logits), stream);
  auto dout = mg::DeviceBuffer::allocate(rows * 4);
  if (!dl || !dout) {
    ++failures;
    return;
  }
  REQUIRE_OK(mg::greedy_select_f16(dl.value(), dout.value(), rows, vocab, stream.handle()));
  CHECK(download<uint32_t>(dout.value(), stream) == expect);
}

// RMSNorm in place (input and output alias, rms_norm.hpp:16) against the
// oracle's restatement of operators.cpp:523-535, bit for bit.
void test_rms_norm(const mg::GpuStream& stream) {
  const uint64_t rows = 5, hidden = 576;
  std::vector<float> x(rows * hidden), w(hidden), expect(rows * hidden);
  uint32_t s = 12345u;
  auto next = [&s]() {
    s = s * 1664525u + 1013904223u;
    return static_cast<float>(s >> 8) * 0x1p-24f * 4.0f - 2.0f;
  };
  for (auto& v : x) v = next();
  for (auto& v : w) v = 1.0f + next() * 0.01f;
  orc_rms_norm_f32(x.data(), w.data(), 1e-5f, expect.data(), rows, hidden);
  auto dx = upload(x, stream);
  auto dw = upload(w, stream);
  if (!dx || !dw) {
    ++failures;
    return;
  }
  REQUIRE_OK(mg::rms_norm_f32(dx.value(), dw.value(), dx.value(), rows, hidden, 1e-5f,
                              stream.handle()));
  const auto y = download<float>(dx.value(), stream);
  CHECK(y.size() == expect.size() &&
        std::memcmp(y.data(), expect.data(), y.size() * sizeof(float)) == 0);
  // the weight may not alias the output
  CHECK(mg::rms_norm_f32(dx.value(), dx.value(), dx.value(), 1, rows * hidden, 1e-5f,
                         stream.handle()).code == mg::ErrorCode::invalid_argument);
}

// A small ragged pack with DFA advance and unrestricted rows, against the
// oracle's decode tail.
void test_decode_tail(const mg::GpuStream& stream, mg::DotOrder order) {
  const uint64_t rows = 24, hidden = 128, vocab = 2048, states = 12;
  uint64_t seed = 0x9E3779B97F4A7C15ull;
  auto rnd = [&seed]() {
    seed ^= seed << 13;
    seed ^= seed >> 7;
    seed ^= seed << 17;
    return seed;
  };
  auto unit = [&rnd]() { return static_cast<float>(rnd() >> 40) * 0x1p-24f; };
  std::vector<float> x(rows * hidden), w(hidden), e(vocab * hidden);
  for (auto& v : x) v = unit() * 4.0f - 2.0f;
  for (auto& v : w) v = 1.0f + (unit() - 0.5f) * 0.04f;
  for (auto& v : e) v = (unit() - 0.5f) * 0.1f;
  const auto e16 = to_half(e);
  // state lists: distinct ascending ids, sizes 1..300
  std::vector<uint32_t> offsets = {0}, tokens, next;
  uint64_t max_count = 0;
  for (uint64_t s = 0; s < states; ++s) {
    const uint64_t n = 1 + rnd() % 300;
    std::vector<char> used(vocab, 0);
    uint64_t got = 0;
    while (got < n) {
      const uint32_t t = static_cast<uint32_t>(rnd() % vocab);
      if (!used[t]) {
        used[t] = 1;
        ++got;
      }
    }
    for (uint32_t t = 0; t < vocab; ++t) {
      if (used[t]) {
        tokens.push_back(t);
        next.push_back(static_cast<uint32_t>(rnd() % states));
      }
    }
    offsets.push_back(static_cast<uint32_t>(tokens.size()));
    max_count = n > max_count ? n : max_count;
  }
  std::vector<uint32_t> row_state(rows), unrestricted;
  for (uint64_t r = 0; r < rows; ++r) {
    row_state[r] = static_cast<uint32_t>(rnd() % states);
    if (r % 7 == 3) {
      row_state[r] = mg::state_unrestricted;
      unrestricted.push_back(static_cast<uint32_t>(r));
    }
  }
  row_state[5] = static_cast<uint32_t>(states + 3);  // invalid state
  std::vector<uint32_t> etok(rows), enext(rows);
  std::vector<float> escore(rows);
  orc_decode_tail(x.data(), w.data(), 1e-5f, e16.data(), nullptr, vocab, hidden,
                  row_state.data(), rows, offsets.data(), tokens.data(), states, next.data(),
                  nullptr, static_cast<int>(order), etok.data(), escore.data(), enext.data(), 1);

  const auto h = stream.handle();
  auto dx = upload(x, stream);
  auto dw = upload(w, stream);
  auto de = upload(e16, stream);
  auto drs = upload(row_state, stream);
  auto doff = upload(offsets, stream);
  auto dtok = upload(tokens, stream);
  auto dnext = upload(next, stream);
  auto dunr = upload(unrestricted, stream);
  auto otok = mg::DeviceBuffer::allocate(rows * 4);
  auto osc = mg::DeviceBuffer::allocate(rows * 4);
  auto onx = mg::DeviceBuffer::allocate(rows * 4);
  if (!dx || !dw || !de || !drs || !doff || !dtok || !dnext || !dunr || !otok || !osc || !onx) {
    ++failures;
    return;
  }
  mg::DecodeTailArgs a;
  a.x = &dx.value();
  a.norm_weight = &dw.value();
  a.epsilon = 1e-5f;
  a.order = order;
  a.embedding = &de.value();
  a.row_state = &drs.value();
  a.state_offsets = &doff.value();
  a.state_tokens = &dtok.value();
  a.state_next = &dnext.value();
  a.unrestricted_rows = &dunr.value();
  a.out_token = &otok.value();
  a.out_score = &osc.value();
  a.out_next_state = &onx.value();
  a.rows = rows;
  a.hidden = hidden;
  a.vocab = vocab;
  a.states = states;
  a.nnz = tokens.size();
  a.max_count = max_count;
  a.unrestricted_count = unrestricted.size();
  auto bytes = mg::decode_tail_workspace_bytes(a);
  if (!bytes) {
    ++failures;
    return;
  }
  auto ws = mg::DeviceBuffer::allocate(bytes.value());
  if (!ws) {
    ++failures;
    return;
  }
  REQUIRE_OK(mg::workspace_init(ws.value(), h));
  for (int step = 0; step < 2; ++step) {  // the workspace is reusable
    REQUIRE_OK(mg::decode_tail_f16(a, ws.value(), h));
    const auto tok = download<uint32_t>(otok.value(), stream);
    const auto sc = download<float>(osc.value(), stream);
    const auto nx = download<uint32_t>(onx.value(), stream);
    CHECK(tok == etok);
    CHECK(nx == enext);
    bool scores_equal = sc.size() == escore.size();
    for (size_t i = 0; scores_equal && i < sc.size(); ++i) {
      scores_equal = std::isnan(sc[i]) ? std::isnan(escore[i])
                                       : std::memcmp(&sc[i], &escore[i], 4) == 0;
    }
    CHECK(scores_equal);
  }
  CHECK(etok[5] == mg::restricted_greedy_invalid_token_id);
}

// A DFA with the reference grammar layer's interface (token_dfa.hpp:30-74):
// the trie of {41: [9, 4], 7: [3, 8, 1], 99: [9, 6]} the reference builds
// (token_dfa_tests.cpp:22-49), states in creation order.
struct MockState {
  uint32_t value{0};
};
struct MockArc {
  uint32_t token{0};
  MockState next{};
};
struct MockDfa {
  std::vector<uint32_t> first{0, 2, 4, 4, 5, 6, 6}, count{2, 2, 0, 1, 1, 0, 0};
  std::vector<MockArc> arcs{{3, {3}}, {9, {1}}, {4, {2}}, {6, {6}}, {8, {4}}, {1, {5}}};
  std::vector<uint32_t> term{UINT32_MAX, UINT32_MAX, 41, UINT32_MAX, UINT32_MAX, 7, 99};
  MockState root() const { return {}; }
  size_t state_count() const { return first.size(); }
  mg::Result<std::span<const MockArc>> allowed(MockState s) const {
    if (s.value >= first.size())
      return mg::Result<std::span<const MockArc>>::failure(
          mg::Status::failure(mg::ErrorCode::invalid_argument));
    return mg::Result<std::span<const MockArc>>::success(
        std::span<const MockArc>(arcs).subspan(first[s.value], count[s.value]));
  }
  bool terminal(MockState s) const { return s.value < term.size() && term[s.value] != UINT32_MAX; }
  mg::Result<uint32_t> decode_terminal(MockState s) const {
    if (!terminal(s))
      return mg::Result<uint32_t>::failure(mg::Status::failure(mg::ErrorCode::invalid_argument));
    return mg::Result<uint32_t>::success(term[s.value]);
  }
};

void test_dfa_export() {
  const MockDfa dfa;
  auto t = mg::export_token_dfa(dfa, 64);
  CHECK(t.has_value());
  if (!t) return;
  const mg::DfaTables& d = t.value();
  CHECK((d.offsets == std::vector<uint32_t>{0, 2, 4, 4, 5, 6, 6, 6}));
  CHECK((d.tokens == std::vector<uint32_t>{3, 9, 4, 6, 8, 1}));
  CHECK((d.next == std::vector<uint32_t>{3, 1, 2, 6, 4, 5}));
  CHECK((d.choice == std::vector<uint32_t>{mg::no_choice, mg::no_choice, 41, mg::no_choice,
                                           mg::no_choice, 7, 99}));
  CHECK(d.max_count == 2 && d.depth == 3 && d.states() == 7 && d.arcs() == 6);
  // a token beyond the vocabulary, descending tokens, a cycle
  CHECK(mg::export_token_dfa(dfa, 9).status().code == mg::ErrorCode::invalid_format);
  mg::DfaTables bad = d;
  std::swap(bad.tokens[0], bad.tokens[1]);
  CHECK(bad.finish(64).code == mg::ErrorCode::invalid_format);
  bad = d;
  bad.next[5] = 0;  // 4 --1--> root
  CHECK(bad.finish(64).code == mg::ErrorCode::invalid_format);
}

// The device-resident decode loop on the mock DFA against the oracle run
// step by step on the host (finished rows hold their terminal state).
void test_restricted_decoder(const mg::GpuStream& stream) {
  const uint64_t rows = 6, hidden = 64, vocab = 64, steps = 5;
  auto exported = mg::export_token_dfa(MockDfa{}, vocab);
  if (!exported) {
    ++failures;
    return;
  }
  const mg::DfaTables tables = exported.value();
  uint64_t seed = 0xD1B54A32D192ED03ull;
  auto unit = [&seed]() {
    seed ^= seed << 13;
    seed ^= seed >> 7;
    seed ^= seed << 17;
    return static_cast<float>(seed >> 40) * 0x1p-24f;
  };
  std::vector<float> e(vocab * hidden), x(steps * rows * hidden);
  for (auto& v : e) v = (unit() - 0.5f) * 0.2f;
  for (auto& v : x) v = unit() * 2.0f - 1.0f;
  const auto e16 = to_half(e);
  const auto h = stream.handle();
  auto de = upload(e16, stream);
  auto dx = upload(x, stream);
  auto dfa = mg::DeviceDfa::upload(tables, h);
  if (!de || !dx || !dfa) {
    ++failures;
    return;
  }
  mg::RestrictedDecoder::Config cfg;
  cfg.rows = rows;
  cfg.hidden = hidden;
  cfg.vocab = vocab;
  cfg.max_steps = steps;
  auto dec = mg::RestrictedDecoder::create(de.value(), nullptr, dfa.value(), cfg, h);
  if (!dec) {
    std::fprintf(stderr, "decoder: code %d\n", static_cast<int>(dec.status().code));
    ++failures;
    return;
  }
  const std::vector<uint32_t> start{0, 0, 1, 3, 2, 0};  // root, mid-way, already finished
  REQUIRE_OK(dec.value().start(start.data(), h));
  for (uint64_t k = 0; k < steps; ++k) {
    const mf_buffer view{dx.value().address().value + k * rows * hidden * 4, rows * hidden * 4};
    REQUIRE_OK(dec.value().step(view, h));
  }
  auto out = dec.value().finish(h);
  if (!out) {
    ++failures;
    return;
  }
  std::vector<uint32_t> state = start, tok(rows), nx(rows);
  std::vector<float> sc(rows);
  bool same = out.value().steps == steps;
  for (uint64_t k = 0; same && k < steps; ++k) {
    orc_decode_tail(x.data() + k * rows * hidden, nullptr, 1e-5f, e16.data(), nullptr, vocab,
                    hidden, state.data(), rows, tables.offsets.data(), tables.tokens.data(),
                    tables.states(), tables.next.data(), nullptr, 0, tok.data(), sc.data(),
                    nx.data(), 1);
    for (uint64_t r = 0; r < rows; ++r) {
      const bool empty = state[r] < tables.states() &&
                         tables.offsets[state[r] + 1] == tables.offsets[state[r]];
      state[r] = empty ? state[r] : nx[r];
      same = same && out.value().tokens[k * rows + r] == tok[r];
    }
  }
  CHECK(same);
  CHECK(out.value().states == state);
  for (uint64_t r = 0; r < rows; ++r) CHECK(out.value().choice[r] == tables.choice[state[r]]);
  CHECK(out.value().choice[4] == 41u);  // started finished, held there
}

void run_gpu() {
  auto stream = mg::GpuStream::create();
  if (!stream) {
    std::fprintf(stderr, "stream creation failed: code %d\n",
                 static_cast<int>(stream.status().code));
    ++failures;
    return;
  }
  std::printf("gpu: tiny head\n");
  test_tiny_head(stream.value());
  std::printf("gpu: greedy\n");
  test_greedy(stream.value());
  std::printf("gpu: rms_norm\n");
  test_rms_norm(stream.value());
  std::printf("gpu: decode tail (fma chain)\n");
  test_decode_tail(stream.value(), mg::DotOrder::fma_chain);
  std::printf("gpu: decode tail (mul-add chain)\n");
  test_decode_tail(stream.value(), mg::DotOrder::mul_add_chain);
  std::printf("gpu: restricted decoder\n");
  test_restricted_decoder(stream.value());
  std::fflush(stdout);
}

}  // namespace

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "--cpu";
  test_status_and_result();
  test_buffers_without_device();
  test_validation_order();
  test_dfa_export();
  if (mode == "--gpu") run_gpu();
  std::printf("%s: %d checks, %d failures\n", mode.c_str(), checks, failures);
  return failures == 0 ? 0 : 1;
}
