// marketforge_gpu.hpp -- C++20 operator API of the MI355X restricted head.
//
// A header-only layer over the C ABI (marketforge_hip.h) that keeps the
// reference operator interface: the names, argument order and meaning, and
// the error behaviour of include/marketforge/cuda/{greedy,rms_norm,linear}.hpp
// over move-only DeviceBuffer / stream objects
// (include/marketforge/cuda/device_buffer.hpp:20-56, cuda_stream.hpp:10-43)
// and Status / Result (include/marketforge/core/status.hpp:7-49, result.hpp).
// Code written against marketforge::cuda compiles against marketforge::gpu
// with the namespace changed; CudaStream and CublasHandle are provided
// under their reference names too.
//
// Everything is noexcept and allocation-free except DeviceBuffer::allocate,
// the stream/handle factories and the set-up of the DFA and decoder objects
// at the end (host vectors, device buffers); ops never synchronize.
#pragma once

#include <algorithm>
#include <cstdint>
#include <optional>
#include <type_traits>
#include <utility>
#include <vector>

#include "marketforge_hip.h"

namespace marketforge::gpu {

// Numbering identical to the reference ErrorCode, so codes round-trip
// through logs and result schemas unchanged.
enum class ErrorCode : std::uint16_t {
  ok = 0,
  invalid_argument = 1,
  unsupported_dtype = 2,
  invalid_shape = 3,
  invalid_model = 4,
  arithmetic_overflow = 5,
  invalid_alignment = 6,
  allocation_failed = 7,
  insufficient_memory = 8,
  insufficient_resources = 9,
  io_error = 10,
  invalid_format = 11,
  invalid_utf8 = 12,
  invalid_json = 13,
  duplicate_key = 14,
  resource_limit = 15,
  truncated_data = 16,
  invalid_tensor = 17,
  missing_tensor = 18,
  unexpected_tensor = 19,
  hash_mismatch = 20,
  cuda_backend_failure = 21,   // a kernel launch failed (HIP code in detail)
  cuda_runtime_failure = 22,   // a runtime call failed (HIP code in detail)
  device_backend_failure = cuda_backend_failure,
  device_runtime_failure = cuda_runtime_failure,
};

struct Status {
  ErrorCode code{ErrorCode::ok};
  std::uint32_t detail{0};

  [[nodiscard]] constexpr bool ok() const noexcept { return code == ErrorCode::ok; }
  [[nodiscard]] static constexpr Status success() noexcept { return {}; }
  [[nodiscard]] static constexpr Status failure(ErrorCode error,
                                                std::uint32_t error_detail = 0) noexcept {
    return Status{error, error_detail};
  }
  friend constexpr bool operator==(const Status&, const Status&) = default;
};

// A value or the failure that prevented it.
template <typename T>
class [[nodiscard]] Result {
 public:
  [[nodiscard]] static Result success(T value) { return Result(std::move(value)); }
  [[nodiscard]] static Result failure(Status status) { return Result(status); }

  [[nodiscard]] bool has_value() const noexcept { return value_.has_value(); }
  [[nodiscard]] explicit operator bool() const noexcept { return has_value(); }
  [[nodiscard]] T& value() & { return *value_; }
  [[nodiscard]] const T& value() const& { return *value_; }
  [[nodiscard]] T&& value() && { return std::move(*value_); }
  [[nodiscard]] Status status() const noexcept { return status_; }

 private:
  explicit Result(T value) : value_(std::move(value)) {}
  explicit Result(Status status) : status_(status) {}
  std::optional<T> value_;
  Status status_{};
};

namespace detail {
[[nodiscard]] inline Status from_c(mf_status s) noexcept {
  return Status{static_cast<ErrorCode>(s.code), s.detail};
}
}  // namespace detail

struct DeviceAddress {
  std::uintptr_t value{0};
  [[nodiscard]] constexpr bool valid() const noexcept { return value != 0; }
  friend constexpr bool operator==(const DeviceAddress&, const DeviceAddress&) = default;
};

struct StreamHandle {
  std::uintptr_t value{0};
  [[nodiscard]] constexpr bool valid() const noexcept { return value != 0; }
  friend constexpr bool operator==(const StreamHandle&, const StreamHandle&) = default;
};

// A non-blocking HIP stream owned by the object.
class GpuStream {
 public:
  GpuStream() noexcept = default;
  [[nodiscard]] static Result<GpuStream> create() noexcept {
    std::uintptr_t h = 0;
    const Status s = detail::from_c(mf_stream_create(&h));
    if (!s.ok()) return Result<GpuStream>::failure(s);
    return Result<GpuStream>::success(GpuStream(StreamHandle{h}));
  }
  GpuStream(const GpuStream&) = delete;
  GpuStream& operator=(const GpuStream&) = delete;
  GpuStream(GpuStream&& other) noexcept : handle_(std::exchange(other.handle_, {})) {}
  GpuStream& operator=(GpuStream&& other) noexcept {
    if (this != &other) {
      release();
      handle_ = std::exchange(other.handle_, {});
    }
    return *this;
  }
  ~GpuStream() noexcept { release(); }

  [[nodiscard]] StreamHandle handle() const noexcept { return handle_; }
  [[nodiscard]] Status synchronize() const noexcept {
    return detail::from_c(mf_stream_synchronize(handle_.value));
  }

 private:
  explicit GpuStream(StreamHandle h) noexcept : handle_(h) {}
  void release() noexcept {
    if (handle_.valid()) (void)mf_stream_destroy(handle_.value);
    handle_ = {};
  }
  StreamHandle handle_{};
};
using CudaStream = GpuStream;

// Device memory owned by the object (a zero-byte buffer owns nothing).
class DeviceBuffer {
 public:
  DeviceBuffer() noexcept = default;
  [[nodiscard]] static Result<DeviceBuffer> allocate(std::uint64_t byte_count) noexcept {
    std::uintptr_t a = 0;
    const Status s = detail::from_c(mf_device_alloc(byte_count, &a));
    if (!s.ok()) return Result<DeviceBuffer>::failure(s);
    return Result<DeviceBuffer>::success(DeviceBuffer(DeviceAddress{a}, byte_count));
  }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& other) noexcept
      : address_(std::exchange(other.address_, {})),
        size_bytes_(std::exchange(other.size_bytes_, 0)) {}
  DeviceBuffer& operator=(DeviceBuffer&& other) noexcept {
    if (this != &other) {
      release();
      address_ = std::exchange(other.address_, {});
      size_bytes_ = std::exchange(other.size_bytes_, 0);
    }
    return *this;
  }
  ~DeviceBuffer() noexcept { release(); }

  [[nodiscard]] std::uint64_t size_bytes() const noexcept { return size_bytes_; }
  [[nodiscard]] DeviceAddress address() const noexcept { return address_; }
  // The C-ABI view of this allocation.
  [[nodiscard]] mf_buffer view() const noexcept { return mf_buffer{address_.value, size_bytes_}; }

  [[nodiscard]] Status copy_from_host_async(const void* source, std::uint64_t byte_count,
                                            std::uint64_t offset,
                                            StreamHandle stream) noexcept {
    return detail::from_c(
        mf_copy_to_device_async(view(), offset, source, byte_count, stream.value));
  }
  [[nodiscard]] Status copy_to_host_async(void* destination, std::uint64_t byte_count,
                                          std::uint64_t offset,
                                          StreamHandle stream) const noexcept {
    return detail::from_c(
        mf_copy_to_host_async(destination, view(), offset, byte_count, stream.value));
  }

 private:
  DeviceBuffer(DeviceAddress a, std::uint64_t n) noexcept : address_(a), size_bytes_(n) {}
  void release() noexcept {
    if (address_.valid()) (void)mf_device_free(address_.value);
    address_ = {};
    size_bytes_ = 0;
  }
  DeviceAddress address_{};
  std::uint64_t size_bytes_{0};
};

// The reference's linear_f16 takes a cuBLAS handle; the MFMA projection here
// needs no library handle, so this is an empty token that keeps the
// signature.
class BlasHandle {
 public:
  BlasHandle() noexcept = default;
  [[nodiscard]] static Result<BlasHandle> create() noexcept {
    return Result<BlasHandle>::success(BlasHandle());
  }
};
using CublasHandle = BlasHandle;

inline constexpr std::uint32_t restricted_greedy_invalid_token_id = MF_INVALID_TOKEN;

// ---- reference operators (same contracts as marketforge::cuda) ------------

// greedy.hpp:17-21
[[nodiscard]] inline Status greedy_select_f16(const DeviceBuffer& logits, DeviceBuffer& token_ids,
                                              std::uint64_t rows, std::uint64_t vocabulary_size,
                                              StreamHandle stream) noexcept {
  return detail::from_c(
      mf_greedy_select_f16(logits.view(), token_ids.view(), rows, vocabulary_size, stream.value));
}
[[nodiscard]] inline Status greedy_select_f32(const DeviceBuffer& logits, DeviceBuffer& token_ids,
                                              std::uint64_t rows, std::uint64_t vocabulary_size,
                                              StreamHandle stream) noexcept {
  return detail::from_c(
      mf_greedy_select_f32(logits.view(), token_ids.view(), rows, vocabulary_size, stream.value));
}

// greedy.hpp:29-33
[[nodiscard]] inline Status restricted_greedy_select_f16(
    const DeviceBuffer& logits, const DeviceBuffer& allowed_token_ids,
    const DeviceBuffer& allowed_token_counts, DeviceBuffer& token_ids, std::uint64_t rows,
    std::uint64_t vocabulary_size, std::uint64_t maximum_allowed_tokens,
    StreamHandle stream) noexcept {
  return detail::from_c(mf_restricted_greedy_select_f16(
      logits.view(), allowed_token_ids.view(), allowed_token_counts.view(), token_ids.view(),
      rows, vocabulary_size, maximum_allowed_tokens, stream.value));
}
[[nodiscard]] inline Status restricted_greedy_select_f32(
    const DeviceBuffer& logits, const DeviceBuffer& allowed_token_ids,
    const DeviceBuffer& allowed_token_counts, DeviceBuffer& token_ids, std::uint64_t rows,
    std::uint64_t vocabulary_size, std::uint64_t maximum_allowed_tokens,
    StreamHandle stream) noexcept {
  return detail::from_c(mf_restricted_greedy_select_f32(
      logits.view(), allowed_token_ids.view(), allowed_token_counts.view(), token_ids.view(),
      rows, vocabulary_size, maximum_allowed_tokens, stream.value));
}

// greedy.hpp:43-49
[[nodiscard]] inline Status restricted_output_head_f16(
    const DeviceBuffer& hidden, const DeviceBuffer& embedding,
    const DeviceBuffer& allowed_token_ids, const DeviceBuffer& allowed_token_counts,
    DeviceBuffer& token_ids, std::uint64_t rows, std::uint64_t hidden_size,
    std::uint64_t vocabulary_size, std::uint64_t maximum_allowed_tokens,
    StreamHandle stream) noexcept {
  return detail::from_c(mf_restricted_output_head_f16(
      hidden.view(), embedding.view(), allowed_token_ids.view(), allowed_token_counts.view(),
      token_ids.view(), rows, hidden_size, vocabulary_size, maximum_allowed_tokens,
      stream.value));
}

// rms_norm.hpp:18-28
[[nodiscard]] inline Status rms_norm_f32(const DeviceBuffer& input, const DeviceBuffer& weight,
                                         DeviceBuffer& output, std::uint64_t rows,
                                         std::uint64_t hidden_size, float epsilon,
                                         StreamHandle stream) noexcept {
  return detail::from_c(mf_rms_norm_f32(input.view(), weight.view(), output.view(), rows,
                                        hidden_size, epsilon, stream.value));
}
[[nodiscard]] inline Status rms_norm_f16(const DeviceBuffer& input, const DeviceBuffer& weight,
                                         DeviceBuffer& output, std::uint64_t rows,
                                         std::uint64_t hidden_size, float epsilon,
                                         StreamHandle stream) noexcept {
  return detail::from_c(mf_rms_norm_f16(input.view(), weight.view(), output.view(), rows,
                                        hidden_size, epsilon, stream.value));
}

// linear.hpp:18-22
[[nodiscard]] inline Status linear_f16(const DeviceBuffer& input, const DeviceBuffer& weight,
                                       DeviceBuffer& output, std::uint64_t rows,
                                       std::uint64_t input_features,
                                       std::uint64_t output_features, BlasHandle& handle,
                                       StreamHandle stream) noexcept {
  (void)handle;
  return detail::from_c(mf_linear_f16(input.view(), weight.view(), output.view(), rows,
                                      input_features, output_features, stream.value));
}

// ---- the packed decode tail ------------------------------------------------

enum class DotOrder : std::int32_t {
  fma_chain = MF_ORDER_FMA_CHAIN,          // greedy.cu:171-176
  mul_add_chain = MF_ORDER_MUL_ADD_CHAIN,  // operators.cpp:584-595
};

inline constexpr std::uint32_t state_unrestricted = MF_STATE_UNRESTRICTED;
inline constexpr std::uint32_t state_invalid = MF_STATE_INVALID;
// DecodeTailArgs::flags: a row in a state with an empty list (a finished
// sequence) keeps that state instead of becoming invalid.
inline constexpr std::uint64_t tail_hold_finished = MF_TAIL_HOLD_FINISHED;
// DecodeTailArgs::flags: every state's list is strictly ascending (as
// TokenDfa keeps its arcs); a call with unrestricted rows then reads the
// table once for both kinds of rows.  With tail_table_pass as well, so does
// a call without them.  Results are unchanged.
inline constexpr std::uint64_t tail_sorted_lists = MF_TAIL_SORTED_LISTS;
inline constexpr std::uint64_t tail_table_pass = MF_TAIL_TABLE_PASS;
// DecodeTailArgs::flags: packs of short lists without unrestricted rows
// still run the separate kernels instead of the one-kernel tail.
inline constexpr std::uint64_t tail_no_fused = MF_TAIL_NO_FUSED;

// Buffers and shape of one decode-tail call (see marketforge_hip.h); null
// pointers are the optional buffers left out.
struct DecodeTailArgs {
  const DeviceBuffer* x = nullptr;                  // f32 [rows, hidden]
  const DeviceBuffer* norm_weight = nullptr;        // f32 [hidden] or null
  float epsilon = 1e-5f;
  DotOrder order = DotOrder::fma_chain;
  const DeviceBuffer* embedding = nullptr;          // f16 [vocab, hidden]
  const DeviceBuffer* row_state = nullptr;          // u32 [rows]
  const DeviceBuffer* state_offsets = nullptr;      // u32 [states + 1]
  const DeviceBuffer* state_tokens = nullptr;       // u32 [nnz]
  const DeviceBuffer* state_next = nullptr;         // u32 [nnz] or null
  const DeviceBuffer* next_table = nullptr;         // i32 [states, vocab] or null
  const DeviceBuffer* unrestricted_rows = nullptr;  // u32 [unrestricted_count] or null
  DeviceBuffer* out_token = nullptr;                // u32 [rows]
  DeviceBuffer* out_score = nullptr;                // f32 [rows] or null
  DeviceBuffer* out_next_state = nullptr;           // u32 [rows] or null
  std::uint64_t rows = 0;
  std::uint64_t hidden = 0;
  std::uint64_t vocab = 0;
  std::uint64_t states = 0;
  std::uint64_t nnz = 0;
  std::uint64_t max_count = 0;
  std::uint64_t unrestricted_count = 0;
  // Sequence table: row r's state is (*row_state)[(*row_sequence)[r]] and its
  // next state goes to the same index of out_next_state, which may be
  // row_state itself.  Null: row_state and out_next_state hold one entry per row.
  const DeviceBuffer* row_sequence = nullptr;       // u32 [rows] or null
  std::uint64_t flags = 0;                          // tail_hold_finished | tail_sorted_lists | tail_table_pass | tail_no_fused
};

namespace detail {
[[nodiscard]] inline mf_buffer view_or_null(const DeviceBuffer* b) noexcept {
  return b != nullptr ? b->view() : mf_buffer{0, 0};
}
[[nodiscard]] inline mf_decode_tail_args to_c(const DecodeTailArgs& a,
                                              const DeviceBuffer* workspace) noexcept {
  mf_decode_tail_args c{};
  c.x = view_or_null(a.x);
  c.norm_weight = view_or_null(a.norm_weight);
  c.epsilon = a.epsilon;
  c.order = static_cast<std::int32_t>(a.order);
  c.embedding = view_or_null(a.embedding);
  c.row_state = view_or_null(a.row_state);
  c.state_offsets = view_or_null(a.state_offsets);
  c.state_tokens = view_or_null(a.state_tokens);
  c.state_next = view_or_null(a.state_next);
  c.next_table = view_or_null(a.next_table);
  c.unrestricted_rows = view_or_null(a.unrestricted_rows);
  c.out_token = view_or_null(a.out_token);
  c.out_score = view_or_null(a.out_score);
  c.out_next_state = view_or_null(a.out_next_state);
  c.workspace = view_or_null(workspace);
  c.rows = a.rows;
  c.hidden = a.hidden;
  c.vocab = a.vocab;
  c.states = a.states;
  c.nnz = a.nnz;
  c.max_count = a.max_count;
  c.unrestricted_count = a.unrestricted_count;
  c.row_sequence = view_or_null(a.row_sequence);
  c.flags = a.flags;
  return c;
}
}  // namespace detail

// Workspace bytes for decode_tail_f16 (validates the arguments).
[[nodiscard]] inline Result<std::uint64_t> decode_tail_workspace_bytes(
    const DecodeTailArgs& args) noexcept {
  const mf_decode_tail_args c = detail::to_c(args, nullptr);
  std::uint64_t n = 0;
  const Status s = detail::from_c(mf_decode_tail_workspace_bytes(&c, &n));
  if (!s.ok()) return Result<std::uint64_t>::failure(s);
  return Result<std::uint64_t>::success(n);
}

// Zero-fills a workspace once before its first use.
[[nodiscard]] inline Status workspace_init(DeviceBuffer& workspace, StreamHandle stream) noexcept {
  return detail::from_c(mf_workspace_init(workspace.view(), stream.value));
}

// One decode step for the whole pack: norm, restricted gather, MFMA head of
// the unrestricted rows, selection and DFA advance.
[[nodiscard]] inline Status decode_tail_f16(const DecodeTailArgs& args, DeviceBuffer& workspace,
                                            StreamHandle stream) noexcept {
  const mf_decode_tail_args c = detail::to_c(args, &workspace);
  return detail::from_c(mf_decode_tail_f16(&c, stream.value));
}

// ---- token DFA export and the device-resident decode loop -----------------

inline constexpr std::uint32_t no_choice = 0xFFFFFFFFu;

// A token DFA as the decode tail reads it: CSR offsets [S + 1], arc tokens
// and arc next states [A] (the allowed spans of token_dfa.cpp:100-109 laid
// end to end), each state's terminal choice (no_choice otherwise), the
// longest list and the most tokens on a root-to-terminal path.
struct DfaTables {
  std::vector<std::uint32_t> offsets;
  std::vector<std::uint32_t> tokens;
  std::vector<std::uint32_t> next;
  std::vector<std::uint32_t> choice;
  std::uint32_t max_count = 0;
  std::uint32_t depth = 0;

  [[nodiscard]] std::uint64_t states() const noexcept {
    return offsets.empty() ? 0 : offsets.size() - 1;
  }
  [[nodiscard]] std::uint64_t arcs() const noexcept { return tokens.size(); }

  // Checks the layout (offsets frame the arcs, tokens strictly ascending per
  // state and below vocabulary_size, next states in range, no cycle) and
  // fills max_count and depth.  invalid_format when it does not hold.
  [[nodiscard]] Status finish(std::uint64_t vocabulary_size) noexcept {
    const std::uint64_t S = states();
    if (S == 0 || offsets.front() != 0 || offsets.back() != tokens.size() ||
        next.size() != tokens.size() || choice.size() != S) {
      return Status::failure(ErrorCode::invalid_format);
    }
    max_count = 0;
    for (std::uint64_t s = 0; s < S; ++s) {
      if (offsets[s + 1] < offsets[s]) return Status::failure(ErrorCode::invalid_format);
      max_count = std::max<std::uint32_t>(max_count, offsets[s + 1] - offsets[s]);
      for (std::uint32_t i = offsets[s]; i < offsets[s + 1]; ++i) {
        if (tokens[i] >= vocabulary_size || next[i] >= S ||
            (i > offsets[s] && tokens[i] <= tokens[i - 1])) {
          return Status::failure(ErrorCode::invalid_format);
        }
      }
    }
    // breadth-first levels from the root; more levels than states is a cycle
    std::vector<std::uint8_t> in_level(S, 0);
    std::vector<std::uint32_t> level{0}, following;
    depth = 0;
    for (std::uint64_t round = 0;; ++round) {
      following.clear();
      for (const std::uint32_t s : level) {
        for (std::uint32_t i = offsets[s]; i < offsets[s + 1]; ++i) {
          if (!in_level[next[i]]) {
            in_level[next[i]] = 1;
            following.push_back(next[i]);
          }
        }
      }
      for (const std::uint32_t s : following) in_level[s] = 0;
      if (following.empty()) break;
      if (round >= S) return Status::failure(ErrorCode::invalid_format);
      ++depth;
      level.swap(following);
    }
    return Status::success();
  }
};

// Exports a DFA through the reference grammar layer's public queries
// (TokenDfa / ActionDfa: state_count(), root(), allowed(state) returning a
// Result over a span of GrammarArc{token, next}, terminal(state),
// decode_terminal(state); include/marketforge/grammar/token_dfa.hpp:30-74).
// choice_of maps a terminal state to the uint32 the tables store (TokenDfa:
// its ChoiceId; ActionDfa: e.g. the action's catalog index).
template <class Dfa, class ChoiceOf>
[[nodiscard]] Result<DfaTables> export_token_dfa(const Dfa& dfa, std::uint64_t vocabulary_size,
                                                 ChoiceOf choice_of) {
  using State = std::remove_cv_t<decltype(dfa.root())>;
  DfaTables t;
  const std::uint64_t S = dfa.state_count();
  if (S == 0 || S > 0xFFFFFFFEull) return Result<DfaTables>::failure(Status::failure(ErrorCode::resource_limit));
  t.offsets.reserve(S + 1);
  t.choice.assign(S, no_choice);
  for (std::uint64_t s = 0; s < S; ++s) {
    t.offsets.push_back(static_cast<std::uint32_t>(t.tokens.size()));
    const State state{static_cast<std::uint32_t>(s)};
    const auto allowed = dfa.allowed(state);
    if (!allowed) return Result<DfaTables>::failure(Status::failure(ErrorCode::invalid_argument));
    for (const auto& arc : allowed.value()) {
      t.tokens.push_back(arc.token);
      t.next.push_back(arc.next.value);
    }
    if (dfa.terminal(state)) t.choice[s] = choice_of(dfa, state);
  }
  t.offsets.push_back(static_cast<std::uint32_t>(t.tokens.size()));
  const Status st = t.finish(vocabulary_size);
  if (!st.ok()) return Result<DfaTables>::failure(st);
  return Result<DfaTables>::success(std::move(t));
}

// TokenDfa: the terminal's ChoiceId.
template <class Dfa>
[[nodiscard]] Result<DfaTables> export_token_dfa(const Dfa& dfa, std::uint64_t vocabulary_size) {
  return export_token_dfa(dfa, vocabulary_size, [](const Dfa& d, auto state) {
    const auto c = d.decode_terminal(state);
    return c ? static_cast<std::uint32_t>(c.value()) : no_choice;
  });
}

namespace detail {
template <typename T>
[[nodiscard]] inline Result<DeviceBuffer> upload_vector(const std::vector<T>& host,
                                                        StreamHandle stream) noexcept {
  // a zero-length list still gets a valid (4-byte) buffer
  const std::uint64_t n = host.empty() ? sizeof(T) : host.size() * sizeof(T);
  auto b = DeviceBuffer::allocate(n);
  if (!b || host.empty()) return b;
  const Status s = b.value().copy_from_host_async(host.data(), n, 0, stream);
  if (!s.ok()) return Result<DeviceBuffer>::failure(s);
  return b;
}
}  // namespace detail

// The tables on the device (offsets, tokens, next); the terminal choices
// stay on the host.  upload() synchronizes the stream once (the host
// vectors are copied by then).
class DeviceDfa {
 public:
  [[nodiscard]] static Result<DeviceDfa> upload(DfaTables tables, StreamHandle stream) noexcept {
    DeviceDfa d;
    auto o = detail::upload_vector(tables.offsets, stream);
    auto t = detail::upload_vector(tables.tokens, stream);
    auto n = detail::upload_vector(tables.next, stream);
    if (!o) return Result<DeviceDfa>::failure(o.status());
    if (!t) return Result<DeviceDfa>::failure(t.status());
    if (!n) return Result<DeviceDfa>::failure(n.status());
    const Status s = detail::from_c(mf_stream_synchronize(stream.value));
    if (!s.ok()) return Result<DeviceDfa>::failure(s);
    d.offsets_ = std::move(o).value();
    d.tokens_ = std::move(t).value();
    d.next_ = std::move(n).value();
    d.tables_ = std::move(tables);
    return Result<DeviceDfa>::success(std::move(d));
  }
  [[nodiscard]] const DfaTables& tables() const noexcept { return tables_; }
  [[nodiscard]] const DeviceBuffer& offsets() const noexcept { return offsets_; }
  [[nodiscard]] const DeviceBuffer& tokens() const noexcept { return tokens_; }
  [[nodiscard]] const DeviceBuffer& next() const noexcept { return next_; }

 private:
  DfaTables tables_;
  DeviceBuffer offsets_, tokens_, next_;
};

// What a decode loop produced: tokens [steps x rows] (row-major by step;
// MF_INVALID_TOKEN after a row has finished), the final states and their
// terminal choices.
struct DecodeOutput {
  std::uint64_t steps = 0;
  std::uint64_t rows = 0;
  std::vector<std::uint32_t> tokens;
  std::vector<std::uint32_t> states;
  std::vector<std::uint32_t> choice;
};

// Greedy restricted decoding of `rows` sequences in lock step with the DFA
// state on the device: step() enqueues one decode-tail call (states alternate
// between two device buffers, finished rows hold their terminal state) and
// never synchronizes; finish() synchronizes once and copies every step's
// tokens.  The replacement of the reference's per-token
// CudaSmolLm2::decode_restricted round trip (src/cuda/smollm2.cu:336-366).
class RestrictedDecoder {
 public:
  struct Config {
    std::uint64_t rows = 0;
    std::uint64_t hidden = 0;
    std::uint64_t vocab = 0;
    std::uint64_t max_steps = 0;
    float epsilon = 1e-5f;
    DotOrder order = DotOrder::fma_chain;
    // false: the separate kernels even where the one-kernel tail applies
    bool fused = true;
  };

  // embedding, norm_weight (null: hidden rows arrive normalized) and dfa
  // are borrowed and must outlive the decoder.
  [[nodiscard]] static Result<RestrictedDecoder> create(const DeviceBuffer& embedding,
                                                        const DeviceBuffer* norm_weight,
                                                        const DeviceDfa& dfa, Config config,
                                                        StreamHandle stream) noexcept {
    RestrictedDecoder d;
    d.config_ = config;
    d.dfa_ = &dfa;
    if (config.rows == 0 || config.max_steps == 0) {
      return Result<RestrictedDecoder>::failure(Status::failure(ErrorCode::invalid_argument));
    }
    auto states = DeviceBuffer::allocate(2 * config.rows * 4);
    auto tokens = DeviceBuffer::allocate(config.max_steps * config.rows * 4);
    auto scores = DeviceBuffer::allocate(config.max_steps * config.rows * 4);
    if (!states) return Result<RestrictedDecoder>::failure(states.status());
    if (!tokens) return Result<RestrictedDecoder>::failure(tokens.status());
    if (!scores) return Result<RestrictedDecoder>::failure(scores.status());
    d.states_ = std::move(states).value();
    d.tokens_ = std::move(tokens).value();
    d.scores_ = std::move(scores).value();
    for (int parity = 0; parity < 2; ++parity) {
      mf_decode_tail_args& a = d.args_[parity];
      a = mf_decode_tail_args{};
      a.x = mf_buffer{256, config.rows * config.hidden * 4};  // set per step
      a.norm_weight = norm_weight != nullptr ? norm_weight->view() : mf_buffer{0, 0};
      a.epsilon = config.epsilon;
      a.order = static_cast<std::int32_t>(config.order);
      a.embedding = embedding.view();
      a.row_state = d.state_view(parity);
      a.state_offsets = dfa.offsets().view();
      a.state_tokens = dfa.tokens().view();
      a.state_next = dfa.next().view();
      a.out_token = d.step_view(d.tokens_, 0);
      a.out_score = d.step_view(d.scores_, 0);
      a.out_next_state = d.state_view(1 - parity);
      a.rows = config.rows;
      a.hidden = config.hidden;
      a.vocab = config.vocab;
      a.states = dfa.tables().states();
      a.nnz = dfa.tables().arcs();
      a.max_count = dfa.tables().max_count;
      a.flags = MF_TAIL_HOLD_FINISHED | (config.fused ? 0u : MF_TAIL_NO_FUSED);
    }
    std::uint64_t ws = 0;
    Status s = detail::from_c(mf_decode_tail_workspace_bytes(&d.args_[0], &ws));
    if (!s.ok()) return Result<RestrictedDecoder>::failure(s);
    auto workspace = DeviceBuffer::allocate(ws);
    if (!workspace) return Result<RestrictedDecoder>::failure(workspace.status());
    d.workspace_ = std::move(workspace).value();
    d.args_[0].workspace = d.args_[1].workspace = d.workspace_.view();
    s = workspace_init(d.workspace_, stream);
    if (!s.ok()) return Result<RestrictedDecoder>::failure(s);
    return Result<RestrictedDecoder>::success(std::move(d));
  }

  // Every row at the DFA root (states == nullptr) or at states[0..rows).
  // The host array must stay valid until the stream reaches the copy.
  [[nodiscard]] Status start(const std::uint32_t* states, StreamHandle stream) noexcept {
    step_ = 0;
    if (states != nullptr) {
      return states_.copy_from_host_async(states, config_.rows * 4, 0, stream);
    }
    root_.assign(config_.rows, 0u);
    return states_.copy_from_host_async(root_.data(), config_.rows * 4, 0, stream);
  }

  // One decode step: hidden is this step's FP32 [rows, hidden] (a view, e.g.
  // a slice of a larger buffer).
  [[nodiscard]] Status step(mf_buffer hidden, StreamHandle stream) noexcept {
    if (step_ >= config_.max_steps) return Status::failure(ErrorCode::resource_limit);
    mf_decode_tail_args& a = args_[step_ % 2];
    a.x = hidden;
    a.out_token = step_view(tokens_, step_);
    a.out_score = step_view(scores_, step_);
    const Status s = detail::from_c(mf_decode_tail_f16(&a, stream.value));
    if (s.ok()) ++step_;
    return s;
  }

  [[nodiscard]] std::uint64_t steps() const noexcept { return step_; }
  // For callers that capture steps into a graph and replay it after start():
  // the buffers now hold k steps (k <= max_steps).
  void assume_steps(std::uint64_t k) noexcept { step_ = std::min(k, config_.max_steps); }
  // The states after the last step (device view).
  [[nodiscard]] mf_buffer current_states() const noexcept { return state_view(step_ % 2); }

  // Synchronizes once and copies the tokens of every step so far, the final
  // states and their terminal choices.
  [[nodiscard]] Result<DecodeOutput> finish(StreamHandle stream) {
    DecodeOutput out;
    out.steps = step_;
    out.rows = config_.rows;
    out.tokens.resize(step_ * config_.rows);
    out.states.resize(config_.rows);
    Status s = Status::success();
    if (step_ > 0) s = tokens_.copy_to_host_async(out.tokens.data(), step_ * config_.rows * 4, 0, stream);
    if (s.ok())
      s = states_.copy_to_host_async(out.states.data(), config_.rows * 4,
                                     (step_ % 2) * config_.rows * 4, stream);
    if (s.ok()) s = detail::from_c(mf_stream_synchronize(stream.value));
    if (!s.ok()) return Result<DecodeOutput>::failure(s);
    out.choice.assign(config_.rows, no_choice);
    const DfaTables& t = dfa_->tables();
    for (std::uint64_t r = 0; r < config_.rows; ++r) {
      if (out.states[r] < t.states()) out.choice[r] = t.choice[out.states[r]];
    }
    return Result<DecodeOutput>::success(std::move(out));
  }

 private:
  [[nodiscard]] mf_buffer state_view(std::uint64_t parity) const noexcept {
    return mf_buffer{states_.address().value + parity * config_.rows * 4, config_.rows * 4};
  }
  [[nodiscard]] mf_buffer step_view(const DeviceBuffer& b, std::uint64_t k) const noexcept {
    return mf_buffer{b.address().value + k * config_.rows * 4, config_.rows * 4};
  }

  Config config_{};
  const DeviceDfa* dfa_ = nullptr;
  DeviceBuffer states_, tokens_, scores_, workspace_;
  mf_decode_tail_args args_[2]{};
  std::vector<std::uint32_t> root_;
  std::uint64_t step_ = 0;
};

}  // namespace marketforge::gpu
