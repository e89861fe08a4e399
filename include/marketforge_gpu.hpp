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
// Everything is noexcept and allocation-free except DeviceBuffer::allocate and
// the stream/handle factories; ops never synchronize.
#pragma once

#include <cstdint>
#include <optional>
#include <utility>

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

}  // namespace marketforge::gpu
