// The reference's CUDA operator layer on MI355X: one translation unit that
// replaces src/cuda/device_buffer.cu, src/cuda/cuda_stream.cu,
// src/cuda/cublas_handle.cu, src/cuda/greedy.cu, src/cuda/rms_norm.cu and
// src/cuda/linear.cu in a ROCm build of the reference.  It keeps the
// reference's headers (include/marketforge/cuda/{device_buffer,cuda_stream,
// cublas_handle,greedy,rms_norm,linear}.hpp) and forwards every call to
// libmarketforge_hip's C ABI (include/marketforge_hip.h), whose validation
// follows the reference's order and error codes.
//
// Build: add <repo>/include to the include path next to the reference's
// include/, link -L<repo>/market_sim_amd/lib -lmarketforge_hip.
#include <cstdint>
#include <utility>

#include "marketforge/cuda/cublas_handle.hpp"
#include "marketforge/cuda/cuda_stream.hpp"
#include "marketforge/cuda/device_buffer.hpp"
#include "marketforge/cuda/greedy.hpp"
#include "marketforge/cuda/linear.hpp"
#include "marketforge/cuda/rms_norm.hpp"
#include "marketforge_hip.h"

namespace marketforge::cuda {
namespace {

mf_buffer view(const DeviceBuffer& b) noexcept { return mf_buffer{b.address().value, b.size_bytes()}; }

// mf_status codes number ErrorCode one to one (include/marketforge_hip.h).
Status status(mf_status s) noexcept {
  if (s.code == MF_OK) return Status::success();
  return Status::failure(static_cast<ErrorCode>(s.code), s.detail);
}

}  // namespace

// ---- DeviceBuffer (device_buffer.cu) ---------------------------------------

Result<DeviceBuffer> DeviceBuffer::allocate(const std::uint64_t byte_count) noexcept {
  if (byte_count == 0) return Result<DeviceBuffer>::success(DeviceBuffer{});
  std::uintptr_t address = 0;
  const mf_status s = mf_device_alloc(byte_count, &address);
  if (s.code != MF_OK) return Result<DeviceBuffer>::failure(status(s));
  return Result<DeviceBuffer>::success(DeviceBuffer(DeviceAddress{address}, byte_count));
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept
    : address_(std::exchange(other.address_, {})), size_bytes_(std::exchange(other.size_bytes_, 0)) {}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
  if (this != &other) {
    release();
    address_ = std::exchange(other.address_, {});
    size_bytes_ = std::exchange(other.size_bytes_, 0);
  }
  return *this;
}

DeviceBuffer::~DeviceBuffer() noexcept { release(); }

Status DeviceBuffer::copy_from_host_async(const void* source, const std::uint64_t byte_count,
                                          const std::uint64_t offset,
                                          const StreamHandle stream) noexcept {
  return status(mf_copy_to_device_async(view(*this), offset, source, byte_count, stream.value));
}

Status DeviceBuffer::copy_to_host_async(void* destination, const std::uint64_t byte_count,
                                        const std::uint64_t offset,
                                        const StreamHandle stream) const noexcept {
  return status(mf_copy_to_host_async(destination, view(*this), offset, byte_count, stream.value));
}

void DeviceBuffer::release() noexcept {
  const std::uintptr_t address = address_.value;
  address_ = {};
  size_bytes_ = 0;
  if (address != 0) (void)mf_device_free(address);
}

// ---- CudaStream (cuda_stream.cu): a non-blocking HIP stream ----------------

Result<CudaStream> CudaStream::create() noexcept {
  std::uintptr_t handle = 0;
  const mf_status s = mf_stream_create(&handle);
  if (s.code != MF_OK) return Result<CudaStream>::failure(status(s));
  return Result<CudaStream>::success(CudaStream(StreamHandle{handle}));
}

CudaStream::CudaStream(CudaStream&& other) noexcept : handle_(std::exchange(other.handle_, {})) {}

CudaStream& CudaStream::operator=(CudaStream&& other) noexcept {
  if (this != &other) {
    release();
    handle_ = std::exchange(other.handle_, {});
  }
  return *this;
}

CudaStream::~CudaStream() noexcept { release(); }

Status CudaStream::synchronize() const noexcept {
  if (!handle_.valid()) return Status::failure(ErrorCode::invalid_argument);
  return status(mf_stream_synchronize(handle_.value));
}

void CudaStream::release() noexcept {
  const std::uintptr_t handle = handle_.value;
  handle_ = {};
  if (handle != 0) (void)mf_stream_destroy(handle);
}

// ---- CublasHandle (cublas_handle.cu) ---------------------------------------
// The projection is this library's own MFMA kernel and needs no library
// handle; the handle only keeps the reference's "valid handle" contract
// (linear_f16 rejects an empty one), so it holds a non-zero token and owns
// nothing.

Result<CublasHandle> CublasHandle::create() noexcept {
  return Result<CublasHandle>::success(CublasHandle(CublasHandleValue{1}));
}

CublasHandle::CublasHandle(CublasHandle&& other) noexcept : handle_(std::exchange(other.handle_, {})) {}

CublasHandle& CublasHandle::operator=(CublasHandle&& other) noexcept {
  if (this != &other) {
    release();
    handle_ = std::exchange(other.handle_, {});
  }
  return *this;
}

CublasHandle::~CublasHandle() noexcept { release(); }

void CublasHandle::release() noexcept { handle_ = {}; }

// ---- operators (greedy.cu, rms_norm.cu, linear.cu) --------------------------

Status greedy_select_f16(const DeviceBuffer& logits, DeviceBuffer& token_ids, std::uint64_t rows,
                         std::uint64_t vocabulary_size, StreamHandle stream) noexcept {
  return status(mf_greedy_select_f16(view(logits), view(token_ids), rows, vocabulary_size, stream.value));
}

Status restricted_greedy_select_f16(const DeviceBuffer& logits, const DeviceBuffer& allowed_token_ids,
                                    const DeviceBuffer& allowed_token_counts, DeviceBuffer& token_ids,
                                    std::uint64_t rows, std::uint64_t vocabulary_size,
                                    std::uint64_t maximum_allowed_tokens, StreamHandle stream) noexcept {
  return status(mf_restricted_greedy_select_f16(view(logits), view(allowed_token_ids),
                                                view(allowed_token_counts), view(token_ids), rows,
                                                vocabulary_size, maximum_allowed_tokens, stream.value));
}

Status restricted_output_head_f16(const DeviceBuffer& hidden, const DeviceBuffer& embedding,
                                  const DeviceBuffer& allowed_token_ids,
                                  const DeviceBuffer& allowed_token_counts, DeviceBuffer& token_ids,
                                  std::uint64_t rows, std::uint64_t hidden_size,
                                  std::uint64_t vocabulary_size, std::uint64_t maximum_allowed_tokens,
                                  StreamHandle stream) noexcept {
  return status(mf_restricted_output_head_f16(view(hidden), view(embedding), view(allowed_token_ids),
                                              view(allowed_token_counts), view(token_ids), rows,
                                              hidden_size, vocabulary_size, maximum_allowed_tokens,
                                              stream.value));
}

Status rms_norm_f32(const DeviceBuffer& input, const DeviceBuffer& weight, DeviceBuffer& output,
                    std::uint64_t rows, std::uint64_t hidden_size, float epsilon,
                    StreamHandle stream) noexcept {
  return status(mf_rms_norm_f32(view(input), view(weight), view(output), rows, hidden_size, epsilon,
                                stream.value));
}

Status rms_norm_f16(const DeviceBuffer& input, const DeviceBuffer& weight, DeviceBuffer& output,
                    std::uint64_t rows, std::uint64_t hidden_size, float epsilon,
                    StreamHandle stream) noexcept {
  return status(mf_rms_norm_f16(view(input), view(weight), view(output), rows, hidden_size, epsilon,
                                stream.value));
}

Status linear_f16(const DeviceBuffer& input, const DeviceBuffer& weight, DeviceBuffer& output,
                  std::uint64_t rows, std::uint64_t input_features, std::uint64_t output_features,
                  CublasHandle& handle, StreamHandle stream) noexcept {
  // the reference checks the handle first (linear.cu:45-47)
  if (!handle.handle().valid()) return Status::failure(ErrorCode::invalid_argument);
  return status(mf_linear_f16(view(input), view(weight), view(output), rows, input_features,
                              output_features, stream.value));
}

}  // namespace marketforge::cuda
