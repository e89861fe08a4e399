// The reference's invalid-metadata operator tests, through the operator shim
// (market_sim_amd/shim/operators_shim.cpp) built against the reference's own
// headers.  Cases restated from tests/cuda/cuda_tests.cu:
//   rms_norm_rejects_invalid_metadata_before_launch         :914-945
//   linear_f16_rejects_invalid_metadata_before_cublas       :952-997
//   greedy_f16_rejects_invalid_metadata_before_launch       :1137-1166
//   restricted_output_head_f16_rejects_invalid_metadata     :1283-1339
//
// Every case is rejected by host-side validation before any device work, so
// the harness runs without a GPU: it supplies host stand-ins for the
// library's allocation and stream entry points (the definitions in this
// executable take the place of the library's), giving the buffers distinct
// addresses that nothing dereferences.  With a GPU present it exits 77
// (skipped) rather than hand such addresses to a device.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <utility>

#include "marketforge/cuda/cublas_handle.hpp"
#include "marketforge/cuda/cuda_stream.hpp"
#include "marketforge/cuda/device_buffer.hpp"
#include "marketforge/cuda/greedy.hpp"
#include "marketforge/cuda/linear.hpp"
#include "marketforge/cuda/rms_norm.hpp"
#include "marketforge_hip.h"

extern "C" {
mf_status mf_device_alloc(uint64_t bytes, uintptr_t* address) {
  void* p = std::aligned_alloc(256, (bytes + 255) / 256 * 256);
  if (p == nullptr) return mf_status{MF_ALLOCATION_FAILED, 0};
  *address = reinterpret_cast<uintptr_t>(p);
  return mf_status{MF_OK, 0};
}
mf_status mf_device_free(uintptr_t address) {
  std::free(reinterpret_cast<void*>(address));
  return mf_status{MF_OK, 0};
}
mf_status mf_stream_create(uintptr_t* stream) {
  *stream = 0x5157u;
  return mf_status{MF_OK, 0};
}
mf_status mf_stream_destroy(uintptr_t) { return mf_status{MF_OK, 0}; }
mf_status mf_stream_synchronize(uintptr_t) { return mf_status{MF_OK, 0}; }
}

namespace {

using marketforge::ErrorCode;
using marketforge::cuda::CublasHandle;
using marketforge::cuda::CudaStream;
using marketforge::cuda::DeviceBuffer;

int failures = 0;
int checks = 0;

void expect(const char* name, ErrorCode got, ErrorCode want) {
  ++checks;
  if (got != want) {
    ++failures;
    std::printf("FAIL %s: code %d, want %d\n", name, static_cast<int>(got), static_cast<int>(want));
  }
}

DeviceBuffer buffer(std::uint64_t bytes) {
  auto r = DeviceBuffer::allocate(bytes);
  if (!r) {
    std::printf("allocation failed\n");
    std::exit(2);
  }
  return std::move(r).value();
}

CudaStream stream_or_die() {
  auto r = CudaStream::create();
  if (!r) {
    std::printf("stream creation failed\n");
    std::exit(2);
  }
  return std::move(r).value();
}

void rms_norm_cases() {
  CudaStream stream = stream_or_die();
  DeviceBuffer input = buffer(8 * sizeof(float));
  DeviceBuffer weight = buffer(4 * sizeof(float));
  DeviceBuffer output = buffer(8 * sizeof(float));
  using marketforge::cuda::rms_norm_f32;
  expect("rms_norm rows 0", rms_norm_f32(input, weight, output, 0, 4, 1.0e-5F, stream.handle()).code,
         ErrorCode::invalid_argument);
  expect("rms_norm NaN epsilon",
         rms_norm_f32(input, weight, output, 2, 4, std::numeric_limits<float>::quiet_NaN(), stream.handle())
             .code,
         ErrorCode::invalid_argument);
  expect("rms_norm no stream", rms_norm_f32(input, weight, output, 2, 4, 1.0e-5F, {}).code,
         ErrorCode::invalid_argument);
  expect("rms_norm size mismatch", rms_norm_f32(input, weight, output, 1, 4, 1.0e-5F, stream.handle()).code,
         ErrorCode::invalid_argument);
}

void linear_cases() {
  CudaStream stream = stream_or_die();
  auto handle_result = CublasHandle::create();
  if (!handle_result) std::exit(2);
  CublasHandle handle = std::move(handle_result).value();
  DeviceBuffer input = buffer(6 * 2);
  DeviceBuffer weight = buffer(6 * 2);
  DeviceBuffer output = buffer(4 * 2);
  using marketforge::cuda::linear_f16;
  expect("linear rows 0", linear_f16(input, weight, output, 0, 3, 2, handle, stream.handle()).code,
         ErrorCode::invalid_argument);
  expect("linear no stream", linear_f16(input, weight, output, 2, 3, 2, handle, {}).code,
         ErrorCode::invalid_argument);
  CublasHandle empty_handle;
  expect("linear empty handle", linear_f16(input, weight, output, 2, 3, 2, empty_handle, stream.handle()).code,
         ErrorCode::invalid_argument);
  expect("linear size mismatch", linear_f16(input, weight, output, 1, 3, 2, handle, stream.handle()).code,
         ErrorCode::invalid_argument);
  expect("linear output aliases input", linear_f16(input, weight, input, 2, 3, 2, handle, stream.handle()).code,
         ErrorCode::invalid_argument);
  expect("linear rows overflow",
         linear_f16(input, weight, output, std::numeric_limits<std::uint64_t>::max(), 2, 2, handle,
                    stream.handle())
             .code,
         ErrorCode::arithmetic_overflow);
}

void greedy_cases() {
  CudaStream stream = stream_or_die();
  DeviceBuffer logits = buffer(8 * 2);
  DeviceBuffer tokens = buffer(sizeof(std::uint32_t));
  using marketforge::cuda::greedy_select_f16;
  expect("greedy rows 0", greedy_select_f16(logits, tokens, 0, 8, stream.handle()).code,
         ErrorCode::invalid_argument);
  expect("greedy no stream", greedy_select_f16(logits, tokens, 1, 8, {}).code, ErrorCode::invalid_argument);
  expect("greedy size mismatch", greedy_select_f16(logits, tokens, 1, 7, stream.handle()).code,
         ErrorCode::invalid_argument);
  expect("greedy vocabulary above uint32",
         greedy_select_f16(logits, tokens, 1,
                           static_cast<std::uint64_t>(std::numeric_limits<std::uint32_t>::max()) + 1,
                           stream.handle())
             .code,
         ErrorCode::resource_limit);
}

void restricted_output_head_cases() {
  constexpr std::uint64_t rows = 1;
  constexpr std::uint64_t hidden_size = 4;
  constexpr std::uint64_t vocabulary_size = 8;
  constexpr std::uint64_t maximum_allowed = 2;
  CudaStream stream = stream_or_die();
  DeviceBuffer hidden = buffer(rows * hidden_size * 2);
  DeviceBuffer embedding = buffer(vocabulary_size * hidden_size * 2);
  DeviceBuffer allowed = buffer(rows * maximum_allowed * sizeof(std::uint32_t));
  DeviceBuffer counts = buffer(rows * sizeof(std::uint32_t));
  DeviceBuffer output = buffer(rows * sizeof(std::uint32_t));
  using marketforge::cuda::restricted_output_head_f16;
  expect("head rows 0",
         restricted_output_head_f16(hidden, embedding, allowed, counts, output, 0, hidden_size,
                                    vocabulary_size, maximum_allowed, stream.handle())
             .code,
         ErrorCode::invalid_argument);
  expect("head maximum_allowed 0",
         restricted_output_head_f16(hidden, embedding, allowed, counts, output, rows, hidden_size,
                                    vocabulary_size, 0, stream.handle())
             .code,
         ErrorCode::invalid_argument);
  expect("head no stream",
         restricted_output_head_f16(hidden, embedding, allowed, counts, output, rows, hidden_size,
                                    vocabulary_size, maximum_allowed, {})
             .code,
         ErrorCode::invalid_argument);
  expect("head output aliases counts",
         restricted_output_head_f16(hidden, embedding, allowed, counts, counts, rows, hidden_size,
                                    vocabulary_size, maximum_allowed, stream.handle())
             .code,
         ErrorCode::invalid_argument);
  expect("head rows above int",
         restricted_output_head_f16(hidden, embedding, allowed, counts, output,
                                    std::numeric_limits<std::uint64_t>::max(), hidden_size,
                                    vocabulary_size, maximum_allowed, stream.handle())
             .code,
         ErrorCode::resource_limit);
}

}  // namespace

int main() {
  int32_t devices = 0;
  const mf_status s = mf_device_count(&devices);
  if (s.code == MF_OK && devices > 0) {
    std::printf("a GPU is present: skipped (host stand-in addresses are for machines without one)\n");
    return 77;
  }
  rms_norm_cases();
  linear_cases();
  greedy_cases();
  restricted_output_head_cases();
  std::printf("%d checks, %d failures\n", checks, failures);
  return failures == 0 ? 0 : 1;
}
