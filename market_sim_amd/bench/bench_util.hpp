// Helpers shared by the benchmark programs over the C++ operator layer:
// HIP-event timing with the reference benches' protocol, uploads, the DFA
// table file of market_sim_amd.dfa.write_tables, reference-order host
// arithmetic for the parity checks.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "marketforge_gpu.hpp"

namespace bench {

namespace mg = marketforge::gpu;

inline bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return false;
}

inline bool status_ok(const mg::Status& s, const char* what) {
  if (s.ok()) return true;
  std::fprintf(stderr, "%s: error code %u detail %u\n", what, static_cast<unsigned>(s.code),
               s.detail);
  return false;
}

// `warmup` untimed launches, a stream synchronization, then one event pair
// around `iterations` back-to-back launches; the average microseconds per
// launch, or a negative value on failure.
template <typename Launch>
double time_launches(const mg::GpuStream& stream, std::uint32_t warmup, std::uint32_t iterations,
                     Launch launch) {
  for (std::uint32_t i = 0; i < warmup; ++i)
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
  const auto s =
      b.value().copy_from_host_async(host.data(), host.size() * sizeof(T), 0, stream.handle());
  if (!s.ok()) return mg::Result<mg::DeviceBuffer>::failure(s);
  return b;
}

template <typename T>
bool download(std::vector<T>& host, const mg::DeviceBuffer& device, const mg::GpuStream& stream) {
  return status_ok(device.copy_to_host_async(host.data(), host.size() * sizeof(T), 0,
                                             stream.handle()),
                   "copy_to_host") &&
         status_ok(stream.synchronize(), "synchronize");
}

// IEEE binary16 <-> binary32, round to nearest even.
inline std::uint16_t to_half(float value) {
  std::uint32_t x;
  std::memcpy(&x, &value, 4);
  const std::uint32_t sign = (x >> 16) & 0x8000u, mag = x & 0x7FFFFFFFu;
  if (mag >= 0x7F800000u)
    return static_cast<std::uint16_t>(sign | 0x7C00u | (mag > 0x7F800000u ? 0x200u : 0u));
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
inline float from_half(std::uint16_t h) {
  const std::uint32_t sign = (static_cast<std::uint32_t>(h) & 0x8000u) << 16;
  const std::uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  std::uint32_t bits;
  if (e == 0) {
    const float v = static_cast<float>(m) * 0x1p-24f;
    std::memcpy(&bits, &v, 4);
    bits |= sign;
  } else if (e == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

// The DFA table file of market_sim_amd.dfa.write_tables: magic "MDF1",
// state count, arc count, then offsets, tokens, next states, choices.
inline bool read_tables(const char* path, mg::DfaTables& t, std::uint64_t vocab) {
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
  return good && t.finish(vocab).ok();
}

inline void print_gpu(std::FILE* out) {
  hipDeviceProp_t p{};
  if (hipGetDeviceProperties(&p, 0) != hipSuccess) {
    std::fprintf(out, "\"gpu\":{\"name\":\"unknown\",\"compute_capability\":\"0.0\"}");
    return;
  }
  // (the marketing name can be empty on a box: the architecture names it then)
  std::string name = p.name;
  if (name.empty()) {
    const std::string arch = p.gcnArchName;
    name = "AMD " + arch.substr(0, arch.find(':'));
  }
  std::fprintf(out, "\"gpu\":{\"name\":\"%s\",\"compute_capability\":\"%d.%d\"}",
               name.c_str(), p.major, p.minor);
}

}  // namespace bench
