// Host-side device plumbing shared by the generator and codec engines:
// grow-only device buffers and the per-launch event profiler.
#ifndef OMNIVOICE_AMD_DEVICE_HPP_
#define OMNIVOICE_AMD_DEVICE_HPP_

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "kernels.hpp"

namespace ovg {

template <typename T>
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  ~DeviceBuffer() { Release(); }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;

  // Grows to `count` elements (contents are lost, new memory is zeroed);
  // returns true when it reallocated. The zeroing runs on the null stream,
  // which work on a non-blocking stream does not wait for, so the null
  // stream is waited for here (and only it, not the other engines' streams):
  // otherwise the zeroing could land after that work's first writes.
  bool Reserve(std::size_t count) {
    if (count <= count_)
      return false;
    Release();
    Check(hipMalloc(reinterpret_cast<void**>(&data_),
                    std::max<std::size_t>(count, 1) * sizeof(T)),
          "hipMalloc");
    Check(hipMemset(data_, 0, std::max<std::size_t>(count, 1) * sizeof(T)),
          "hipMemset");
    Check(hipStreamSynchronize(nullptr), "hipMemset");
    count_ = count;
    return true;
  }
  T* get() const { return data_; }
  std::size_t size() const { return count_; }
  std::size_t bytes() const { return count_ * sizeof(T); }

 private:
  void Release() {
    if (data_ != nullptr)
      (void)hipFree(data_);
    data_ = nullptr;
    count_ = 0;
  }
  T* data_ = nullptr;
  std::size_t count_ = 0;
};

struct KernelStat {
  std::int64_t launches = 0;
  double ms = 0.0, flops = 0.0, bytes = 0.0;
};

// Records HIP events around each launch of an eager sequence.
class Profiler {
 public:
  explicit Profiler(hipStream_t stream) : stream_(stream) {}
  ~Profiler() {
    for (auto& e : entries_) {
      (void)hipEventDestroy(e.begin);
      (void)hipEventDestroy(e.end);
    }
  }
  template <typename F>
  void Run(const char* name, double flops, double bytes, F&& launch) {
    Entry e;
    e.name = name;
    e.flops = flops;
    e.bytes = bytes;
    Check(hipEventCreate(&e.begin), "hipEventCreate");
    Check(hipEventCreate(&e.end), "hipEventCreate");
    // The launcher's kernels record the events themselves (CurrentTiming).
    CurrentTiming() = LaunchTiming{e.begin, e.end};
    try {
      launch();
    } catch (...) {
      CurrentTiming() = LaunchTiming{};
      throw;
    }
    CurrentTiming() = LaunchTiming{};
    entries_.push_back(e);
  }
  void Collect(std::map<std::string, KernelStat>* stats) {
    Check(hipStreamSynchronize(stream_), "profile");
    for (const auto& e : entries_) {
      float ms = 0.0F;
      Check(hipEventElapsedTime(&ms, e.begin, e.end), "hipEventElapsedTime");
      KernelStat& s = (*stats)[e.name];
      s.launches += 1;
      s.ms += ms;
      s.flops += e.flops;
      s.bytes += e.bytes;
    }
  }

 private:
  struct Entry {
    std::string name;
    double flops = 0, bytes = 0;
    hipEvent_t begin = nullptr, end = nullptr;
  };
  hipStream_t stream_;
  std::vector<Entry> entries_;
};

}  // namespace ovg

#endif  // OMNIVOICE_AMD_DEVICE_HPP_
