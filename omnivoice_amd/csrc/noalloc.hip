// ovg_op_linear_noalloc: ovg_op_linear (the generator's GEMM behind the C
// ABI) without any device allocation, for callers that cannot allocate:
// code under HIP graph capture, serving loops that forbid hipMalloc.
//
// The only device memory ovg_op_linear allocates is the split-K partials of
// small-M shapes (the second launch sums them in split order). Here they
// live in `scratch`, a file-scope device array of kScratchFloats floats
// (4 MiB per GPU, held until the process ends). Every shape ovg_op_linear
// accepts needs at most 1032192 of them (1 row by 8064 outputs by 1024
// inputs: 63 tiles of 32 rows in 4 splits); a plan that needed more would be
// rejected with an error. The partials are written in full before they are
// read, so nothing needs clearing between calls. All calls on one GPU share
// its array: calls that overlap on one GPU (two streams, two threads) race.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/omnivoice_mi355x.h"
#include "kernels.hpp"

namespace {

constexpr std::size_t kScratchFloats = std::size_t{1} << 20;
static_assert(kScratchFloats == OVG_LINEAR_NOALLOC_SCRATCH_FLOATS,
              "the header states the scratch size");

}  // namespace

// The device array itself. In host code its name is only a stand-in for the
// symbol: the device address is taken per GPU with hipGetSymbolAddress.
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
float* scratch_address[kMaxDevices] = {};

// The current GPU's copy of `scratch`, looked up once per device with that
// device current.
float* DeviceScratch() {
  int device = 0;
  ovg::Check(hipGetDevice(&device), "hipGetDevice");
  ovg::Require(device >= 0 && device < kMaxDevices, "device index out of range");
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_address[device] == nullptr) {
    void* address = nullptr;
    ovg::Check(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)),
               "hipGetSymbolAddress(scratch)");
    ovg::Require(address != nullptr, "no device address for the scratch array");
    scratch_address[device] = static_cast<float*>(address);
  }
  return scratch_address[device];
}

void SetError(char* error, std::size_t len, const std::string& message) {
  if (error == nullptr || len == 0)
    return;
  const std::size_t n = std::min(len - 1, message.size());
  std::memcpy(error, message.data(), n);
  error[n] = '\0';
}

bool FitsInt(int64_t v) { return v >= 0 && v <= (int64_t{1} << 30); }

}  // namespace

extern "C" int ovg_op_linear_noalloc(const void* x, const void* w, float* y, int64_t rows,
                                     int64_t in, int64_t out, int accumulate, void* stream,
                                     char* error, size_t error_len) {
  try {
    ovg::Require(x && w && y, "null pointer");
    ovg::Require(rows >= 1 && in >= 64 && out >= 1 && FitsInt(rows) && FitsInt(in) &&
                     FitsInt(out),
                 "empty or oversized shape");
    const auto epi = accumulate ? ovg::Epilogue::kAccumulate : ovg::Epilogue::kStore;
    // The plan of ovg_op_linear, so both give the same result bit for bit.
    const ovg::GemmPlan plan = ovg::PlanGemm(static_cast<int>(rows), static_cast<int>(out),
                                             static_cast<int>(in), epi, true);
    if (plan.partial_floats > kScratchFloats)
      throw ovg::Error("split-K partials of " + std::to_string(plan.partial_floats) +
                       " floats exceed the " + std::to_string(kScratchFloats) +
                       "-float scratch of the no-allocation entry point");
    ovg::GemmParams p{};
    p.x = static_cast<const ovg::half_t*>(x);
    p.w = static_cast<const ovg::half_t*>(w);
    p.lda = static_cast<int>(in);
    p.ldb = static_cast<int>(in);
    p.m = static_cast<int>(rows);
    p.n = static_cast<int>(out);
    p.k = static_cast<int>(in);
    p.splits = plan.splits;
    p.partials = plan.splits > 1 ? DeviceScratch() : nullptr;
    p.y = y;
    p.ldc = static_cast<int>(out);
    ovg::LaunchGemm(p, plan, epi, static_cast<hipStream_t>(stream));
    return OVG_OK;
  } catch (const std::exception& failure) {
    SetError(error, error_len, std::string("linear: ") + failure.what());
    return OVG_ERROR;
  }
}
