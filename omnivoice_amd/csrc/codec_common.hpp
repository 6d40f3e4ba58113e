// Host helpers shared by the audio decoder and encoder engines: the
// synthetic weight specification, the tensor source (synthetic or a
// checkpoint), uploads and the convolution weight layout.
#ifndef OMNIVOICE_AMD_CODEC_COMMON_HPP_
#define OMNIVOICE_AMD_CODEC_COMMON_HPP_

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <exception>
#include <initializer_list>
#include <string>
#include <vector>

#include "../../include/omnivoice_mi355x.h"
#include "checkpoint.hpp"
#include "device.hpp"
#include "host.hpp"

namespace ovg {

// Synthetic tensor values: float(offset + scale n), or float(exp(scale n))
// for the Snake alphas, n = SynthNormal(seed, id, element) over the flat
// index in the checkpoint tensor's own shape.
inline void SynthCodec(std::uint64_t seed, std::uint64_t id, double scale, bool exponential,
                       std::uint64_t first, std::size_t count, float* out,
                       double offset = 0.0) {
  for (std::size_t e = 0; e < count; ++e) {
    const double n = SynthNormal(seed, id, first + e);
    out[e] = static_cast<float>(exponential ? std::exp(scale * n) : offset + scale * n);
  }
}

// A tensor source: the synthetic specification or a checkpoint.
class Source {
 public:
  Source(std::uint64_t seed, const SafetensorsFile* file) : seed_(seed), file_(file) {}
  std::vector<float> Get(const std::string& name, std::initializer_list<std::int64_t> shape,
                         std::uint64_t id, double scale, bool exponential = false,
                         double offset = 0.0) const {
    std::size_t count = 1;
    for (const std::int64_t d : shape)
      count *= static_cast<std::size_t>(d);
    std::vector<float> out(count);
    if (file_ != nullptr) {
      const float* data = file_->F32(name, shape);
      std::memcpy(out.data(), data, count * sizeof(float));
    } else {
      SynthCodec(seed_, id, scale, exponential, 0, count, out.data(), offset);
    }
    return out;
  }

 private:
  std::uint64_t seed_;
  const SafetensorsFile* file_;
};

// A synchronous copy from pageable memory may return before its data has
// landed, and kernels on a non-blocking stream do not wait for it: wait for
// the device before the buffer is used.
template <typename T>
void Upload(DeviceBuffer<T>& buffer, const std::vector<T>& host) {
  buffer.Reserve(host.size());
  Check(hipMemcpy(buffer.get(), host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice),
        "upload codec weights");
  Check(hipDeviceSynchronize(), "upload codec weights");
}

// Conv1d weights [out][in][kernel] -> [kernel][in][out]. With kernel 1 and
// in = channels x taps this is also the layout of a convolution run over
// im2col columns: [channels x taps][out].
inline std::vector<float> ConvLayout(const std::vector<float>& w, int out, int in, int kernel) {
  std::vector<float> r(w.size());
  for (int o = 0; o < out; ++o)
    for (int i = 0; i < in; ++i)
      for (int k = 0; k < kernel; ++k)
        r[(static_cast<std::size_t>(k) * in + i) * out + o] =
            w[(static_cast<std::size_t>(o) * in + i) * kernel + k];
  return r;
}

// Runs one C entry point's body: an exception becomes OVG_ERROR with
// `prefix` + its message in the caller's buffer (truncated to fit).
template <typename F>
int CodecGuard(const char* prefix, char* error, std::size_t len, F&& body) {
  try {
    return body();
  } catch (const std::exception& failure) {
    if (error != nullptr && len > 0) {
      const std::string message = std::string(prefix) + failure.what();
      const std::size_t n = std::min(len - 1, message.size());
      std::memcpy(error, message.data(), n);
      error[n] = '\0';
    }
    return OVG_ERROR;
  }
}

}  // namespace ovg

#endif  // OMNIVOICE_AMD_CODEC_COMMON_HPP_
