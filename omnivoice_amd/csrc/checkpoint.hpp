// Host-side reader of an OmniVoice checkpoint's model.safetensors: the
// format the reference loads in Generator::Load (generator.cpp:364-434 with
// safetensors.cpp:156-247): an 8-byte little-endian header length, a JSON
// header {name: {"dtype", "shape", "data_offsets": [begin, end]}} plus an
// optional "__metadata__" entry, then the payload the offsets index.
#ifndef OMNIVOICE_AMD_CHECKPOINT_HPP_
#define OMNIVOICE_AMD_CHECKPOINT_HPP_

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace ovg {

// `root` / `name` as std::filesystem::path joins them: an empty root gives
// `name` itself (relative to the working directory).
std::string JoinPath(const std::string& root, const std::string& name);

// A read-only mapping of one safetensors file. Open and F32 throw ovg::Error
// with a message naming the file or tensor at fault.
class SafetensorsFile {
 public:
  static std::unique_ptr<SafetensorsFile> Open(const std::string& path);
  ~SafetensorsFile();
  SafetensorsFile(const SafetensorsFile&) = delete;
  SafetensorsFile& operator=(const SafetensorsFile&) = delete;

  // The float32 tensor `name`, which must have exactly `shape`.
  const float* F32(const std::string& name,
                   std::initializer_list<std::int64_t> shape) const;
  std::size_t tensor_count() const { return tensors_.size(); }

 private:
  struct Entry {
    std::string dtype;
    std::vector<std::int64_t> shape;
    std::uint64_t begin = 0, end = 0;
  };
  SafetensorsFile() = default;
  std::string path_;
  const unsigned char* data_ = nullptr;
  std::size_t size_ = 0;
  std::uint64_t payload_ = 0;
  std::map<std::string, Entry> tensors_;
};

}  // namespace ovg

#endif  // OMNIVOICE_AMD_CHECKPOINT_HPP_
