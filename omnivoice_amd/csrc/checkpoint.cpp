#include "checkpoint.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <string_view>

#include "kernels.hpp"

namespace ovg {
namespace {

// Largest header the format allows.
constexpr std::uint64_t kMaxHeader = 100'000'000;

// A JSON value, as much of JSON as a safetensors header uses.
struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  double number = 0.0;
  bool integral = false;
  std::int64_t integer = 0;
  std::string text;
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;
};

class JsonParser {
 public:
  explicit JsonParser(std::string_view s) : s_(s) {}

  Json Document() {
    Json v = Value(0);
    Skip();
    Require(pos_ == s_.size(), "header: trailing characters");
    return v;
  }

 private:
  void Skip() {
    while (pos_ < s_.size() && (s_[pos_] == ' ' || s_[pos_] == '\t' ||
                                s_[pos_] == '\n' || s_[pos_] == '\r'))
      ++pos_;
  }
  char Peek() {
    Skip();
    Require(pos_ < s_.size(), "header: unexpected end");
    return s_[pos_];
  }
  void Expect(char c) {
    Require(Peek() == c, std::string("header: expected '") + c + "'");
    ++pos_;
  }
  bool Literal(std::string_view word) {
    if (s_.substr(pos_, word.size()) != word)
      return false;
    pos_ += word.size();
    return true;
  }

  Json Value(int depth) {
    Require(depth < 16, "header: nested too deeply");
    Json v;
    const char c = Peek();
    if (c == '{') {
      v.kind = Json::kObject;
      ++pos_;
      if (Peek() == '}') {
        ++pos_;
        return v;
      }
      for (;;) {
        std::string key = String();
        Expect(':');
        v.members.emplace_back(std::move(key), Value(depth + 1));
        if (Peek() == ',') {
          ++pos_;
          continue;
        }
        Expect('}');
        return v;
      }
    }
    if (c == '[') {
      v.kind = Json::kArray;
      ++pos_;
      if (Peek() == ']') {
        ++pos_;
        return v;
      }
      for (;;) {
        v.items.push_back(Value(depth + 1));
        if (Peek() == ',') {
          ++pos_;
          continue;
        }
        Expect(']');
        return v;
      }
    }
    if (c == '"') {
      v.kind = Json::kString;
      v.text = String();
      return v;
    }
    if (Literal("true") || Literal("false")) {
      v.kind = Json::kBool;
      return v;
    }
    if (Literal("null"))
      return v;
    return Number();
  }

  std::string String() {
    Expect('"');
    std::string out;
    while (true) {
      Require(pos_ < s_.size(), "header: unterminated string");
      const char c = s_[pos_++];
      if (c == '"')
        return out;
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      Require(pos_ < s_.size(), "header: unterminated escape");
      const char e = s_[pos_++];
      switch (e) {
        case '"': case '\\': case '/': out.push_back(e); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          Require(pos_ + 4 <= s_.size(), "header: short \\u escape");
          unsigned code = 0;
          for (int i = 0; i < 4; ++i) {
            const char h = s_[pos_++];
            code <<= 4;
            if (h >= '0' && h <= '9') code |= static_cast<unsigned>(h - '0');
            else if (h >= 'a' && h <= 'f') code |= static_cast<unsigned>(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') code |= static_cast<unsigned>(h - 'A' + 10);
            else Require(false, "header: bad \\u escape");
          }
          // Names and dtypes are ASCII; other code points are kept as UTF-8.
          if (code < 0x80) {
            out.push_back(static_cast<char>(code));
          } else if (code < 0x800) {
            out.push_back(static_cast<char>(0xC0 | (code >> 6)));
            out.push_back(static_cast<char>(0x80 | (code & 0x3F)));
          } else {
            out.push_back(static_cast<char>(0xE0 | (code >> 12)));
            out.push_back(static_cast<char>(0x80 | ((code >> 6) & 0x3F)));
            out.push_back(static_cast<char>(0x80 | (code & 0x3F)));
          }
          break;
        }
        default: Require(false, "header: bad escape");
      }
    }
  }

  Json Number() {
    Json v;
    v.kind = Json::kNumber;
    const std::size_t start = pos_;
    if (pos_ < s_.size() && s_[pos_] == '-')
      ++pos_;
    bool digits = false, fraction = false;
    while (pos_ < s_.size()) {
      const char c = s_[pos_];
      if (c >= '0' && c <= '9') {
        digits = true;
      } else if (c == '.' || c == 'e' || c == 'E' || c == '+' || c == '-') {
        fraction = true;
      } else {
        break;
      }
      ++pos_;
    }
    Require(digits, "header: bad value");
    const std::string text(s_.substr(start, pos_ - start));
    v.number = std::strtod(text.c_str(), nullptr);
    if (!fraction && text.size() <= 18) {
      v.integral = true;
      v.integer = std::strtoll(text.c_str(), nullptr, 10);
    }
    return v;
  }

  std::string_view s_;
  std::size_t pos_ = 0;
};

std::string ShapeText(const std::vector<std::int64_t>& shape) {
  std::string out = "[";
  for (std::size_t i = 0; i < shape.size(); ++i)
    out += (i ? ", " : "") + std::to_string(shape[i]);
  return out + "]";
}

std::size_t DTypeBytes(const std::string& dtype) {
  if (dtype == "F64" || dtype == "I64" || dtype == "U64") return 8;
  if (dtype == "F32" || dtype == "I32" || dtype == "U32") return 4;
  if (dtype == "F16" || dtype == "BF16" || dtype == "I16" || dtype == "U16") return 2;
  if (dtype == "I8" || dtype == "U8" || dtype == "BOOL" || dtype == "F8_E4M3" ||
      dtype == "F8_E5M2")
    return 1;
  return 0;
}

}  // namespace

std::string JoinPath(const std::string& root, const std::string& name) {
  if (root.empty())
    return name;
  return root.back() == '/' ? root + name : root + "/" + name;
}

std::unique_ptr<SafetensorsFile> SafetensorsFile::Open(const std::string& path) {
  std::unique_ptr<SafetensorsFile> file(new SafetensorsFile());
  file->path_ = path;
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  Require(fd >= 0, "cannot open " + path + ": " + std::strerror(errno));
  struct stat st {};
  if (::fstat(fd, &st) != 0 || st.st_size < 8) {
    ::close(fd);
    throw Error(path + ": file is shorter than its header length");
  }
  file->size_ = static_cast<std::size_t>(st.st_size);
  void* map = ::mmap(nullptr, file->size_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  Require(map != MAP_FAILED, "cannot map " + path + ": " + std::strerror(errno));
  file->data_ = static_cast<const unsigned char*>(map);
  std::uint64_t header = 0;
  for (int i = 7; i >= 0; --i)
    header = (header << 8) | file->data_[i];
  Require(header >= 2 && header <= kMaxHeader && header <= file->size_ - 8,
          path + ": implausible header length");
  file->payload_ = 8 + header;
  const std::uint64_t payload_bytes = file->size_ - file->payload_;
  Json doc;
  try {
    doc = JsonParser(std::string_view(
                         reinterpret_cast<const char*>(file->data_ + 8), header))
              .Document();
  } catch (const Error& e) {
    throw Error(path + ": " + e.what());
  }
  Require(doc.kind == Json::kObject, path + ": header is not a JSON object");
  std::vector<std::pair<std::uint64_t, std::uint64_t>> ranges;
  for (const auto& [name, v] : doc.members) {
    if (name == "__metadata__")
      continue;
    const std::string where = path + ": " + name;
    Require(v.kind == Json::kObject, where + " is not an object");
    Entry e;
    bool has_dtype = false, has_shape = false, has_offsets = false;
    for (const auto& [key, field] : v.members) {
      if (key == "dtype" && field.kind == Json::kString) {
        e.dtype = field.text;
        has_dtype = true;
      } else if (key == "shape" && field.kind == Json::kArray) {
        for (const Json& d : field.items) {
          Require(d.kind == Json::kNumber && d.integral && d.integer >= 0,
                  where + ": bad shape");
          e.shape.push_back(d.integer);
        }
        has_shape = true;
      } else if (key == "data_offsets" && field.kind == Json::kArray &&
                 field.items.size() == 2) {
        for (const Json& d : field.items)
          Require(d.kind == Json::kNumber && d.integral && d.integer >= 0,
                  where + ": bad data_offsets");
        e.begin = static_cast<std::uint64_t>(field.items[0].integer);
        e.end = static_cast<std::uint64_t>(field.items[1].integer);
        has_offsets = true;
      }
    }
    Require(has_dtype && has_shape && has_offsets,
            where + ": needs dtype, shape and data_offsets");
    Require(e.begin <= e.end && e.end <= payload_bytes,
            where + ": data outside the file");
    const std::size_t element = DTypeBytes(e.dtype);
    Require(element != 0, where + ": unknown dtype " + e.dtype);
    std::uint64_t count = 1;
    for (const std::int64_t d : e.shape)
      count *= static_cast<std::uint64_t>(d);
    Require(count * element == e.end - e.begin,
            where + ": size does not match its shape");
    ranges.emplace_back(e.begin, e.end);
    Require(file->tensors_.emplace(name, std::move(e)).second,
            where + " appears twice");
  }
  Require(!file->tensors_.empty(), path + ": no tensors");
  std::sort(ranges.begin(), ranges.end());
  for (std::size_t i = 1; i < ranges.size(); ++i)
    Require(ranges[i - 1].second <= ranges[i].first,
            path + ": tensors overlap");
  return file;
}

SafetensorsFile::~SafetensorsFile() {
  if (data_ != nullptr)
    ::munmap(const_cast<unsigned char*>(data_), size_);
}

const float* SafetensorsFile::F32(const std::string& name,
                                  std::initializer_list<std::int64_t> shape) const {
  const auto found = tensors_.find(name);
  const std::string file_name = path_.substr(path_.find_last_of('/') + 1);
  Require(found != tensors_.end(), file_name + " lacks " + name);
  const Entry& e = found->second;
  const std::vector<std::int64_t> expected(shape);
  Require(e.dtype == "F32" && e.shape == expected,
          name + " is " + e.dtype + " " + ShapeText(e.shape) + ", expected F32 " +
              ShapeText(expected));
  return reinterpret_cast<const float*>(data_ + payload_ + e.begin);
}

}  // namespace ovg
