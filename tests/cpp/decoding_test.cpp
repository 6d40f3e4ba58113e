// The reference's decoding checks (tests/decoding_test.cpp of
// gufo-extensions/omnivoice) against this library's decoding.hpp surface:
// the fixture's schedules and conditional inputs, and the greedy
// position-choice known answer. The fixture comes as plain text (written by
// tests/test_cpp_api.py from tests/golden/generator_cases.json):
//   schedule <total> <steps> <t_shift> <count>...
//   input <codebooks> <mask> <text n> <ids>... <reference frames>
//         <codes>... <target frames> <expected length> <expected ids>...
#include <cstdint>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "omnivoice/decoding.hpp"

namespace ov = gufo::models::omnivoice;

namespace {

int failures = 0;

void Expect(bool condition, const std::string& what) {
  if (!condition) {
    std::cout << "FAIL " << what << '\n';
    ++failures;
  }
}

template <typename T>
std::vector<T> ReadValues(std::istream& in, std::size_t n) {
  std::vector<T> values(n);
  for (auto& v : values)
    in >> v;
  return values;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::cerr << "usage: decoding_test <fixture.txt>\n";
    return 2;
  }
  std::ifstream in(argv[1]);
  std::string kind;
  int cases = 0;
  while (in >> kind) {
    if (kind == "schedule") {
      std::size_t total = 0, steps = 0;
      float t_shift = 0.0F;
      in >> total >> steps >> t_shift;
      const auto expected = ReadValues<std::size_t>(in, steps);
      Expect(ov::UnmaskSchedule(total, steps, t_shift) == expected,
             "schedule of " + std::to_string(total) + " codes");
    } else if (kind == "input") {
      std::size_t codebooks = 0, text_n = 0, reference_frames = 0;
      std::size_t target_frames = 0, length = 0;
      std::uint32_t mask = 0;
      in >> codebooks >> mask >> text_n;
      const auto text = ReadValues<std::uint32_t>(in, text_n);
      in >> reference_frames;
      const auto reference =
          ReadValues<std::int32_t>(in, codebooks * reference_frames);
      in >> target_frames >> length;
      const auto expected = ReadValues<std::int32_t>(in, codebooks * length);
      const auto input = ov::ConditionalInput::Build(
          text, reference, reference_frames, target_frames, codebooks, mask);
      Expect(input.length == length && input.ids == expected &&
                 input.audio_start == text_n &&
                 input.target_frames == target_frames,
             "conditional input with " + std::to_string(text_n) + " tokens");
    } else {
      std::cerr << "unknown fixture line " << kind << '\n';
      return 2;
    }
    ++cases;
  }
  // Greedy choice: two codebooks of three frames, codebook 1 pays a penalty
  // of 5; frame 1 of codebook 0 is already filled.
  ov::DecodingConfig decoding;
  decoding.position_temperature = 0.0F;
  ov::PositionSelector selector(decoding, 0);
  std::vector<std::int32_t> codes = {1024, 7, 1024, 1024, 1024, 1024};
  const auto chosen = selector.Fill(2, 2, 3, {10, 11, 12, 13, 14, 15},
                                    {-0.5F, -0.1F, -2.0F, -0.2F, -0.3F, -9.0F},
                                    1024, &codes);
  Expect(chosen == std::vector<std::size_t>({0, 2}) &&
             codes == std::vector<std::int32_t>({10, 7, 12, 1024, 1024, 1024}),
         "greedy position choice");
  std::cout << (failures == 0 ? "ok" : "FAIL") << " decoding: " << cases
            << " fixture cases, " << failures << " failures\n";
  return failures == 0 ? 0 : 1;
}
