// tune.hpp -- gfx950 tune cache (kernel configuration per GEMM shape).
#pragma once

#include <cstddef>
#include <string>

namespace lchip {

struct TuneEntry {
  std::string kernel;  // kernel family: "f32_mfma", "half_tn", "half_skinny"
  int tile_m = 0;
  int tile_n = 0;
  int tile_k = 0;
  int waves = 0;
  int split_k = 1;
};

void tuneRecord(std::size_t m, std::size_t k, std::size_t n, int dtype, const std::string& arch, const TuneEntry& e);
bool tuneLookup(std::size_t m, std::size_t k, std::size_t n, int dtype, const std::string& arch, TuneEntry* out);
void tuneReset();
std::size_t tuneSize();

}  // namespace lchip
