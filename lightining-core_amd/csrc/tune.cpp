// tune.cpp -- gfx950 tune cache for the GEMM kernels.
//
// Keeps the reference's on-disk convention (src/ops/matmul_metal.mm:133-139,
// :416-517; tests/test_python_tune_cache_format_smoke.py:35-88): a header line
// "#lc_tune_cache,matmul,2", a "#columns,..." line, then one CSV row per
// shape.  The key is (m, k, n, dtype, arch) and the value is the gfx950 kernel
// configuration chosen for it (block tile, waves, split-K).  A file with a
// wrong header is ignored and the cache left empty (the reference clears and
// re-tunes on a corrupt header, src/attention_metal.mm:297-302).
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <tuple>

#include "lc_internal.hpp"
#include "tune.hpp"

namespace lchip {
namespace {

using Key = std::tuple<std::size_t, std::size_t, std::size_t, int, std::string>;

std::mutex g_tune_mu;
std::map<Key, TuneEntry>& table() {
  static auto* t = new std::map<Key, TuneEntry>();
  return *t;
}

const char* kHeader = "#lc_tune_cache,matmul,2";
const char* kColumns = "#columns,m,k,n,dtype,arch,kernel,tile_m,tile_n,tile_k,waves,split_k";

}  // namespace

void tuneRecord(std::size_t m, std::size_t k, std::size_t n, int dtype, const std::string& arch,
                const TuneEntry& e) {
  std::lock_guard<std::mutex> lock(g_tune_mu);
  table()[Key{m, k, n, dtype, arch}] = e;
}

bool tuneLookup(std::size_t m, std::size_t k, std::size_t n, int dtype, const std::string& arch, TuneEntry* out) {
  std::lock_guard<std::mutex> lock(g_tune_mu);
  auto it = table().find(Key{m, k, n, dtype, arch});
  if (it == table().end()) {
    return false;
  }
  *out = it->second;
  return true;
}

void tuneReset() {
  std::lock_guard<std::mutex> lock(g_tune_mu);
  table().clear();
}

std::size_t tuneSize() {
  std::lock_guard<std::mutex> lock(g_tune_mu);
  return table().size();
}

}  // namespace lchip

using namespace lchip;

extern "C" {

lcError_t lcMatMulResetTuning(void) {
  tuneReset();
  return LC_SUCCESS;
}

lcError_t lcHipTuneCacheSave(const char* path) {
  if (path == nullptr) {
    return LC_INVALID_VALUE;
  }
  std::ofstream f(path, std::ios::trunc);
  if (!f) {
    return toLc(fail(Status::kInvalidValue, std::string("tune cache: cannot write ") + path));
  }
  f << kHeader << "\n" << kColumns << "\n";
  std::lock_guard<std::mutex> lock(g_tune_mu);
  for (const auto& kv : table()) {
    const auto& k = kv.first;
    const auto& e = kv.second;
    f << std::get<0>(k) << "," << std::get<1>(k) << "," << std::get<2>(k) << "," << std::get<3>(k) << ","
      << std::get<4>(k) << "," << e.kernel << "," << e.tile_m << "," << e.tile_n << "," << e.tile_k << ","
      << e.waves << "," << e.split_k << "\n";
  }
  return LC_SUCCESS;
}

lcError_t lcHipTuneCacheLoad(const char* path) {
  if (path == nullptr) {
    return LC_INVALID_VALUE;
  }
  std::ifstream f(path);
  if (!f) {
    return toLc(fail(Status::kInvalidValue, std::string("tune cache: cannot read ") + path));
  }
  std::string line;
  if (!std::getline(f, line) || line.rfind(kHeader, 0) != 0) {
    tuneReset();
    return toLc(fail(Status::kInvalidValue, "tune cache: bad header (cache cleared)"));
  }
  std::map<Key, TuneEntry> loaded;
  while (std::getline(f, line)) {
    if (line.empty() || line[0] == '#') {
      continue;
    }
    std::stringstream ss(line);
    std::string tok[11];
    int i = 0;
    while (i < 11 && std::getline(ss, tok[i], ',')) {
      ++i;
    }
    if (i != 11) {
      continue;
    }
    try {
      Key key{std::stoull(tok[0]), std::stoull(tok[1]), std::stoull(tok[2]), std::stoi(tok[3]), tok[4]};
      TuneEntry e;
      e.kernel = tok[5];
      e.tile_m = std::stoi(tok[6]);
      e.tile_n = std::stoi(tok[7]);
      e.tile_k = std::stoi(tok[8]);
      e.waves = std::stoi(tok[9]);
      e.split_k = std::stoi(tok[10]);
      loaded[key] = e;
    } catch (...) {
      continue;
    }
  }
  std::lock_guard<std::mutex> lock(g_tune_mu);
  table() = loaded;
  return LC_SUCCESS;
}

}  // extern "C"
