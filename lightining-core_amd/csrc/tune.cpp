// tune.cpp -- gfx950 tune caches and the runtime profile autoload.
//
// File conventions follow the reference (src/ops/matmul_metal.mm:133-139,
// :416-517; src/attention_metal.mm:184-336; tests/test_python_tune_cache_
// format_smoke.py:35-88): a header "#lc_tune_cache,<kind>,<version>", a
// "#columns,..." line, then one CSV row per key.  Versions 1 and 2 are read,
// version 2 is written; a header of another kind or version clears the table
// (the reference re-tunes then).  Rows are re-keyed for gfx950:
//   matmul    m,k,n,dtype,arch,kernel,tile_m,tile_n,tile_k,waves,split_k
//   attention HF|HT,seq,dim,causal,resident_hint,sync_hint,[compute_loss,]arch,splits
// Rows in the reference's own layouts (matmul: 5 or 6 columns, Metal tiles;
// attention: F / T rows whose mode is a Metal forward / train mode) mean
// nothing on gfx950; they are kept verbatim and written back so a file
// shared with the reference keeps its rows.  gfx950 attention rows use their
// own kinds (HF forward, HT train step), which the reference's reader skips,
// and carry the arch; the value is the fp32 kernel's split count (1, 2, 4, 8,
// or 16 for the 16-query / 16-key kernels), and a row whose value is not one
// of those is dropped.
//
// The runtime profile autoload restates src/runtime.cpp:101-168.
#include <algorithm>
#include <array>
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "lc_internal.hpp"
#include "tune.hpp"

namespace lchip {
namespace {

constexpr const char* kTag = "#lc_tune_cache";
constexpr int kVersion = 2;
constexpr int kMinVersion = 1;

std::string trim(const std::string& s) {
  std::size_t b = 0;
  std::size_t e = s.size();
  while (b < e && std::isspace(static_cast<unsigned char>(s[b]))) ++b;
  while (e > b && std::isspace(static_cast<unsigned char>(s[e - 1]))) --e;
  return s.substr(b, e - b);
}

std::vector<std::string> splitCsv(const std::string& line) {
  std::vector<std::string> cols;
  std::stringstream ss(line);
  std::string tok;
  while (std::getline(ss, tok, ',')) {
    cols.push_back(trim(tok));
  }
  return cols;
}

bool envMeansFalse(const char* raw) {
  if (raw == nullptr) {
    return false;
  }
  std::string v = trim(raw);
  for (char& c : v) {
    c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
  }
  return v == "0" || v == "false" || v == "off" || v == "no";
}

std::string pathFrom(const char* env, const char* fallback) {
  const char* p = std::getenv(env);
  return (p != nullptr && p[0] != '\0') ? std::string(p) : std::string(fallback);
}

// Reads a cache file: returns false when it cannot be opened.  `header_ok`
// is false when a tag line names another kind or an unsupported version;
// `rows` receives every non-comment line split into columns.
bool readCacheFile(const std::string& path, const char* kind, bool* header_ok,
                   std::vector<std::vector<std::string>>* rows) {
  std::ifstream f(path);
  if (!f.is_open()) {
    return false;
  }
  *header_ok = true;
  std::string line;
  while (std::getline(f, line)) {
    const std::string t = trim(line);
    if (t.empty()) {
      continue;
    }
    std::vector<std::string> cols = splitCsv(t);
    if (cols.empty()) {
      continue;
    }
    if (!cols[0].empty() && cols[0][0] == '#') {
      if (cols[0] == kTag) {
        int v = -1;
        try {
          v = cols.size() == 3 ? std::stoi(cols[2]) : -1;
        } catch (...) {
          v = -1;
        }
        if (cols.size() != 3 || cols[1] != kind || v < kMinVersion || v > kVersion) {
          *header_ok = false;
          return true;
        }
      }
      continue;
    }
    rows->push_back(std::move(cols));
  }
  return true;
}

// ---------------------------------------------------------------------------
// matmul
// ---------------------------------------------------------------------------
using Key = std::tuple<std::size_t, std::size_t, std::size_t, int, std::string>;

struct MatmulCache {
  std::mutex mu;
  std::map<Key, TuneEntry> table;
  std::vector<std::string> foreign;  // reference-layout rows, kept verbatim
  bool loaded = false;
  std::string path;
};

MatmulCache& mm() {
  static auto* c = new MatmulCache();  // process lifetime
  return *c;
}

const char* kMatmulColumns = "#columns,m,k,n,dtype,arch,kernel,tile_m,tile_n,tile_k,waves,split_k";

// Parses rows into a table; false for a bad header.
bool parseMatmul(const std::string& path, std::map<Key, TuneEntry>* table, std::vector<std::string>* foreign,
                 bool* opened) {
  bool header_ok = true;
  std::vector<std::vector<std::string>> rows;
  *opened = readCacheFile(path, "matmul", &header_ok, &rows);
  if (!*opened) {
    return true;
  }
  if (!header_ok) {
    return false;
  }
  for (const auto& c : rows) {
    if (c.size() == 11) {
      try {
        TuneEntry e;
        e.kernel = c[5];
        e.tile_m = std::stoi(c[6]);
        e.tile_n = std::stoi(c[7]);
        e.tile_k = std::stoi(c[8]);
        e.waves = std::stoi(c[9]);
        e.split_k = std::stoi(c[10]);
        (*table)[Key{std::stoull(c[0]), std::stoull(c[1]), std::stoull(c[2]), std::stoi(c[3]), c[4]}] = e;
      } catch (...) {
        // malformed rows are ignored, as the reference does
      }
    } else if (c.size() == 5 || c.size() == 6) {
      std::string joined;
      for (std::size_t i = 0; i < c.size(); ++i) {
        joined += (i ? "," : "") + c[i];
      }
      foreign->push_back(joined);
    }
  }
  return true;
}

bool writeMatmul(const std::string& path, const std::map<Key, TuneEntry>& table,
                 const std::vector<std::string>& foreign) {
  std::ofstream f(path, std::ios::trunc);
  if (!f.is_open()) {
    return false;
  }
  f << kTag << ",matmul," << kVersion << "\n" << kMatmulColumns << "\n";
  for (const auto& kv : table) {
    const auto& k = kv.first;
    const auto& e = kv.second;
    f << std::get<0>(k) << "," << std::get<1>(k) << "," << std::get<2>(k) << "," << std::get<3>(k) << ","
      << std::get<4>(k) << "," << e.kernel << "," << e.tile_m << "," << e.tile_n << "," << e.tile_k << "," << e.waves
      << "," << e.split_k << "\n";
  }
  for (const auto& row : foreign) {
    f << row << "\n";
  }
  return f.good();
}

void loadMatmulOnce(MatmulCache& c) {
  if (c.loaded) {
    return;
  }
  c.loaded = true;
  c.path = pathFrom("CJ_MATMUL_TUNE_CACHE_FILE", ".lightning_core_matmul_tune_cache.csv");
  bool opened = false;
  std::map<Key, TuneEntry> t;
  std::vector<std::string> foreign;
  if (parseMatmul(c.path, &t, &foreign, &opened)) {
    for (auto& kv : t) {
      c.table.insert(kv);  // entries recorded before the load win
    }
    c.foreign = std::move(foreign);
  }
}

bool sameEntry(const TuneEntry& a, const TuneEntry& b) {
  return a.kernel == b.kernel && a.tile_m == b.tile_m && a.tile_n == b.tile_n && a.tile_k == b.tile_k &&
         a.waves == b.waves && a.split_k == b.split_k;
}

// ---------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------
using AKey = std::tuple<char, std::size_t, std::size_t, int, int, int, int, std::string>;

AKey akey(const AttnTuneKey& k) {
  return AKey{k.kind, k.seq, k.dim, k.causal, k.resident_hint, k.sync_hint, k.kind == 'T' ? k.compute_loss : 0,
              k.arch};
}

struct AttnCache {
  std::mutex mu;
  std::map<AKey, int> table;
  std::vector<std::string> foreign;  // reference-layout F / T rows, kept verbatim
  bool loaded = false;
  std::string path;
};

AttnCache& at() {
  static auto* c = new AttnCache();  // process lifetime
  return *c;
}

const char* kAttnColumns = "#columns,kind,seq,dim,causal,resident_hint,sync_hint,compute_loss_or_mode,mode";
const char* kAttnHipColumns = "#columns_hip,kind,seq,dim,causal,resident_hint,sync_hint,compute_loss(HT),arch,splits";

bool validSplit(int mode) { return mode == 1 || mode == 2 || mode == 4 || mode == 8; }
bool validSplit(char, int mode) { return validSplit(mode) || mode == 16; }

std::string joinCsv(const std::vector<std::string>& c) {
  std::string joined;
  for (std::size_t i = 0; i < c.size(); ++i) {
    joined += (i ? "," : "") + c[i];
  }
  return joined;
}

bool parseAttn(const std::string& path, std::map<AKey, int>* table, std::vector<std::string>* foreign,
               bool* opened) {
  bool header_ok = true;
  std::vector<std::vector<std::string>> rows;
  *opened = readCacheFile(path, "attention", &header_ok, &rows);
  if (!*opened) {
    return true;
  }
  if (!header_ok) {
    return false;
  }
  for (const auto& c : rows) {
    try {
      if (c.size() == 8 && c[0] == "HF") {
        const int mode = std::stoi(c[7]);
        if (validSplit('F', mode)) {
          (*table)[AKey{'F', std::stoull(c[1]), std::stoull(c[2]), std::stoi(c[3]), std::stoi(c[4]),
                        std::stoi(c[5]), 0, c[6]}] = mode;
        }
      } else if (c.size() == 9 && c[0] == "HT") {
        const int mode = std::stoi(c[8]);
        if (validSplit('T', mode)) {
          (*table)[AKey{'T', std::stoull(c[1]), std::stoull(c[2]), std::stoi(c[3]), std::stoi(c[4]),
                        std::stoi(c[5]), std::stoi(c[6]), c[7]}] = mode;
        }
      } else if ((c.size() == 7 && c[0] == "F") || (c.size() == 8 && c[0] == "T")) {
        foreign->push_back(joinCsv(c));
      }
    } catch (...) {
      // malformed rows are ignored
    }
  }
  return true;
}

bool writeAttn(const std::string& path, const std::map<AKey, int>& table, const std::vector<std::string>& foreign) {
  std::ofstream f(path, std::ios::trunc);
  if (!f.is_open()) {
    return false;
  }
  f << kTag << ",attention," << kVersion << "\n" << kAttnColumns << "\n" << kAttnHipColumns << "\n";
  for (const auto& row : foreign) {
    f << row << "\n";
  }
  for (const auto& kv : table) {
    const auto& k = kv.first;
    f << (std::get<0>(k) == 'T' ? "HT" : "HF") << "," << std::get<1>(k) << "," << std::get<2>(k) << ","
      << std::get<3>(k) << "," << std::get<4>(k) << "," << std::get<5>(k) << ",";
    if (std::get<0>(k) == 'T') {
      f << std::get<6>(k) << ",";
    }
    f << std::get<7>(k) << "," << kv.second << "\n";
  }
  return f.good();
}

void loadAttnOnce(AttnCache& c) {
  if (c.loaded) {
    return;
  }
  c.loaded = true;
  c.path = pathFrom("CJ_ATTN_TUNE_CACHE_FILE", ".lightning_core_attn_tune_cache.csv");
  bool opened = false;
  std::map<AKey, int> t;
  std::vector<std::string> foreign;
  if (parseAttn(c.path, &t, &foreign, &opened)) {
    for (auto& kv : t) {
      c.table.insert(kv);
    }
    c.foreign = std::move(foreign);
  }
}

}  // namespace

void tuneRecord(std::size_t m, std::size_t k, std::size_t n, int dtype, const std::string& arch,
                const TuneEntry& e) {
  MatmulCache& c = mm();
  std::lock_guard<std::mutex> lock(c.mu);
  loadMatmulOnce(c);
  const Key key{m, k, n, dtype, arch};
  auto it = c.table.find(key);
  if (it != c.table.end() && sameEntry(it->second, e)) {
    return;
  }
  c.table[key] = e;
  (void)writeMatmul(c.path, c.table, c.foreign);  // best effort, as the reference's save
}

bool tuneLookup(std::size_t m, std::size_t k, std::size_t n, int dtype, const std::string& arch, TuneEntry* out) {
  MatmulCache& c = mm();
  std::lock_guard<std::mutex> lock(c.mu);
  loadMatmulOnce(c);
  auto it = c.table.find(Key{m, k, n, dtype, arch});
  if (it == c.table.end()) {
    return false;
  }
  *out = it->second;
  return true;
}

void tuneReset() {
  MatmulCache& c = mm();
  std::lock_guard<std::mutex> lock(c.mu);
  c.table.clear();
  c.loaded = true;  // a reset drops the file's entries too (re-tune from scratch)
  if (c.path.empty()) {
    c.path = pathFrom("CJ_MATMUL_TUNE_CACHE_FILE", ".lightning_core_matmul_tune_cache.csv");
  }
}

std::size_t tuneSize() {
  MatmulCache& c = mm();
  std::lock_guard<std::mutex> lock(c.mu);
  return c.table.size();
}

bool attnTuneLookup(const AttnTuneKey& key, int* mode) {
  AttnCache& c = at();
  std::lock_guard<std::mutex> lock(c.mu);
  loadAttnOnce(c);
  auto it = c.table.find(akey(key));
  if (it == c.table.end()) {
    return false;
  }
  *mode = it->second;
  return true;
}

void attnTuneRecord(const AttnTuneKey& key, int mode) {
  if (!validSplit(key.kind, mode)) {
    return;
  }
  AttnCache& c = at();
  std::lock_guard<std::mutex> lock(c.mu);
  loadAttnOnce(c);
  const AKey k = akey(key);
  auto it = c.table.find(k);
  if (it != c.table.end() && it->second == mode) {
    return;
  }
  c.table[k] = mode;
  (void)writeAttn(c.path, c.table, c.foreign);
}

void attnTuneReset() {
  AttnCache& c = at();
  std::lock_guard<std::mutex> lock(c.mu);
  c.table.clear();
  c.loaded = true;
  if (c.path.empty()) {
    c.path = pathFrom("CJ_ATTN_TUNE_CACHE_FILE", ".lightning_core_attn_tune_cache.csv");
  }
}

std::size_t attnTuneSize() {
  AttnCache& c = at();
  std::lock_guard<std::mutex> lock(c.mu);
  return c.table.size();
}

bool autotuneEnabled(const char* env_name) {
  ensureRuntimeProfileLoaded();
  return !envMeansFalse(std::getenv(env_name));
}

// src/runtime.cpp:101-168: CJ_RUNTIME_PROFILE_ENV_FILE or the first readable
// candidate; "KEY=VALUE" lines, '#' comments, only CJ_* keys, never
// overriding a variable that is already set (and non-empty).
void ensureRuntimeProfileLoaded() {
  static std::once_flag once;
  std::call_once(once, []() {
    if (envMeansFalse(std::getenv("CJ_RUNTIME_PROFILE_AUTOLOAD"))) {
      return;
    }
    std::string path;
    const char* raw = std::getenv("CJ_RUNTIME_PROFILE_ENV_FILE");
    if (raw != nullptr && raw[0] != '\0') {
      path = raw;
    } else {
      static constexpr std::array<const char*, 7> kCandidates = {
          "build/benchmarks/model_runtime_profile.env", "../build/benchmarks/model_runtime_profile.env",
          "../../build/benchmarks/model_runtime_profile.env", "model_runtime_profile.env",
          "../model_runtime_profile.env", "benchmarks/model_runtime_profile.env",
          "../benchmarks/model_runtime_profile.env"};
      for (const char* cand : kCandidates) {
        std::ifstream probe(cand);
        if (probe.good()) {
          path = cand;
          break;
        }
      }
    }
    if (path.empty()) {
      return;
    }
    std::ifstream in(path);
    std::string line;
    while (std::getline(in, line)) {
      const std::string t = trim(line);
      if (t.empty() || t[0] == '#') {
        continue;
      }
      const std::size_t eq = t.find('=');
      if (eq == std::string::npos || eq == 0 || eq + 1 >= t.size()) {
        continue;
      }
      const std::string key = trim(t.substr(0, eq));
      const std::string val = trim(t.substr(eq + 1));
      if (key.empty() || val.empty() || key.rfind("CJ_", 0) != 0) {
        continue;
      }
      const char* existing = std::getenv(key.c_str());
      if (existing == nullptr || existing[0] == '\0') {
        (void)::setenv(key.c_str(), val.c_str(), 1);
      }
    }
  });
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
  MatmulCache& c = mm();
  std::lock_guard<std::mutex> lock(c.mu);
  loadMatmulOnce(c);
  if (!writeMatmul(path, c.table, c.foreign)) {
    return toLc(fail(Status::kInvalidValue, std::string("tune cache: cannot write ") + path));
  }
  return LC_SUCCESS;
}

lcError_t lcHipTuneCacheLoad(const char* path) {
  if (path == nullptr) {
    return LC_INVALID_VALUE;
  }
  std::map<Key, TuneEntry> t;
  std::vector<std::string> foreign;
  bool opened = false;
  const bool ok = parseMatmul(path, &t, &foreign, &opened);
  MatmulCache& c = mm();
  std::lock_guard<std::mutex> lock(c.mu);
  if (!opened) {
    return toLc(fail(Status::kInvalidValue, std::string("tune cache: cannot read ") + path));
  }
  c.loaded = true;
  c.path = path;
  if (!ok) {
    c.table.clear();
    c.foreign.clear();
    return toLc(fail(Status::kInvalidValue, "tune cache: unsupported header (cache cleared)"));
  }
  c.table = std::move(t);
  c.foreign = std::move(foreign);
  return LC_SUCCESS;
}

size_t lcHipTuneCacheSize(void) { return tuneSize(); }

lcError_t lcHipAttentionTuneCacheSave(const char* path) {
  if (path == nullptr) {
    return LC_INVALID_VALUE;
  }
  AttnCache& c = at();
  std::lock_guard<std::mutex> lock(c.mu);
  loadAttnOnce(c);
  if (!writeAttn(path, c.table, c.foreign)) {
    return toLc(fail(Status::kInvalidValue, std::string("attention tune cache: cannot write ") + path));
  }
  return LC_SUCCESS;
}

lcError_t lcHipAttentionTuneCacheLoad(const char* path) {
  if (path == nullptr) {
    return LC_INVALID_VALUE;
  }
  std::map<AKey, int> t;
  std::vector<std::string> foreign;
  bool opened = false;
  const bool ok = parseAttn(path, &t, &foreign, &opened);
  AttnCache& c = at();
  std::lock_guard<std::mutex> lock(c.mu);
  if (!opened) {
    return toLc(fail(Status::kInvalidValue, std::string("attention tune cache: cannot read ") + path));
  }
  c.loaded = true;
  c.path = path;
  if (!ok) {
    c.table.clear();
    c.foreign.clear();
    return toLc(fail(Status::kInvalidValue, "attention tune cache: unsupported header (cache cleared)"));
  }
  c.table = std::move(t);
  c.foreign = std::move(foreign);
  return LC_SUCCESS;
}

lcError_t lcHipAttentionResetTuning(void) {
  attnTuneReset();
  return LC_SUCCESS;
}

size_t lcHipAttentionTuneCacheSize(void) { return attnTuneSize(); }

void lcPreloadRuntimeProfileEnv(void) { ensureRuntimeProfileLoaded(); }

}  // extern "C"
