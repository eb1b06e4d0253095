// tune.hpp -- gfx950 tune caches (GEMM kernel variant per shape, fp32
// attention key splits per shape) and the CJ_* runtime profile autoload.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

namespace lchip {

// One GEMM configuration.  `kernel` names the variant ("f32_dp_64x64x64",
// "half_lds_256x256", ...); the tile / wave / split fields describe it for a
// reader of the cache file.
struct TuneEntry {
  std::string kernel;
  int tile_m = 0;
  int tile_n = 0;
  int tile_k = 0;
  int waves = 0;
  int split_k = 1;
};

// The matmul cache.  Lookups load the cache file once per process
// (CJ_MATMUL_TUNE_CACHE_FILE, else .lightning_core_matmul_tune_cache.csv in
// the working directory); a record that changes the table rewrites it.
void tuneRecord(std::size_t m, std::size_t k, std::size_t n, int dtype, const std::string& arch, const TuneEntry& e);
bool tuneLookup(std::size_t m, std::size_t k, std::size_t n, int dtype, const std::string& arch, TuneEntry* out);
void tuneReset();
std::size_t tuneSize();

// The attention cache: the reference's key (kind 'F' forward or 'T' train
// step, seq, dim, causal, resident_hint, sync_hint, compute_loss for 'T')
// plus the arch; the value is the fp32 kernel's split count (1, 2, 4 or 8
// waves per 32 queries; the train step's dV kernel for 'T').  The file
// holds them as HF / HT rows next to the reference's own F / T rows, which are
// kept but never read as split counts.
// File: CJ_ATTN_TUNE_CACHE_FILE, else .lightning_core_attn_tune_cache.csv.
struct AttnTuneKey {
  char kind = 'F';
  std::size_t seq = 0;
  std::size_t dim = 0;
  uint8_t causal = 0;
  uint8_t resident_hint = 0;
  uint8_t sync_hint = 0;
  uint8_t compute_loss = 0;  // 'T' rows only
  std::string arch;          // e.g. "gfx950"
};
bool attnTuneLookup(const AttnTuneKey& key, int* mode);
void attnTuneRecord(const AttnTuneKey& key, int mode);
void attnTuneReset();
std::size_t attnTuneSize();

// First-call autotuning is on unless the variable is 0 / false / off / no
// (CJ_MATMUL_AUTOTUNE, CJ_ATTN_AUTOTUNE).
bool autotuneEnabled(const char* env_name);

// Imports CJ_* assignments from the runtime profile file once per process
// (CJ_RUNTIME_PROFILE_ENV_FILE, else the first of the reference's
// cwd-relative candidates that exists), without overriding variables that are
// already set; CJ_RUNTIME_PROFILE_AUTOLOAD=0 turns it off.
void ensureRuntimeProfileLoaded();

}  // namespace lchip
