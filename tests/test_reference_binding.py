"""The reference-side binding of the integration guide, compiled (CPU only).

The guide's first section (the dispatcher hook) gives the `detail::` wrappers a maintainer adds to
the reference tree (`attentionForwardHipWithPolicy`,
`attentionTrainStepHipWithPolicy`, `matMulHipWithPolicy`).  This test takes
that code block verbatim from the document and compiles it with g++ against
the reference's own headers (`/root/reference/include`) and this library's
header, twice:

* with recording stand-ins for the three lc* entry points, so a call with a
  distinct value in every field of the reference's `AttentionConfig` /
  `AttentionIoPolicy` / matmul flags shows each value arriving in the right
  field of the C structs (a field-order slip in the wrappers fails here);
* linked against liblightning_core_hip.so: with no GPU in this container each
  wrapper must come back as `runtime::Status::kNotSupported`, the status the
  reference's dispatcher turns into its CPU fallback.

It also compiles the reference's frozen C header (`lightning_core.h`) and
compares its struct sizes with what the library reports (lcGetStructSize),
so the ABI check does not rest on hard-coded numbers.  The reference's status
numbering and this header's are compared the same way.  Skipped where the
reference tree or g++ is absent.
"""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = "/root/reference/include"
LIB = os.path.join(ROOT, "lightining-core_amd", "liblightning_core_hip.so")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_INC) or shutil.which("g++") is None,
                                reason="needs the reference headers and g++")


def _wrapper_block():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("## 1. C++ dispatcher hook"):]
    m = re.search(r"```cpp\n(.*?)```", sec, re.S)
    assert m, "no C++ block in the integration guide's dispatcher-hook section"
    block = m.group(1)
    assert "attentionForwardHipWithPolicy" in block and "matMulHipWithPolicy" in block
    return block


def _build_and_run(tmp_path, name, source, link_lib):
    src = tmp_path / f"{name}.cpp"
    exe = tmp_path / name
    src.write_text(source)
    cmd = ["g++", "-std=c++17", "-O0", "-Wall", "-Werror=return-type", "-I" + REF_INC,
           "-I" + os.path.join(ROOT, "include"), str(src), "-o", str(exe)]
    if link_lib:
        cmd += [LIB, "-Wl,-rpath," + os.path.dirname(LIB)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


_MAIN_COMMON = r"""
#include <cstdio>
#include <cstdlib>
#include "lightning_core/core/runtime.hpp"
namespace rt = lightning_core::runtime;
#define CHECK(c) do { if (!(c)) { std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); std::exit(1); } } while (0)
// lcError_t and runtime::Status share their numbering (lightning_core_c_api.cpp:9-27)
static_assert(static_cast<int>(rt::Status::kSuccess) == LC_SUCCESS, "status");
static_assert(static_cast<int>(rt::Status::kInvalidValue) == LC_INVALID_VALUE, "status");
static_assert(static_cast<int>(rt::Status::kOutOfMemory) == LC_OUT_OF_MEMORY, "status");
static_assert(static_cast<int>(rt::Status::kNotSupported) == LC_NOT_SUPPORTED, "status");
static_assert(static_cast<int>(rt::Status::kDriverError) == LC_DRIVER_ERROR, "status");
static_assert(static_cast<int>(rt::Status::kUnknown) == LC_UNKNOWN, "status");
"""


def test_wrappers_map_every_field(tmp_path):
    stubs = r"""
static lcAttentionConfig g_cfg;
static lcAttentionIoPolicy g_pol;
static lcMatMulIoPolicy g_mm;
static lcDeviceKind g_dev;
static float g_lr;
extern "C" lcError_t lcAttentionForwardWithPolicy(const float*, const float*, const float*, float*,
                                                  const lcAttentionConfig* c, lcDeviceKind d,
                                                  const lcAttentionIoPolicy* p) {
  g_cfg = *c; g_pol = *p; g_dev = d; return LC_NOT_SUPPORTED;
}
extern "C" lcError_t lcAttentionTrainStepWithPolicy(const float*, const float*, float*, const float*, float*,
                                                    float lr, const lcAttentionConfig* c, lcDeviceKind d, float*,
                                                    const lcAttentionIoPolicy* p) {
  g_cfg = *c; g_pol = *p; g_dev = d; g_lr = lr; return LC_DRIVER_ERROR;
}
extern "C" lcError_t lcMatMulWithPolicy(const float*, const float*, float*, size_t, size_t, size_t,
                                        lcDeviceKind d, const lcMatMulIoPolicy* p) {
  g_mm = *p; g_dev = d; return LC_OUT_OF_MEMORY;
}
"""
    main = _MAIN_COMMON + r"""
int main() {
  using namespace lightning_core;
  AttentionConfig cfg{77, 33, true};
  AttentionIoPolicy p;
  p.upload_q = false; p.upload_k = true; p.upload_v = false; p.upload_target = true;
  p.download_out = false; p.download_v = true; p.synchronize = false; p.loss_every = 7;
  p.output_scale = 2.5f; p.output_bias = -0.75f; p.output_relu = true;
  float x = 0.0f;
  CHECK(detail::attentionForwardHipWithPolicy(&x, &x, &x, &x, cfg, p) == rt::Status::kNotSupported);
  CHECK(g_dev == LC_DEVICE_HIP);
  CHECK(g_cfg.seq_len == 77 && g_cfg.head_dim == 33 && g_cfg.causal == 1);
  CHECK(g_pol.upload_q == 0 && g_pol.upload_k == 1 && g_pol.upload_v == 0 && g_pol.upload_target == 1);
  CHECK(g_pol.download_out == 0 && g_pol.download_v == 1 && g_pol.synchronize == 0 && g_pol.loss_every == 7);
  CHECK(g_pol.output_scale == 2.5f && g_pol.output_bias == -0.75f && g_pol.output_relu == 1);
  // the complementary pattern, through the train-step wrapper
  AttentionConfig cfg2{5, 9, false};
  AttentionIoPolicy q;
  q.upload_q = true; q.upload_k = false; q.upload_v = true; q.upload_target = false;
  q.download_out = true; q.download_v = false; q.synchronize = true; q.loss_every = 3;
  q.output_scale = -1.0f; q.output_bias = 4.0f; q.output_relu = false;
  CHECK(detail::attentionTrainStepHipWithPolicy(&x, &x, &x, &x, &x, 0.125f, cfg2, &x, q) ==
        rt::Status::kDriverError);
  CHECK(g_cfg.seq_len == 5 && g_cfg.head_dim == 9 && g_cfg.causal == 0 && g_lr == 0.125f);
  CHECK(g_pol.upload_q == 1 && g_pol.upload_k == 0 && g_pol.upload_v == 1 && g_pol.upload_target == 0);
  CHECK(g_pol.download_out == 1 && g_pol.download_v == 0 && g_pol.synchronize == 1 && g_pol.loss_every == 3);
  CHECK(g_pol.output_scale == -1.0f && g_pol.output_bias == 4.0f && g_pol.output_relu == 0);
  CHECK(detail::matMulHipWithPolicy(&x, &x, &x, 2, 3, 4, true, false, true, false) == rt::Status::kOutOfMemory);
  CHECK(g_mm.upload_a == 1 && g_mm.upload_b == 0 && g_mm.download_out == 1 && g_mm.synchronize == 0);
  CHECK(detail::matMulHipWithPolicy(&x, &x, &x, 2, 3, 4, false, true, false, true) == rt::Status::kOutOfMemory);
  CHECK(g_mm.upload_a == 0 && g_mm.upload_b == 1 && g_mm.download_out == 0 && g_mm.synchronize == 1);
  std::printf("fields ok\n");
  return 0;
}
"""
    out = _build_and_run(tmp_path, "binding_fields", _wrapper_block() + stubs + main, link_lib=False)
    assert "fields ok" in out


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_wrappers_reach_the_library(tmp_path):
    main = _MAIN_COMMON + r"""
int main() {
  using namespace lightning_core;
  const int hip = lcIsHipAvailable();
  std::vector<float> q(16 * 8, 0.5f), out(16 * 8, 0.0f);
  AttentionConfig cfg{16, 8, false};
  AttentionIoPolicy p;
  const rt::Status sa = detail::attentionForwardHipWithPolicy(q.data(), q.data(), q.data(), out.data(), cfg, p);
  std::vector<float> a(4 * 3, 1.0f), b(3 * 2, 1.0f), c(4 * 2, 0.0f);
  const rt::Status sm = detail::matMulHipWithPolicy(a.data(), b.data(), c.data(), 4, 3, 2, true, true, true, true);
  std::printf("hip=%d attention=%d matmul=%d\n", hip, static_cast<int>(sa), static_cast<int>(sm));
  if (!hip) {
    // no gfx950 device: the dispatcher's cue for its CPU fallback
    CHECK(sa == rt::Status::kNotSupported && sm == rt::Status::kNotSupported);
  } else {
    CHECK(sa == rt::Status::kSuccess && sm == rt::Status::kSuccess && c[0] == 3.0f);
  }
  return 0;
}
"""
    src = "#include <vector>\n" + _wrapper_block() + main
    out = _build_and_run(tmp_path, "binding_lib", src, link_lib=True)
    assert "hip=" in out


def test_reference_struct_sizes_match_the_library(tmp_path):
    prog = r"""
#include <cstdio>
#include "lightning_core/lightning_core.h"
int main() {
  std::printf("%zu %zu %zu %zu %zu %zu\n", sizeof(lcBackendCapabilities), sizeof(lcComputeInterfaceContract),
              sizeof(lcMemoryInterfaceContract), sizeof(lcSyncInterfaceContract),
              sizeof(lcProfilerInterfaceContract), sizeof(lcBackendInterfaceContract));
  return 0;
}
"""
    src = tmp_path / "sizes.cpp"
    exe = tmp_path / "sizes"
    src.write_text(prog)
    r = subprocess.run(["g++", "-std=c++17", "-I" + REF_INC, str(src), "-o", str(exe)], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    ref_sizes = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()]
    assert len(ref_sizes) == 6
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    lib = ctypes.CDLL(LIB)
    lib.lcGetStructSize.restype = ctypes.c_size_t
    lib.lcGetStructSize.argtypes = [ctypes.c_int]
    assert [lib.lcGetStructSize(i) for i in range(1, 7)] == ref_sizes
