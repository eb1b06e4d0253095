"""The runtime device layer, threading and failure reporting on the hip device.

* lcMalloc / lcMemcpy (H2D, D2D, D2H) / lcDeviceSynchronize / lcFree round
  trip, bit-exact (reference src/runtime.cpp:193-298, tests/test_runtime.cpp:
  68-92, tests/test_matmul.cpp:107-135);
* backend name, preferred devices and the hip capability row once a gfx950
  device is visible (src/runtime.cpp:387-398);
* one AttentionSession driven by 4 threads, the reference's shared-session
  pattern (tests/test_attention.cpp:170-221), and the cached attention2d
  session used from 4 threads, both checked against the CPU oracle;
* the stream-K GEMM's bounded wait: with the spin limit forced to 0 from the
  host every owner gives up at once (every kernel still exits), the call
  reports LC_DRIVER_ERROR, and the next GEMM is correct;
* an allocation no device can hold reports LC_OUT_OF_MEMORY
  (src/runtime.cpp:193-214, the kOutOfMemory status);
* the in-flight cap of enqueue-only launches (matmul 256,
  src/ops/matmul_metal.mm:27, :1864-1878; attention 64,
  src/attention_metal.mm:26, :1448-1462): the capped call synchronises the
  stream and records a device_synchronize trace event, and the results of
  the enqueued launches match the oracle;
* the completion-flag wait of plain calls with host arrays (attention2d,
  matmul2d, the fused conv -> attention call): with its spin budget forced to
  0 from the host (CJ_HIP_DONE_WAIT_US, read once, so in a child process)
  every call takes the stream-sync path, and calls in a row stay right.
"""
import ctypes
import os
import subprocess
import sys
import textwrap
import threading

import numpy as np
import pytest

from gpu_util import assert_parity, note, require_hip
from lightning_core import _native as N
from lightning_core import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lc():
    return require_hip()


def test_device_memory_roundtrip(lc):
    lib = N.load()
    n = 1 << 20
    host = synth.uniform((n,), stream=71)
    back = np.zeros(n, np.float32)
    d0, d1 = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.lcMalloc(ctypes.byref(d0), n * 4) == N.LC_SUCCESS
    assert lib.lcMalloc(ctypes.byref(d1), n * 4) == N.LC_SUCCESS
    try:
        assert d0.value and d1.value and d0.value != d1.value
        assert lib.lcMemcpy(d0, host.ctypes.data_as(ctypes.c_void_p), n * 4,
                            N.LC_MEMCPY_HOST_TO_DEVICE) == N.LC_SUCCESS
        assert lib.lcMemcpy(d1, d0, n * 4, N.LC_MEMCPY_DEVICE_TO_DEVICE) == N.LC_SUCCESS
        assert lib.lcDeviceSynchronize() == N.LC_SUCCESS
        assert lib.lcMemcpy(back.ctypes.data_as(ctypes.c_void_p), d1, n * 4,
                            N.LC_MEMCPY_DEVICE_TO_HOST) == N.LC_SUCCESS
        np.testing.assert_array_equal(back, host)
        h2h = np.zeros(16, np.float32)
        assert lib.lcMemcpy(h2h.ctypes.data_as(ctypes.c_void_p), host.ctypes.data_as(ctypes.c_void_p), 64,
                            N.LC_MEMCPY_HOST_TO_HOST) == N.LC_SUCCESS
        np.testing.assert_array_equal(h2h, host[:16])
        # the reference's argument checks (runtime.cpp:193-214, :232-240)
        assert lib.lcMalloc(None, 16) == N.LC_INVALID_VALUE
        assert lib.lcMalloc(ctypes.byref(ctypes.c_void_p()), 0) == N.LC_INVALID_VALUE
        assert lib.lcMemcpy(None, d0, 4, N.LC_MEMCPY_DEVICE_TO_DEVICE) == N.LC_INVALID_VALUE
    finally:
        assert lib.lcFree(d0) == N.LC_SUCCESS
        assert lib.lcFree(d1) == N.LC_SUCCESS
    assert lib.lcFree(None) == N.LC_SUCCESS
    note("[runtime] lcMalloc/lcMemcpy H2D->D2D->D2H/lcFree: 4 MiB bit-exact")


def test_backend_identity_on_gpu(lc):
    lib = N.load()
    assert lc.backend_name() == "hip"
    dev = ctypes.c_int(-1)
    assert lib.lcGetPreferredDeviceForInference(ctypes.byref(dev)) == N.LC_SUCCESS and dev.value == N.LC_DEVICE_HIP
    assert lib.lcGetPreferredDeviceForTraining(ctypes.byref(dev)) == N.LC_SUCCESS and dev.value == N.LC_DEVICE_HIP
    count = ctypes.c_int(0)
    assert lib.lcGetDeviceCount(ctypes.byref(count)) == N.LC_SUCCESS and count.value >= 1
    caps = lc.runtime_backend_capabilities("hip")
    assert caps["built"] and caps["available"] and caps["compute_surface"] and caps["memory_surface"]
    assert lc.runtime_active_backend_capabilities()["device"] == "hip"
    assert lc.runtime_active_backend_interfaces()["memory"]["driver_tag"] == "hip.device_memory"
    info = lc.device_info()
    assert info["gcn_arch"].startswith("gfx950") and info["compute_units"] > 0
    note(f"[runtime] device {info['name']} {info['gcn_arch']} CUs={info['compute_units']}")


def test_shared_session_four_threads_train(lc, oracle):
    """tests/test_attention.cpp:170-221 on the hip device: 4 threads x 16 train
    steps on one session (loss_every = 2), each thread with its own V; every
    thread's last loss is finite and non-negative, and one more step from a
    known V matches the oracle."""
    s, d = 4, 4
    sess = lc.AttentionSession(s, d, causal=True)
    sess.set_default_policy(lc.AttentionIoPolicy(loss_every=2))
    q = np.full((s, d), 0.3, np.float32)
    k = np.full((s, d), 0.2, np.float32)
    t = np.zeros((s, d), np.float32)
    last = [None] * 4
    errors = []

    def worker(i):
        try:
            v = np.full((s, d), 0.1 + 0.01 * i, np.float32)
            loss = -1.0
            for _ in range(16):
                _, v, loss = sess.train_step(q, k, v, t, 0.01)
            last[i] = loss
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "a train-step thread did not finish"
    assert not errors, errors
    assert all(x is not None and np.isfinite(x) and x >= 0.0 for x in last), last
    qn, kn, vn, tn = (synth.normal((s, d), stream=80 + i) for i in range(4))
    out, v_new, loss = sess.train_step_with_policy(qn, kn, vn, tn, 0.5, lc.AttentionIoPolicy(loss_every=1))
    r_out, r_v, r_loss = oracle.attention_train_step(qn, kn, vn, tn, 0.5, True)
    assert_parity(r_out, out.reshape(s, d), "f32", "shared session after 4 threads: out")
    assert_parity(r_v, v_new.reshape(s, d), "f32", "shared session after 4 threads: v")
    assert abs(loss - r_loss) <= 1e-4 * max(abs(r_loss), 1e-6)
    sess.close()
    note(f"[threads] shared session: last losses {last}")


def test_cached_attention_session_four_threads(lc, oracle):
    """attention2d from 4 threads on the same (S, D) key: one cached session,
    concurrent calls, a cache clear in the middle; every result matches the
    oracle for that thread's inputs."""
    s, d = 96, 64
    inputs = [tuple(synth.normal((s, d), stream=90 + 3 * i + j) for j in range(3)) for i in range(4)]
    refs = [oracle.attention(*x, False) for x in inputs]
    errors = []
    barrier = threading.Barrier(4)

    def worker(i):
        try:
            barrier.wait(timeout=30)
            for it in range(12):
                got = lc.attention2d(*inputs[i], causal=False)
                err = np.abs(got - refs[i]).max() / np.abs(refs[i]).max()
                if not err <= 1e-4:
                    errors.append(f"thread {i} iter {it}: {err:.3e}")
                if i == 0 and it == 5:
                    lc.clear_attention2d_session_cache()
        except Exception as e:  # noqa: BLE001
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads)
    assert not errors, errors
    lc.clear_attention2d_session_cache()
    note("[threads] cached attention2d session: 4 threads x 12 calls match the oracle")


def test_streamk_wait_timeout_is_reported(lc, oracle):
    """CJ_HIP_STREAMK_SPIN_LIMIT=0: an owner never polls, so every split tile's
    owner gives up at once (no kernel waits); the launch's failure word turns
    into LC_DRIVER_ERROR at the sync.  The next GEMM (default limit) is right:
    flags carry a per-launch epoch, so what the failed launch left is never
    taken for ready."""
    m, k, n = 1000, 777, 1030
    a, b = synth.uniform((m, k), stream=1), synth.uniform((k, n), stream=2)
    ref = oracle.matmul(a, b)
    old = {v: os.environ.get(v) for v in ("CJ_HIP_GEMM_F32", "CJ_HIP_STREAMK_SPIN_LIMIT")}
    # another shape first, so the policy-level resident slot settles this
    # shape's variant afresh (under the forced stream-K choice)
    lc.matmul2d(np.ones((8, 8), np.float32), np.ones((8, 8), np.float32))
    os.environ["CJ_HIP_GEMM_F32"] = "sk"
    try:
        assert_parity(ref, lc.matmul2d(a, b), "f32", "stream-K before the forced timeout")
        os.environ["CJ_HIP_STREAMK_SPIN_LIMIT"] = "0"
        note("[case] stream-K forced timeout (spin limit 0)")
        with pytest.raises(lc.LightningCoreError) as ei:
            lc.matmul2d(a, b)
        assert ei.value.status == N.LC_DRIVER_ERROR and "stream-K" in str(ei.value)
        del os.environ["CJ_HIP_STREAMK_SPIN_LIMIT"]
        # the error was consumed: the device and the next launches are fine
        assert N.load().lcDeviceSynchronize() == N.LC_SUCCESS
        for _ in range(2):
            assert_parity(ref, lc.matmul2d(a, b), "f32", "stream-K after the forced timeout")
    finally:
        for key, val in old.items():
            if val is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = val


def test_oversize_malloc_reports_out_of_memory(lc):
    lib = N.load()
    p = ctypes.c_void_p()
    note("[case] lcMalloc of 1 PiB")
    assert lib.lcMalloc(ctypes.byref(p), 1 << 50) == N.LC_OUT_OF_MEMORY
    assert not p.value
    assert "hipMalloc" in lib.lcGetLastErrorMessage().decode()
    # the failure is not sticky: the next allocation and a sync succeed
    assert lib.lcMalloc(ctypes.byref(p), 4096) == N.LC_SUCCESS
    assert lib.lcFree(p) == N.LC_SUCCESS
    assert lib.lcDeviceSynchronize() == N.LC_SUCCESS


def _forced_syncs(op_code):
    return [e for e in lc_trace() if e["type"] == "device_synchronize" and e["detail1"] == 1
            and e["detail0"] == op_code]


def lc_trace():
    import lightning_core
    return lightning_core.runtime_trace_events()


def test_enqueue_only_launches_are_capped(lc, oracle):
    m, k, n = 96, 64, 80
    a, b = synth.uniform((m, k), stream=41), synth.uniform((k, n), stream=42)
    ref = oracle.matmul(a, b)
    lc.runtime_trace_enable(True)
    try:
        # upload once and synchronise, then 300 launch-only calls: the 256th
        # reaches the cap and synchronises; then a downloading call
        lc.matmul_with_policy(a, b, m, k, n, policy=lc.MatMulIoPolicy(True, True, False, True))
        lc.runtime_trace_clear()
        launch_only = lc.MatMulIoPolicy(False, False, False, False)
        note("[case] 300 enqueue-only matmul calls")
        for _ in range(300):
            lc.matmul_with_policy(None, None, m, k, n, policy=launch_only)
        forced = _forced_syncs(1)
        assert len(forced) == 1, forced
        assert forced[0]["size_bytes"] == 256 and forced[0]["status"] == lc_status_name(N.LC_SUCCESS)
        out = lc.matmul_with_policy(None, None, m, k, n, policy=lc.MatMulIoPolicy(False, False, True, True))
        assert_parity(ref, out.reshape(m, n), "f32", "matmul after 300 enqueue-only launches")
        # attention sessions: 100 launch-only forwards, the 64th synchronises
        s, d = 64, 32
        q, kk, v = (synth.normal((s, d), stream=43 + i) for i in range(3))
        sess = lc.AttentionSession(s, d, causal=True)
        sess.forward_with_policy(q, kk, v, lc.AttentionIoPolicy(download_out=False, synchronize=True))
        lc.runtime_trace_clear()
        pol = lc.AttentionIoPolicy(upload_q=False, upload_k=False, upload_v=False, download_out=False,
                                   synchronize=False)
        note("[case] 100 enqueue-only attention forwards")
        for _ in range(100):
            sess.forward_with_policy(q, kk, v, pol)
        forced = _forced_syncs(6)
        assert len(forced) == 1, forced
        assert forced[0]["size_bytes"] == 64
        got = sess.forward_with_policy(q, kk, v, lc.AttentionIoPolicy(upload_q=False, upload_k=False,
                                                                      upload_v=False))
        assert_parity(oracle.attention(q, kk, v, True), got.reshape(s, d), "f32",
                      "attention after 100 enqueue-only launches")
        sess.close()
    finally:
        lc.runtime_trace_enable(False)
        lc.runtime_trace_clear()


def lc_status_name(code):
    return N.load().lcGetErrorString(code).decode()


def test_done_flag_wait_falls_back_to_stream_sync(lc):
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = {k: v for k, v in os.environ.items() if not k.startswith("CJ_")}
    env["CJ_HIP_DONE_WAIT_US"] = "0"
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(root, "lightining-core_amd"), os.path.dirname(__file__),
                                         env.get("PYTHONPATH", "")])
    code = """
        import numpy as np
        import lightning_core as lc
        import oracle_lib
        from lightning_core import synth
        from gpu_util import assert_parity
        orc = oracle_lib.load()
        x = synth.normal((1, 3, 8, 8), stream=700)
        w = synth.normal((16, 3, 3, 3), std=0.3, stream=701)
        conv_ref = orc.conv_attention(x, w, None, 48, 48, (1, 1), (1, 1)).ravel()
        for i in range(6):
            s, d = ((64, 32), (256, 64), (33, 200))[i % 3]
            q, k, v = (synth.normal((s, d), stream=710 + 3 * i + j) for j in range(3))
            causal = i % 2 == 1
            assert_parity(orc.attention(q, k, v, causal), lc.attention2d(q, k, v, causal), "f32", f"attention {i}")
            m, kk, n = ((64, 64, 64), (100, 77, 130), (1, 5, 300))[i % 3]
            a, b = synth.uniform((m, kk), stream=740 + 2 * i), synth.uniform((kk, n), stream=741 + 2 * i)
            assert_parity(orc.matmul(a, b), lc.matmul2d(a, b), "f32", f"matmul {i}")
            got = np.asarray(lc.api.conv_attention_torchstrong_nchw(x, w, None, 48, 48, 1, 1, 1, 1)).ravel()
            assert_parity(conv_ref, got, "f32", f"conv attention {i}")
        print("ok")
    """
    note("[case] plain calls with the completion-flag spin budget 0 (child process)")
    r = subprocess.run([sys.executable, "-u", "-c", textwrap.dedent(code)], cwd=root, env=env, capture_output=True,
                       text=True, timeout=110)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout[-3000:] + r.stderr[-3000:]
