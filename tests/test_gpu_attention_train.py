"""attention train step on the hip device vs the CPU oracle.

The step is the reference's dV-only SGD step (src/attention_cpu.cpp:114-163,
dispatch src/attention.cpp:203-244, session sampling :285-343): forward,
loss = mean((out - target)^2), v -= lr * P^T . 2 (out - target) / (S*D).
Checked: the golden vectors written from the compiled reference, seeded
shapes (C1's S=256 D=64, causal and not, odd sizes, S=2048 D=128), several
steps on the resident V, the loss_every sampling and the validation rules.

The update lr * dV is small next to V; it is compared on its own
(max |v_gpu - v_ref| against max |v_ref - v_before|), plus the fp32 rounding
of V itself.
"""
import ctypes

import numpy as np
import pytest

import oracle_lib
from gpu_util import assert_parity, note, require_hip
from lightning_core import synth

pytestmark = pytest.mark.gpu

UPDATE_TOL = 1e-3


@pytest.fixture(scope="module")
def lc():
    return require_hip()


def _check_step(what, ref, got, v0):
    out_r, v_r, loss_r = ref
    out_g, v_g, loss_g = got
    assert_parity(np.asarray(out_r).ravel(), np.asarray(out_g).ravel(), "f32", f"{what} out")
    v0 = np.asarray(v0, np.float64).ravel()
    v_r = np.asarray(v_r, np.float64).ravel()
    v_g = np.asarray(v_g, np.float64).ravel()
    upd = np.max(np.abs(v_r - v0))
    err = np.max(np.abs(v_g - v_r))
    slack = 4 * np.finfo(np.float32).eps * np.max(np.abs(v0))
    note(f"[parity] {what} update max|dv|={upd:.3e} err={err:.3e} ({err / max(upd, 1e-30):.2e} of the update)")
    assert err <= UPDATE_TOL * upd + slack
    note(f"[parity] {what} loss ref={loss_r:.6e} got={loss_g:.6e}")
    assert abs(loss_g - loss_r) <= 1e-4 * abs(loss_r)


@pytest.mark.parametrize("case", oracle_lib.golden_cases("train_attention"), ids=lambda c: c["name"])
def test_train_step_golden(lc, case):
    p = case["params"]
    s, d = p["seq_len"], p["head_dim"]
    q, k, v, t = (oracle_lib.golden_input(case, n) for n in ("q", "k", "v", "target"))
    sess = lc.AttentionSession(s, d, causal=p["causal"])
    got = sess.train_step(q, k, v, t, p["learning_rate"])
    exp = np.asarray(case["expected"], np.float32)
    _check_step(case["name"], (exp[:s * d], exp[s * d:2 * s * d], float(exp[-1])), got, v)
    sess.close()


@pytest.mark.parametrize("s,d,causal,lr", [(256, 64, False, 2.0), (256, 64, True, 2.0), (100, 33, True, 5.0),
                                           (7, 5, False, 1.0), (2048, 128, True, 50.0), (300, 256, False, 20.0)])
def test_train_step_shapes(lc, oracle, s, d, causal, lr):
    q, k, v, t = (synth.normal((s, d), stream=500 + i) for i in range(4))
    sess = lc.AttentionSession(s, d, causal=causal)
    got = sess.train_step(q, k, v, t, lr)
    ref = oracle.attention_train_step(q, k, v, t, lr, causal)
    _check_step(f"train S={s} D={d} causal={causal}", ref, got, v)
    sess.close()


def test_train_steps_on_resident_v(lc, oracle):
    # four steps that keep V on the device (upload_v / download_v off after
    # the first), then one that downloads: equals four oracle steps
    s, d, lr = 128, 64, 4.0
    q, k, v, t = (synth.normal((s, d), stream=520 + i) for i in range(4))
    sess = lc.AttentionSession(s, d, causal=True)
    first = lc.AttentionIoPolicy(download_out=False, download_v=False, synchronize=False)
    keep = lc.AttentionIoPolicy(upload_q=False, upload_k=False, upload_v=False, upload_target=False,
                                download_out=False, download_v=False, synchronize=False)
    last = lc.AttentionIoPolicy(upload_q=False, upload_k=False, upload_v=False, upload_target=False)
    sess.train_step_with_policy(q, k, v, t, lr, first)
    for _ in range(2):
        sess.train_step_with_policy(q, k, v, t, lr, keep)
    out_g, v_g, loss_g = sess.train_step_with_policy(q, k, v, t, lr, last)
    vr = np.asarray(v, np.float32)
    for _ in range(4):
        out_r, vr_next, loss_r = oracle.attention_train_step(q, k, vr, t, lr, True)
        v_prev, vr = vr, vr_next
    _check_step("4 resident steps", (out_r, vr, loss_r), (out_g, v_g, loss_g), v_prev)
    sess.close()


def test_plain_steps_in_a_row_then_resident_steps(lc, oracle):
    # Plain steps (every input uploaded, out and V downloaded) of up to 65536
    # values per tensor stage through pinned memory and wait on a completion
    # flag; a row of them with changing shapes, mixed with plain forward calls
    # that share the staging and the flag, each matches the oracle, and the V
    # a plain step leaves on the device feeds the next resident step.
    shapes = [(256, 64, False, 2.0), (100, 33, True, 5.0), (7, 5, False, 1.0), (255, 256, True, 20.0),
              (256, 64, True, 2.0)]
    for i, (s, d, causal, lr) in enumerate(shapes):
        q, k, v, t = (synth.normal((s, d), stream=900 + 4 * i + j) for j in range(4))
        sess = lc.AttentionSession(s, d, causal=causal)
        got = sess.train_step(q, k, v, t, lr)
        _check_step(f"plain step {i}: S={s} D={d} causal={causal}", oracle.attention_train_step(q, k, v, t, lr, causal),
                    got, v)
        fq, fk, fv = (synth.normal((64, 32), stream=950 + 3 * i + j) for j in range(3))
        assert_parity(oracle.attention(fq, fk, fv), lc.attention2d(fq, fk, fv), "f32", f"forward between steps {i}")
        if i == len(shapes) - 1:
            v1 = np.asarray(got[1], np.float32).reshape(s, d)
            keep = lc.AttentionIoPolicy(upload_q=False, upload_k=False, upload_v=False, upload_target=False)
            got2 = sess.train_step_with_policy(q, k, v, t, lr, keep)
            _check_step("resident step after a plain one", oracle.attention_train_step(q, k, v1, t, lr, causal), got2,
                        v1)
        sess.close()


@pytest.mark.parametrize("s,d,causal", [(256, 64, False), (100, 48, True)])
def test_train_run_cached_matches_steps(lc, s, d, causal):
    # train_run_cached(lr, n) (the C loop of resident steps) leaves the same V
    # as n resident train_step_with_policy calls: same kernels, same order.
    q, k, v, t = (synth.normal((s, d), stream=700 + i) for i in range(4))
    lr = 0.5
    up = lc.AttentionIoPolicy(download_out=False, download_v=False, synchronize=True)
    keep = lc.AttentionIoPolicy(upload_q=False, upload_k=False, upload_v=False, upload_target=False,
                                download_out=False, download_v=False, synchronize=False)
    get_v = lc.AttentionIoPolicy(upload_q=False, upload_k=False, upload_v=False, upload_target=False,
                                 download_out=True, download_v=True, synchronize=True)
    a = lc.AttentionSession(s, d, causal=causal)
    b = lc.AttentionSession(s, d, causal=causal)
    for sess in (a, b):
        sess.train_step_with_policy(q, k, v, t, lr, up)
    for _ in range(5):
        a.train_step_with_policy(q, k, v, t, lr, keep)
    b.train_run_cached(lr, 5)
    out_a, va, _ = a.train_step_with_policy(q, k, v.copy(), t, lr, get_v)
    out_b, vb, _ = b.train_step_with_policy(q, k, v.copy(), t, lr, get_v)
    np.testing.assert_array_equal(va, vb)
    np.testing.assert_array_equal(out_a, out_b)
    assert not np.array_equal(va, v)
    with pytest.raises(RuntimeError, match="invalid value"):
        b.train_run_cached(0.0, 1)
    fresh = lc.AttentionSession(s, d, causal=causal)
    with pytest.raises(RuntimeError, match="no resident input"):
        fresh.train_run_cached(lr, 1)
    for sess in (a, b, fresh):
        sess.close()


def test_loss_every_sampling(lc):
    # loss_every = 3: steps 0, 3, 6 measure the loss, the others repeat the
    # last measured value (src/attention.cpp:309-336)
    s, d, lr = 64, 32, 20.0
    q, k, v, t = (synth.normal((s, d), stream=530 + i) for i in range(4))
    sess = lc.AttentionSession(s, d)
    pol = lc.AttentionIoPolicy(loss_every=3)
    losses = []
    for _ in range(7):
        _, v, loss = sess.train_step_with_policy(q, k, v, t, lr, pol)
        losses.append(loss)
    note(f"[train] sampled losses {losses}")
    assert losses[1] == losses[0] and losses[2] == losses[0]
    assert losses[4] == losses[3] and losses[5] == losses[3]
    assert losses[3] < losses[0] and losses[6] < losses[3]  # SGD on V lowers the loss
    sess.close()


def test_train_step_validation(lc):
    s, d = 8, 4
    q = np.zeros((s, d), np.float32)
    sess = lc.AttentionSession(s, d)
    with pytest.raises(RuntimeError, match="invalid value"):
        sess.train_step(q, q, q, q, 0.0)  # learning_rate <= 0 (src/attention.cpp:229-232)
    sess.close()
    # the one-shot C entry rejects a null target whatever the policy
    lib = lc._core._lib()
    cfg = lc._native.AttentionConfig(s, d, 0)
    fp = q.ctypes.data_as(lc._native.FP)
    out = np.zeros((s, d), np.float32)
    st = lib.lcAttentionTrainStep(fp, fp, q.copy().ctypes.data_as(lc._native.FP), None,
                                  out.ctypes.data_as(lc._native.FP), 0.1, ctypes.byref(cfg), 3, None)
    assert st == 2  # LC_INVALID_VALUE


def test_one_shot_train_step_matches_session(lc, oracle):
    s, d, lr = 96, 48, 3.0
    q, k, v, t = (synth.normal((s, d), stream=540 + i) for i in range(4))
    lib = lc._core._lib()
    cfg = lc._native.AttentionConfig(s, d, 1)
    v_io = np.array(v, np.float32)
    out = np.zeros((s, d), np.float32)
    loss = ctypes.c_float(0.0)
    FP = lc._native.FP
    st = lib.lcAttentionTrainStep(q.ctypes.data_as(FP), k.ctypes.data_as(FP), v_io.ctypes.data_as(FP),
                                  t.ctypes.data_as(FP), out.ctypes.data_as(FP), lr, ctypes.byref(cfg), 3,
                                  ctypes.pointer(loss))
    assert st == 0
    _check_step("one-shot train", oracle.attention_train_step(q, k, v, t, lr, True), (out, v_io, loss.value), v)
