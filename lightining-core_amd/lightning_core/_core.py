"""Implementation of the lightning_core Python surface over the C ABI."""
from __future__ import annotations

import ctypes
import threading

import numpy as np

from . import _native as N

__all__ = [
    "AttentionIoPolicy", "AttentionSession", "MatMulIoPolicy", "MatMulResidentSession", "MatMulMetalResidentSession",
    "VitBlockSession", "HipTimer",
    "attention2d", "attention2d_into", "attention_forward", "attention_forward_with_policy", "attention2d_session",
    "clear_attention2d_session_cache", "attention_batched", "attention_implementation_name",
    "matmul2d", "matmul2d_into", "matmul", "matmul_np", "matmul_np_into", "matmul_with_policy",
    "matmul2d_resident_session", "matmul_reset_tuning", "conv2d_nchw", "vit_block",
    "matmul_np_with_policy", "matmul_np_into_with_policy", "conv2d_nchw_into",
    "runtime_backend_capabilities", "runtime_active_backend_capabilities", "runtime_backend_interfaces",
    "runtime_active_backend_interfaces", "runtime_backend_interface_contract", "backend_name", "is_hip_available",
    "hip_available", "cuda_available", "metal_available", "is_cuda_available", "is_metal_available",
    "memory_model_name", "runtime_sync_policy_set", "runtime_sync_policy_get", "runtime_sync_apply",
    "runtime_sync_apply_default", "device_info", "api_version", "runtime_trace_enable", "runtime_trace_enabled",
    "runtime_trace_clear", "runtime_trace_events", "runtime_trace_capacity", "runtime_trace_event_capacity",
    "runtime_trace_timeline", "decode_dispatch_detail",
    "tune_cache_save", "tune_cache_load", "tune_cache_size", "attention_tune_cache_save",
    "attention_tune_cache_load", "attention_reset_tuning", "attention_tune_cache_size",
    "preload_runtime_profile_env", "device_synchronize", "LightningCoreError",
]

_DEVICES = {"cpu": N.LC_DEVICE_CPU, "cuda": N.LC_DEVICE_CUDA, "metal": N.LC_DEVICE_METAL, "hip": N.LC_DEVICE_HIP}
_DEVICE_NAMES = {v: k for k, v in _DEVICES.items()}
_DTYPES = {"f32": N.LC_DTYPE_F32, "float32": N.LC_DTYPE_F32, "bf16": N.LC_DTYPE_BF16, "bfloat16": N.LC_DTYPE_BF16,
           "f16": N.LC_DTYPE_F16, "float16": N.LC_DTYPE_F16}


class LightningCoreError(RuntimeError):
    """A non-success lcError_t; `status` holds the code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class SessionClosedError(LightningCoreError):
    """A call on a session that close() (or the session-cache clear) ended."""


def _lib():
    return N.load()


def _parse_device(name: str) -> int:
    """python/bindings/bind_common.hpp:23-34, with "hip" added."""
    try:
        return _DEVICES[name]
    except KeyError:
        raise ValueError("device must be 'cpu', 'cuda', 'metal', or 'hip'") from None


def _parse_dtype(name: str) -> int:
    try:
        return _DTYPES[name]
    except KeyError:
        raise ValueError("compute_dtype must be 'f32', 'bf16' or 'f16'") from None


def _check(status: int) -> None:
    """bind_common.hpp:46-50: non-success -> RuntimeError(getErrorString)."""
    if status != N.LC_SUCCESS:
        lib = _lib()
        base = lib.lcGetErrorString(status).decode()
        detail = lib.lcGetLastErrorMessage().decode()
        raise LightningCoreError(status, f"{base}: {detail}" if detail else base)


def _f32(a) -> np.ndarray:
    """py::array_t<float, c_style | forcecast>."""
    return np.ascontiguousarray(a, dtype=np.float32)


try:  # the compiled buffer-address helper, built next to the C library
    from ._addr import addr as _addr
except ImportError:  # not built: numpy's own (slower) route
    _addr = None


def _fp(a):
    """Address of a C-contiguous array for a void* buffer parameter."""
    if a is None:
        return None
    return _addr(a) if _addr is not None else a.ctypes.data


def _require_2d(a: np.ndarray, name: str, what: str):
    if a.ndim != 2:
        raise ValueError(f"{name} must be a 2D float32 array shaped {what}")
    return a.shape


# --- policies -----------------------------------------------------------------

class AttentionIoPolicy:
    """AttentionIoPolicy (reference include/lightning_core/core/attention.hpp:16-32)."""

    _FIELDS = ("upload_q", "upload_k", "upload_v", "upload_target", "download_out", "download_v", "synchronize",
               "loss_every", "output_scale", "output_bias", "output_relu")

    def __init__(self, **kw):
        c = _lib().lcAttentionIoPolicyDefault()
        for f in self._FIELDS:
            v = getattr(c, f)
            setattr(self, f, float(v) if f.startswith("output_s") or f == "output_bias" else
                    (bool(v) if f not in ("loss_every",) else int(v)))
        for k, v in kw.items():
            if k not in self._FIELDS:
                raise TypeError(f"unknown policy field {k!r}")
            setattr(self, k, v)

    def _c(self) -> N.AttentionIoPolicyC:
        c = N.AttentionIoPolicyC()
        for f in self._FIELDS:
            v = getattr(self, f)
            setattr(c, f, float(v) if f in ("output_scale", "output_bias") else int(v))
        return c

    @classmethod
    def _from_c(cls, c):
        p = cls()
        for f in cls._FIELDS:
            v = getattr(c, f)
            setattr(p, f, float(v) if f in ("output_scale", "output_bias") else (int(v) if f == "loss_every" else
                                                                                     bool(v)))
        return p


class MatMulIoPolicy:
    """MatMulIoPolicy (reference include/lightning_core/core/ops/policy.hpp:8-13)."""

    def __init__(self, upload_a=True, upload_b=True, download_out=True, synchronize=True):
        self.upload_a = upload_a
        self.upload_b = upload_b
        self.download_out = download_out
        self.synchronize = synchronize

    def _c(self):
        return N.MatMulIoPolicyC(int(self.upload_a), int(self.upload_b), int(self.download_out),
                                 int(self.synchronize))


# --- attention ----------------------------------------------------------------

def attention_implementation_name(device: str = "hip") -> str:
    return _lib().lcAttentionImplementationName(_parse_device(device)).decode()


class AttentionSession:
    """AttentionSession (attention.hpp:86-129) with session-owned device buffers.

    `AttentionSession(seq_len, head_dim, causal=False, device="hip")` binds a
    single-head fp32 problem; `AttentionSession.batched(...)` binds batch*heads
    problems with a compute dtype.
    """

    def __init__(self, seq_len: int, head_dim: int, causal: bool = False, device: str = "hip", *, _batched=None):
        lib = _lib()
        h = ctypes.c_void_p()
        if _batched is None:
            cfg = N.AttentionConfig(seq_len, head_dim, int(causal))
            _check(lib.lcAttentionSessionCreate(ctypes.byref(cfg), _parse_device(device), ctypes.byref(h)))
            self.shape = (seq_len, head_dim)
        else:
            _check(lib.lcAttentionSessionCreateBatched(ctypes.byref(_batched), _parse_device(device),
                                                       ctypes.byref(h)))
            self.shape = (_batched.batch, _batched.heads, _batched.seq_len, _batched.head_dim)
        self._h = h
        # Held around every C call on the handle and around close(): ctypes
        # drops the GIL during a call, so without it another thread could
        # destroy the session while a call still uses it.  The library's
        # context mutex serialises the device work itself.
        self._lock = threading.RLock()
        self.causal = bool(causal)
        self.device = device

    @classmethod
    def batched(cls, batch, heads, seq_len, head_dim, causal=False, compute_dtype="bf16", device="hip"):
        cfg = N.AttentionBatchedConfig(batch, heads, seq_len, head_dim, int(causal), _parse_dtype(compute_dtype))
        return cls(seq_len, head_dim, causal, device, _batched=cfg)

    def _invoke(self, fname, *args):
        with self._lock:
            if not self._h.value:
                raise SessionClosedError(N.LC_INVALID_VALUE, "attention session is closed")
            return getattr(_lib(), fname)(self._h, *args)

    def close(self):
        lock = getattr(self, "_lock", None)
        if lock is None:
            return
        with lock:
            if self._h.value:
                _lib().lcAttentionSessionDestroy(self._h)
                self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def numel(self):
        return int(np.prod(self.shape))

    def set_default_policy(self, policy: AttentionIoPolicy):
        c = policy._c()
        _check(self._invoke("lcAttentionSessionSetDefaultPolicy", ctypes.byref(c)))

    def default_policy(self) -> AttentionIoPolicy:
        c = N.AttentionIoPolicyC()
        _check(self._invoke("lcAttentionSessionGetDefaultPolicy", ctypes.byref(c)))
        return AttentionIoPolicy._from_c(c)

    def _args(self, q, k, v):
        q, k, v = _f32(q), _f32(k), _f32(v)
        if q.size != self.numel or k.size != self.numel or v.size != self.numel:
            raise ValueError("q/k/v sizes must match")
        return q, k, v

    def forward(self, q, k, v):
        q, k, v = self._args(q, k, v)
        out = np.zeros(self.numel, np.float32)
        _check(self._invoke("lcAttentionSessionForward", _fp(q), _fp(k), _fp(v), _fp(out)))
        return out

    def forward_with_policy(self, q, k, v, policy: AttentionIoPolicy):
        q, k, v = self._args(q, k, v)
        out = np.zeros(self.numel, np.float32)
        c = policy._c()
        _check(self._invoke("lcAttentionSessionForwardWithPolicy", _fp(q), _fp(k), _fp(v), _fp(out),
                            ctypes.byref(c)))
        return out

    def forward_into(self, q, k, v, out):
        q, k, v = self._args(q, k, v)
        _require_out(out, self.numel)
        _check(self._invoke("lcAttentionSessionForward", _fp(q), _fp(k), _fp(v), _fp(out)))

    def forward_with_policy_into(self, q, k, v, out, policy: AttentionIoPolicy):
        q, k, v = self._args(q, k, v)
        _require_out(out, self.numel)
        c = policy._c()
        _check(self._invoke("lcAttentionSessionForwardWithPolicy", _fp(q), _fp(k), _fp(v), _fp(out),
                            ctypes.byref(c)))

    def run_cached(self, repeat_count: int = 1):
        """Launch-only repeat over the resident inputs, then synchronise."""
        _check(self._invoke("lcAttentionSessionRunCached", repeat_count))

    def train_run_cached(self, learning_rate: float, repeat_count: int = 1):
        """repeat_count resident train steps in C (no uploads, downloads or
        loss; V updated on the device), then synchronise: the loop of the
        reference's training benchmark (bench_attention.cpp:248-269)."""
        _check(self._invoke("lcAttentionSessionTrainRunCached", float(learning_rate), repeat_count))

    def _train_args(self, q, k, v, target):
        q, k, v = self._args(q, k, v)
        target = _f32(target)
        if target.size != self.numel:
            raise ValueError("q/k/v/target sizes must match")
        return q, k, v.copy(), target

    def train_step(self, q, k, v, target, learning_rate: float):
        """bind_attention.cpp:200-215: returns (out, updated v, loss); the
        caller's v is not modified (pybind takes it by value)."""
        q, k, v, target = self._train_args(q, k, v, target)
        out = np.zeros(self.numel, np.float32)
        loss = ctypes.c_float(0.0)
        _check(self._invoke("lcAttentionSessionTrainStep", _fp(q), _fp(k), _fp(v), _fp(target), _fp(out),
                            float(learning_rate), ctypes.pointer(loss)))
        return out, v, float(loss.value)

    def train_step_with_policy(self, q, k, v, target, learning_rate: float, policy: AttentionIoPolicy):
        """bind_attention.cpp:216-233."""
        q, k, v, target = self._train_args(q, k, v, target)
        out = np.zeros(self.numel, np.float32)
        loss = ctypes.c_float(0.0)
        c = policy._c()
        _check(self._invoke("lcAttentionSessionTrainStepWithPolicy", _fp(q), _fp(k), _fp(v), _fp(target), _fp(out),
                            float(learning_rate), ctypes.pointer(loss), ctypes.byref(c)))
        return out, v, float(loss.value)


def _require_out(out, n):
    if not isinstance(out, np.ndarray) or out.dtype != np.float32 or not out.flags.c_contiguous:
        raise ValueError("out must be a C-contiguous float32 numpy array")
    if out.size != n:
        raise ValueError("out size mismatch")


_session_cache: dict = {}
_session_cache_lock = threading.Lock()
_session_tls = threading.local()


def clear_attention2d_session_cache():
    """bind_attention.cpp:124-127.  Closes the cached sessions; a call already
    running on one finishes first (the session's own lock)."""
    with _session_cache_lock:
        sessions = list(_session_cache.values())
        _session_cache.clear()
    for s in sessions:
        s.close()


def _cached_session(seq_len, head_dim, causal, device):
    """bind_attention.cpp:36-69: one session per (S, D, causal, device), found
    through a per-thread last-session slot, else the shared map under a lock.

    The cached session uses the reference's one-shot policy (upload, download,
    synchronize) so every call is self-contained.
    """
    key = (seq_len, head_dim, bool(causal), device)
    slot = getattr(_session_tls, "slot", None)
    if slot is not None and slot[0] == key and slot[1]._h.value:
        return slot[1]
    with _session_cache_lock:
        s = _session_cache.get(key)
    if s is None:
        fresh = AttentionSession(seq_len, head_dim, causal, device)
        fresh.set_default_policy(AttentionIoPolicy())
        with _session_cache_lock:
            s = _session_cache.setdefault(key, fresh)
        if s is not fresh:  # another thread inserted one first
            fresh.close()
    _session_tls.slot = (key, s)
    return s


def _cached_forward_into(seq_len, head_dim, causal, device, q, k, v, out):
    """Forward on the cached session; if a concurrent cache clear closed it
    between lookup and call, the lookup runs once more (a new session)."""
    for attempt in range(2):
        try:
            _cached_session(seq_len, head_dim, causal, device).forward_into(q, k, v, out)
            return
        except SessionClosedError:
            if attempt:
                raise


def _attn2d_shapes(q, k, v):
    q, k, v = _f32(q), _f32(k), _f32(v)
    s, d = _require_2d(q, "q", "[seq_len, head_dim]")
    ks = _require_2d(k, "k", "[seq_len, head_dim]")
    vs = _require_2d(v, "v", "[seq_len, head_dim]")
    if ks != (s, d) or vs != (s, d):
        raise ValueError("q/k/v must have identical 2D shape [seq_len, head_dim]")
    return q, k, v, s, d


def attention2d(q, k, v, causal: bool = False, device: str = "hip"):
    """bind_attention.cpp:298-327."""
    q, k, v, s, d = _attn2d_shapes(q, k, v)
    out = np.empty((s, d), np.float32)
    _cached_forward_into(s, d, causal, _check_dev(device), q, k, v, out)
    return out


def attention2d_into(q, k, v, out, causal: bool = False, device: str = "hip"):
    """bind_attention.cpp:329-365."""
    q, k, v, s, d = _attn2d_shapes(q, k, v)
    if not isinstance(out, np.ndarray) or out.shape != (s, d):
        raise ValueError("out must be a 2D float32 array shaped [seq_len, head_dim]")
    _cached_forward_into(s, d, causal, _check_dev(device), q, k, v, out)


def attention_forward(q, k, v, seq_len: int, head_dim: int, causal: bool = False, device: str = "hip"):
    """bind_attention.cpp:234-276 (flat inputs)."""
    q, k, v = _f32(q).ravel(), _f32(k).ravel(), _f32(v).ravel()
    n = seq_len * head_dim
    for name, a in (("q", q), ("k", k), ("v", v)):
        if a.size != n:
            raise ValueError(f"{name} size mismatch")
    out = np.empty(n, np.float32)
    _cached_forward_into(seq_len, head_dim, causal, _check_dev(device), q, k, v, out)
    return out


def attention_forward_with_policy(q, k, v, seq_len: int, head_dim: int, causal: bool = False, device: str = "hip",
                                  policy: AttentionIoPolicy | None = None):
    """bind_attention.cpp:278-296."""
    q, k, v = _f32(q).ravel(), _f32(k).ravel(), _f32(v).ravel()
    n = seq_len * head_dim
    if q.size != n or k.size != n or v.size != n:
        raise ValueError("q/k/v length must match seq_len * head_dim")
    policy = policy or AttentionIoPolicy()
    out = np.zeros(n, np.float32)
    cfg = N.AttentionConfig(seq_len, head_dim, int(causal))
    c = policy._c()
    _check(_lib().lcAttentionForwardWithPolicy(_fp(q), _fp(k), _fp(v), _fp(out), ctypes.byref(cfg),
                                               _parse_device(device), ctypes.byref(c)))
    return out


def attention2d_session(q, causal: bool = False, device: str = "hip"):
    """bind_attention.cpp:367-378."""
    q = _f32(q)
    s, d = _require_2d(q, "q", "[seq_len, head_dim]")
    return AttentionSession(s, d, causal, device)


def attention_batched(q, k, v, causal: bool = False, compute_dtype: str = "bf16", device: str = "hip",
                      policy: AttentionIoPolicy | None = None):
    """Multi-head attention over [batch, heads, S, D] (new surface; fp32 in/out,
    inputs rounded to compute_dtype on upload, fp32 accumulate)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    if q.ndim != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q/k/v must have identical 4D shape [batch, heads, seq_len, head_dim]")
    b, h, s, d = q.shape
    cfg = N.AttentionBatchedConfig(b, h, s, d, int(causal), _parse_dtype(compute_dtype))
    out = np.empty_like(q)
    pc = (policy or AttentionIoPolicy())._c()
    _check(_lib().lcAttentionForwardBatched(_fp(q), _fp(k), _fp(v), _fp(out), ctypes.byref(cfg),
                                            _parse_device(device), ctypes.byref(pc)))
    return out


def _check_dev(device):
    _parse_device(device)
    return device


# --- matmul -------------------------------------------------------------------

def _mm_policy_call(a, b, out, m, k, n, device, policy):
    pc = policy._c()
    _check(_lib().lcMatMulWithPolicy(_fp(a), _fp(b), _fp(out), m, k, n, _parse_device(device), ctypes.byref(pc)))


def matmul2d(a, b, device: str = "hip"):
    """bind_ops.cpp:1164-1185."""
    a, b = _f32(a), _f32(b)
    m, k = _require_2d(a, "a", "[m, k]")
    kb, n = _require_2d(b, "b", "[k, n]")
    if k != kb:
        raise ValueError("matmul2d shape mismatch: a.shape[1] must equal b.shape[0]")
    out = np.empty((m, n), np.float32)
    _mm_policy_call(a, b, out, m, k, n, device, MatMulIoPolicy())
    return out


def matmul2d_into(a, b, out, device: str = "hip"):
    """bind_ops.cpp:1187-1209 (out may be 2-D [m, n] or flat)."""
    a, b = _f32(a), _f32(b)
    m, k = _require_2d(a, "a", "[m, k]")
    kb, n = _require_2d(b, "b", "[k, n]")
    if k != kb:
        raise ValueError("matmul2d_into shape mismatch: a.shape[1] must equal b.shape[0]")
    _require_out(out, m * n)
    _mm_policy_call(a, b, out, m, k, n, device, MatMulIoPolicy())


def matmul(a, b, m: int, k: int, n: int, device: str = "hip"):
    """bind_ops.cpp:550-589 (flat inputs, flat output)."""
    a, b = _f32(a).ravel(), _f32(b).ravel()
    if a.size != m * k or b.size != k * n:
        raise ValueError("a or b shape mismatch")
    out = np.empty(m * n, np.float32)
    _mm_policy_call(a, b, out, m, k, n, device, MatMulIoPolicy())
    return out


matmul_np = matmul


def matmul_np_into(a, b, out, m: int, k: int, n: int, device: str = "hip"):
    """bind_ops.cpp:610-633."""
    a, b = _f32(a).ravel(), _f32(b).ravel()
    if a.size != m * k or b.size != k * n:
        raise ValueError("a or b shape mismatch")
    if out.size != m * n:
        raise ValueError("out shape mismatch")
    _require_out(out, m * n)
    _mm_policy_call(a, b, out, m, k, n, device, MatMulIoPolicy())


def _policy_operands(a, b, m, k, n, policy):
    """bind_ops.cpp:635-726: a and b must hold m*k and k*n floats.  Here an
    operand may also be None: the C entry then uses the resident one when the
    policy does not upload it, and answers "invalid value" when it does
    (ops.hpp:367-370).  An operand that is given is checked all the same."""
    a = None if a is None else _f32(a).ravel()
    b = None if b is None else _f32(b).ravel()
    if (a is not None and a.size != m * k) or (b is not None and b.size != k * n):
        raise ValueError("a or b shape mismatch")
    return a, b


def matmul_with_policy(a, b, m: int, k: int, n: int, device: str = "hip", policy: MatMulIoPolicy | None = None,
                       out=None):
    """bind_ops.cpp:635-675 (ops::matMulWithPolicy<float>): returns `out`
    (allocated when None and the policy downloads; else checked: a C-contiguous
    float32 array of m*n values)."""
    policy = policy or MatMulIoPolicy()
    a, b = _policy_operands(a, b, m, k, n, policy)
    if out is None:
        if policy.download_out:
            out = np.zeros(m * n, np.float32)
    else:
        _require_out(out, m * n)
    _mm_policy_call(a, b, out, m, k, n, device, policy)
    return out


def matmul_np_with_policy(a, b, m: int, k: int, n: int, device: str = "hip", policy: MatMulIoPolicy | None = None):
    """bind_ops.cpp:677-699: flat float32 result of m*n values."""
    policy = policy or MatMulIoPolicy()
    a, b = _policy_operands(a, b, m, k, n, policy)
    out = np.zeros(m * n, np.float32)
    _mm_policy_call(a, b, out, m, k, n, device, policy)
    return out


def matmul_np_into_with_policy(a, b, out, m: int, k: int, n: int, device: str = "hip",
                               policy: MatMulIoPolicy | None = None):
    """bind_ops.cpp:701-726."""
    policy = policy or MatMulIoPolicy()
    a, b = _policy_operands(a, b, m, k, n, policy)
    if not isinstance(out, np.ndarray) or out.size != m * n:
        raise ValueError("out shape mismatch")
    _require_out(out, m * n)
    _mm_policy_call(a, b, out, m, k, n, device, policy)


def matmul_reset_tuning():
    _check(_lib().lcMatMulResetTuning())


class MatMulResidentSession:
    """MatMulMetalResidentSession<float> (ops.hpp:1339-1379) on the hip device,
    with session-owned device buffers and a compute dtype."""

    def __init__(self, m: int, k: int, n: int, compute_dtype: str = "f32"):
        h = ctypes.c_void_p()
        _check(_lib().lcMatMulResidentSessionCreate(m, k, n, _parse_dtype(compute_dtype), ctypes.byref(h)))
        self._h = h
        self.m, self.k, self.n = m, k, n
        self.compute_dtype = compute_dtype

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            _lib().lcMatMulResidentSessionDestroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _ab(self, a, b):
        a = None if a is None else _f32(a).ravel()
        b = None if b is None else _f32(b).ravel()
        if a is not None and a.size != self.m * self.k:
            raise ValueError("a size mismatch")
        if b is not None and b.size != self.k * self.n:
            raise ValueError("b size mismatch")
        return a, b

    def _out(self, out):
        if out is None:
            return np.zeros(self.m * self.n, np.float32)
        _require_out(out, self.m * self.n)
        return out

    def start_into(self, a, b, out=None):
        a, b = self._ab(a, b)
        out = self._out(out)
        _check(_lib().lcMatMulResidentSessionStart(self._h, _fp(a), _fp(b), _fp(out)))
        return out

    def run_into(self, a=None, b=None, out=None):
        _check(_lib().lcMatMulResidentSessionRun(self._h, None, None, None))
        return out

    def finish_into(self, a=None, b=None, out=None):
        out = self._out(out)
        _check(_lib().lcMatMulResidentSessionFinish(self._h, None, None, _fp(out)))
        return out

    def sync_into(self, a=None, b=None, out=None):
        _check(_lib().lcMatMulResidentSessionSync(self._h, None, None, None))
        return out

    def run_batch_sync_into(self, a, b, out, repeat_count: int):
        a, b = self._ab(a, b)
        out = self._out(out)
        _check(_lib().lcMatMulResidentSessionRunBatchSync(self._h, _fp(a), _fp(b), _fp(out), repeat_count))

    def run_batch_sync_no_download_into(self, a, b, out, repeat_count: int):
        _check(_lib().lcMatMulResidentSessionRunBatchSyncNoDownload(self._h, None, None, None, repeat_count))

    def run_batch_sync_cached_no_download(self, repeat_count: int):
        _check(_lib().lcMatMulResidentSessionRunBatchSyncCachedNoDownload(self._h, repeat_count))

    def time_launches(self, count: int) -> np.ndarray:
        """Per-launch durations (ms) of `count` launch-only GEMMs on the resident
        inputs, a hipEvent pair around each (measurement helper; no reference
        counterpart)."""
        ms = np.zeros(count, np.float32)
        _check(_lib().lcMatMulResidentSessionTimeLaunches(self._h, count, ms.ctypes.data_as(ctypes.c_void_p)))
        return ms

    def kernel_name(self) -> str:
        """"<tune-cache variant> <kernel function>" of the GEMM this shape runs."""
        buf = ctypes.create_string_buffer(128)
        _check(_lib().lcMatMulResidentSessionKernelName(self._h, buf, len(buf)))
        return buf.value.decode()

    # reference list-returning names (bind_ops.cpp:196-240)
    def start(self, a, b, out_size=None):
        return self.start_into(a, b)

    def run(self, a=None, b=None, out_size=None):
        self.run_into()
        return np.zeros(self.m * self.n, np.float32)

    def finish(self, a=None, b=None, out_size=None):
        return self.finish_into()

    def sync(self, a=None, b=None, out_size=None):
        self.sync_into()
        return np.zeros(self.m * self.n, np.float32)


MatMulMetalResidentSession = MatMulResidentSession


def matmul2d_resident_session(a, b, compute_dtype: str = "f32"):
    """bind_ops.cpp:1211-1226."""
    a, b = _f32(a), _f32(b)
    m, k = _require_2d(a, "a", "[m, k]")
    kb, n = _require_2d(b, "b", "[k, n]")
    if k != kb:
        raise ValueError("matmul2d_resident_session shape mismatch: a.shape[1] must equal b.shape[0]")
    return MatMulResidentSession(m, k, n, compute_dtype)


# --- conv / vit -----------------------------------------------------------------

def _conv_geometry(x, w, stride_h, stride_w, pad_h, pad_w):
    """bind_ops.cpp:737-765 / :818-846: validation and output size."""
    bn, c, h, wd = x.shape
    oc, wc, kh, kw = w.shape
    if c != wc:
        raise ValueError("x channels and w in_channels mismatch")
    if stride_h == 0 or stride_w == 0:
        raise ValueError("stride must be > 0")
    if h + 2 * pad_h < kh or wd + 2 * pad_w < kw:
        raise ValueError("invalid padding/kernel for input size")
    oh = (h + 2 * pad_h - kh) // stride_h + 1
    ow = (wd + 2 * pad_w - kw) // stride_w + 1
    return (bn, c, h, wd, oc, kh, kw), (bn, oc, oh, ow)


def _conv_bias(bias, oc):
    if bias is None:
        return None
    b = _f32(bias).ravel()
    if b.size != oc:
        raise ValueError("bias shape mismatch")
    return b


def _conv_call(x, w, b, out, dims, stride_h, stride_w, pad_h, pad_w, device, apply_relu):
    bn, c, h, wd, oc, kh, kw = dims
    _check(_lib().lcConv2dNchw(_fp(x), _fp(w), _fp(b), _fp(out), bn, c, h, wd, oc, kh, kw, stride_h, stride_w, pad_h,
                               pad_w, _parse_device(device), int(apply_relu)))


def conv2d_nchw(x, w, bias=None, stride_h=1, stride_w=1, pad_h=0, pad_w=0, device: str = "hip",
                apply_relu: bool = False):
    """ops::conv2dNchw<float> (ops.hpp:855-1213), bind_ops.cpp:728-804:
    x [B,C,H,W], w [OC,C,KH,KW] -> [B,OC,OH,OW].  `apply_relu` is the
    C++ entry's flag (default off, as there)."""
    x, w = _f32(x), _f32(w)
    if x.ndim != 4 or w.ndim != 4:
        raise ValueError("x and w must be 4D arrays (NCHW and OIHW)")
    dims, oshape = _conv_geometry(x, w, stride_h, stride_w, pad_h, pad_w)
    b = _conv_bias(bias, dims[4])
    out = np.empty(oshape, np.float32)
    _conv_call(x, w, b, out, dims, stride_h, stride_w, pad_h, pad_w, device, apply_relu)
    return out


def conv2d_nchw_into(x, w, bias, out, stride_h=1, stride_w=1, pad_h=0, pad_w=0, device: str = "hip",
                     apply_relu: bool = False):
    """bind_ops.cpp:806-888: writes into a 4-D float32 `out` of the output shape."""
    x, w = _f32(x), _f32(w)
    if x.ndim != 4 or w.ndim != 4 or not isinstance(out, np.ndarray) or out.ndim != 4:
        raise ValueError("x, w, out must be 4D arrays")
    dims, oshape = _conv_geometry(x, w, stride_h, stride_w, pad_h, pad_w)
    if tuple(out.shape) != oshape:
        raise ValueError("out shape mismatch")
    _require_out(out, out.size)
    b = _conv_bias(bias, dims[4])
    _conv_call(x, w, b, out, dims, stride_h, stride_w, pad_h, pad_w, device, apply_relu)


class VitBlockSession:
    """ViT-style block: patch-embed conv + ReLU -> QKV -> per-head attention ->
    output projection, resident weights (new composition surface)."""

    def __init__(self, batch, in_channels, image_h, image_w, patch, embed, heads, compute_dtype="f16",
                 device="hip"):
        self.cfg = N.VitBlockConfig(batch, in_channels, image_h, image_w, patch, embed, heads,
                                    _parse_dtype(compute_dtype))
        h = ctypes.c_void_p()
        _check(_lib().lcVitBlockSessionCreate(ctypes.byref(self.cfg), _parse_device(device), ctypes.byref(h)))
        self._h = h
        self.tokens = ((image_h - patch) // patch + 1) * ((image_w - patch) // patch + 1)
        self.out_shape = (batch, self.tokens, embed)
        self.in_shape = (batch, in_channels, image_h, image_w)

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            _lib().lcVitBlockSessionDestroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_weights(self, w_conv, w_qkv, w_o):
        w_conv, w_qkv, w_o = _f32(w_conv), _f32(w_qkv), _f32(w_o)
        e = self.cfg.embed
        if w_conv.size != e * self.cfg.in_channels * self.cfg.patch ** 2 or w_qkv.size != e * 3 * e or \
                w_o.size != e * e:
            raise ValueError("weight shape mismatch")
        _check(_lib().lcVitBlockSessionSetWeights(self._h, _fp(w_conv), _fp(w_qkv), _fp(w_o)))

    def forward(self, x=None, download=True):
        xa = None
        if x is not None:
            xa = _f32(x)
            if xa.shape != self.in_shape:
                raise ValueError("x shape mismatch")
        out = np.empty(self.out_shape, np.float32) if download else None
        _check(_lib().lcVitBlockSessionForward(self._h, _fp(xa), _fp(out)))
        return out

    def run_cached(self, repeat_count: int = 1):
        _check(_lib().lcVitBlockSessionRunCached(self._h, repeat_count))


def vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype="f16", device="hip"):
    x = _f32(x)
    bn, c, h, w = x.shape
    e, _, p, _ = np.shape(w_conv)
    s = VitBlockSession(bn, c, h, w, p, e, heads, compute_dtype, device)
    try:
        s.set_weights(w_conv, w_qkv, w_o)
        return s.forward(x)
    finally:
        s.close()


# --- runtime ------------------------------------------------------------------

def _caps_dict(c) -> dict:
    return {"device": _DEVICE_NAMES.get(c.device, str(c.device)), "built": bool(c.built),
            "available": bool(c.available), "compute_surface": bool(c.compute_surface),
            "memory_surface": bool(c.memory_surface), "sync_surface": bool(c.sync_surface),
            "profiling_surface": bool(c.profiling_surface), "runtime_trace_surface": bool(c.runtime_trace_surface),
            "sync_policy_surface": bool(c.sync_policy_surface),
            "memory_model": _lib().lcGetMemoryModelName(c.memory_model).decode()}


def runtime_backend_capabilities(device: str = "hip") -> dict:
    """bind_runtime.cpp:421-425."""
    c = N.BackendCapabilities()
    _check(_lib().lcGetBackendCapabilities(_parse_device(device), ctypes.byref(c)))
    return _caps_dict(c)


def runtime_active_backend_capabilities() -> dict:
    """bind_runtime.cpp:426-427."""
    c = N.BackendCapabilities()
    _check(_lib().lcGetActiveBackendCapabilities(ctypes.byref(c)))
    return _caps_dict(c)


def _contract_dict(c) -> dict:
    """bind_runtime.cpp:39-77 (toBackendInterfaceContractDict)."""
    model = _lib().lcGetMemoryModelName
    return {"device": _DEVICE_NAMES.get(c.device, str(c.device)), "capabilities": _caps_dict(c.capabilities),
            "compute": {"available": bool(c.compute.available),
                        "op_dispatch_trace_surface": bool(c.compute.op_dispatch_trace_surface),
                        "driver_tag": c.compute.driver_tag.decode()},
            "memory": {"available": bool(c.memory.available), "allocator_surface": bool(c.memory.allocator_surface),
                       "memcpy_surface": bool(c.memory.memcpy_surface),
                       "memory_model": model(c.memory.memory_model).decode(),
                       "driver_tag": c.memory.driver_tag.decode()},
            "sync": {"available": bool(c.sync.available), "sync_policy_surface": bool(c.sync.sync_policy_surface),
                     "trace_sync_boundary_surface": bool(c.sync.trace_sync_boundary_surface),
                     "driver_tag": c.sync.driver_tag.decode()},
            "profiler": {"available": bool(c.profiler.available),
                         "runtime_trace_surface": bool(c.profiler.runtime_trace_surface),
                         "op_dispatch_trace_surface": bool(c.profiler.op_dispatch_trace_surface),
                         "trace_capacity": c.profiler.trace_capacity, "driver_tag": c.profiler.driver_tag.decode()}}


def runtime_backend_interfaces(device: str = "hip") -> dict:
    """bind_runtime.cpp:428-432."""
    c = N.BackendInterfaceContract()
    _check(_lib().lcGetBackendInterfaceContract(_parse_device(device), ctypes.byref(c)))
    return _contract_dict(c)


def runtime_active_backend_interfaces() -> dict:
    """bind_runtime.cpp:433-434."""
    c = N.BackendInterfaceContract()
    _check(_lib().lcGetActiveBackendInterfaceContract(ctypes.byref(c)))
    return _contract_dict(c)


runtime_backend_interface_contract = runtime_backend_interfaces


def backend_name() -> str:
    """bind_runtime.cpp:392."""
    return _lib().lcBackendName().decode()


def is_hip_available() -> bool:
    return bool(_lib().lcIsHipAvailable())


def cuda_available() -> bool:
    """bind_runtime.cpp:390."""
    return bool(_lib().lcIsCudaAvailable())


def metal_available() -> bool:
    """bind_runtime.cpp:391."""
    return bool(_lib().lcIsMetalAvailable())


hip_available = is_hip_available
is_cuda_available = cuda_available
is_metal_available = metal_available


def memory_model_name() -> str:
    """bind_runtime.cpp:393-394."""
    lib = _lib()
    return lib.lcGetMemoryModelName(lib.lcGetMemoryModel()).decode()


_SYNC_MODES = {"auto": 0, "always": 1, "never": 2}
_SYNC_MODE_NAMES = {v: k for k, v in _SYNC_MODES.items()}


def _sync_policy(mode, trace_sync_boundary):
    """bind_runtime.cpp:11-22 (parseSyncMode)."""
    if mode not in _SYNC_MODES:
        raise ValueError("sync mode must be 'auto', 'always', or 'never'")
    return N.SyncPolicy(_SYNC_MODES[mode], int(bool(trace_sync_boundary)))


def runtime_sync_policy_set(mode: str = "auto", trace_sync_boundary: bool = False):
    """bind_runtime.cpp:395-403."""
    _check(_lib().lcSetDefaultSyncPolicy(_sync_policy(mode, trace_sync_boundary)))


def runtime_sync_policy_get() -> dict:
    """bind_runtime.cpp:404-410."""
    p = _lib().lcGetDefaultSyncPolicy()
    return {"mode": _SYNC_MODE_NAMES.get(p.mode, "auto"), "trace_sync_boundary": bool(p.trace_sync_boundary)}


def runtime_sync_apply(mode: str = "auto", trace_sync_boundary: bool = False):
    """bind_runtime.cpp:411-419 (deviceSynchronizeWithPolicy)."""
    _check(_lib().lcApplySyncPolicy(_sync_policy(mode, trace_sync_boundary)))


def runtime_sync_apply_default():
    """bind_runtime.cpp:420."""
    _check(_lib().lcApplyDefaultSyncPolicy())


def device_synchronize():
    _check(_lib().lcDeviceSynchronize())


def device_info() -> dict:
    d = N.HipDeviceInfo()
    _check(_lib().lcHipGetDeviceInfo(ctypes.byref(d)))
    return {"name": d.name.decode(), "gcn_arch": d.gcn_arch.decode(), "compute_units": d.compute_units,
            "max_clock_khz": d.max_clock_khz, "total_memory_bytes": d.total_memory_bytes,
            "l2_cache_bytes": d.l2_cache_bytes}


def api_version():
    a, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(_lib().lcGetApiVersion(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
    return (a.value, b.value, c.value)


def runtime_trace_enable(enabled: bool = True):
    """bind_runtime.cpp:435."""
    _lib().lcSetRuntimeTraceEnabled(int(enabled))


def runtime_trace_enabled() -> bool:
    """bind_runtime.cpp:436."""
    return bool(_lib().lcIsRuntimeTraceEnabled())


def runtime_trace_clear():
    """bind_runtime.cpp:437."""
    _lib().lcClearRuntimeTraceEvents()


def runtime_trace_capacity() -> int:
    """bind_runtime.cpp:438."""
    return int(_lib().lcGetRuntimeTraceEventCapacity())


runtime_trace_event_capacity = runtime_trace_capacity


def decode_dispatch_detail(encoded: int):
    r, s, f = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    if not _lib().lcDecodeRuntimeTraceDispatchDetail(encoded, ctypes.byref(r), ctypes.byref(s), ctypes.byref(f)):
        return None
    return {"requested": _DEVICE_NAMES[r.value], "selected": _DEVICE_NAMES[s.value], "fallback": bool(f.value)}


def _raw_trace_events():
    lib = _lib()
    n = lib.lcGetRuntimeTraceEvents(None, 0)
    arr = (N.RuntimeTraceEvent * max(n, 1))()
    got = lib.lcGetRuntimeTraceEvents(arr, n)
    return lib, arr[:got]


def _trace_row(lib, ev) -> dict:
    """One event with its op-dispatch fields decoded (bind_runtime.cpp:117-141,
    :439-464); op and devices are "" for other event types."""
    row = {"type": lib.lcRuntimeTraceEventTypeName(ev.type).decode(),
           "status": lib.lcGetErrorString(ev.status).decode(), "timestamp_ns": int(ev.timestamp_ns),
           "size_bytes": int(ev.size_bytes), "detail0": int(ev.detail0), "detail1": int(ev.detail1),
           "op": "", "requested_device": "", "selected_device": "", "fallback": False}
    if row["type"] == "op_dispatch":
        row["op"] = lib.lcRuntimeTraceOpKindName(ev.detail0).decode()
        d = decode_dispatch_detail(ev.detail1)
        if d is not None:
            row["requested_device"] = d["requested"]
            row["selected_device"] = d["selected"]
            row["fallback"] = d["fallback"]
    return row


def runtime_trace_events() -> list:
    """bind_runtime.cpp:439-464: events as dicts, oldest first."""
    lib, events = _raw_trace_events()
    return [_trace_row(lib, ev) for ev in events]


_EVENT_SORT_KEYS = ("index", "timestamp_ns", "offset_ns", "delta_prev_ns", "delta_next_ns", "size_bytes")
_GROUP_SORT_KEYS = ("key", "count", "total_delta_next_ns", "avg_delta_next_ns", "max_delta_next_ns",
                    "total_size_bytes")


def _timeline_group_key(row, group_by):
    """bind_runtime.cpp:180-206 (makeGroupKey)."""
    if group_by == "type":
        return row["type"]
    if group_by == "status":
        return row["status"]
    if group_by == "type_status":
        return row["type"] + "|" + row["status"]
    if group_by in ("op", "op_selected_device", "op_path"):
        if not row["op"]:
            return "non_op"
        if group_by == "op":
            return row["op"]
        sel = row["selected_device"] or "unknown"
        if group_by == "op_selected_device":
            return row["op"] + "|" + sel
        return row["op"] + "|" + sel + "|" + ("fallback" if row["fallback"] else "direct")
    raise ValueError("group_by must be one of: type, status, type_status, op, op_selected_device, op_path")


def _sorted_stable(rows, value, tie, descending):
    """std::stable_sort with orderedLess on (value, then tie): descending
    reverses both comparisons, as the reference's comparator does."""
    return sorted(rows, key=lambda r: (value(r), tie(r)), reverse=descending)


def runtime_trace_timeline(event_sort_by: str = "timestamp_ns", event_descending: bool = False,
                           group_by: str = "type", group_sort_by: str = "total_delta_next_ns",
                           group_descending: bool = True, hotspot_top_k: int = 8) -> dict:
    """bind_runtime.cpp:465-529: the trace as a timeline (offsets and gaps
    between consecutive events), grouped, with the largest gaps as hotspots."""
    if event_sort_by not in _EVENT_SORT_KEYS:
        raise ValueError("event_sort_by must be one of: " + ", ".join(_EVENT_SORT_KEYS))
    if group_sort_by not in _GROUP_SORT_KEYS:
        raise ValueError("group_sort_by must be one of: " + ", ".join(_GROUP_SORT_KEYS))
    lib, events = _raw_trace_events()
    rows = []
    base = events[0].timestamp_ns if events else 0
    for i, ev in enumerate(events):
        row = _trace_row(lib, ev)
        ts = row["timestamp_ns"]
        prev_ts = events[i - 1].timestamp_ns if i > 0 else None
        next_ts = events[i + 1].timestamp_ns if i + 1 < len(events) else None
        row["index"] = i
        row["offset_ns"] = ts - base if ts >= base else 0
        row["delta_prev_ns"] = ts - prev_ts if prev_ts is not None and ts >= prev_ts else 0
        row["delta_next_ns"] = next_ts - ts if next_ts is not None and next_ts >= ts else 0
        rows.append(row)
    out = {"event_count": len(rows), "event_sort_by": event_sort_by, "event_descending": bool(event_descending),
           "group_by": group_by, "group_sort_by": group_sort_by, "group_descending": bool(group_descending),
           "hotspot_top_k": int(hotspot_top_k),
           "notes": "delta_next_ns is elapsed time until the next runtime trace event."}
    if not rows:
        out.update({"window_ns": 0, "events": [], "groups": [], "hotspots": []})
        return out
    window = rows[-1]["timestamp_ns"] - rows[0]["timestamp_ns"]
    window = window if window >= 0 else 0
    out["window_ns"] = window
    out["events"] = [_timeline_event(r) for r in
                     _sorted_stable(rows, lambda r: r[event_sort_by], lambda r: r["index"], event_descending)]
    groups = {}
    for r in rows:
        key = _timeline_group_key(r, group_by)
        g = groups.get(key)
        if g is None:
            g = groups[key] = {"key": key, "count": 0, "total_delta_next_ns": 0, "max_delta_next_ns": 0,
                               "total_size_bytes": 0, "first_timestamp_ns": r["timestamp_ns"],
                               "last_timestamp_ns": r["timestamp_ns"]}
        g["last_timestamp_ns"] = r["timestamp_ns"]
        g["count"] += 1
        g["total_delta_next_ns"] += r["delta_next_ns"]
        g["max_delta_next_ns"] = max(g["max_delta_next_ns"], r["delta_next_ns"])
        g["total_size_bytes"] += r["size_bytes"]

    def gvalue(g):
        if group_sort_by == "avg_delta_next_ns":
            return g["total_delta_next_ns"] // g["count"] if g["count"] else 0
        return g[group_sort_by]

    glist = list(groups.values())
    if group_sort_by == "key":
        glist = sorted(glist, key=lambda g: g["key"], reverse=group_descending)
    else:
        glist = _sorted_stable(glist, gvalue, lambda g: g["key"], group_descending)
    for g in glist:
        g["avg_delta_next_ns"] = g["total_delta_next_ns"] / g["count"] if g["count"] else 0.0
        g["window_share_pct"] = 100.0 * g["total_delta_next_ns"] / window if window else 0.0
    out["groups"] = [{k: g[k] for k in ("key", "count", "total_delta_next_ns", "avg_delta_next_ns",
                                        "max_delta_next_ns", "total_size_bytes", "first_timestamp_ns",
                                        "last_timestamp_ns", "window_share_pct")} for g in glist]
    hot = _sorted_stable(rows, lambda r: r["delta_next_ns"], lambda r: r["index"], True)
    limit = len(hot) if hotspot_top_k == 0 else min(int(hotspot_top_k), len(hot))
    out["hotspots"] = [_timeline_event(r) for r in hot[:limit]]
    return out


def _timeline_event(r) -> dict:
    """bind_runtime.cpp:166-178 (toTimelineEventDict)."""
    return {k: r[k] for k in ("index", "type", "status", "op", "requested_device", "selected_device", "fallback",
                              "timestamp_ns", "offset_ns", "delta_prev_ns", "delta_next_ns", "size_bytes",
                              "detail0", "detail1")}


def tune_cache_save(path: str):
    """Writes the gfx950 matmul tune cache (#lc_tune_cache,matmul,2)."""
    _check(_lib().lcHipTuneCacheSave(path.encode()))


def tune_cache_load(path: str):
    """Reads a matmul tune cache (versions 1-2) and makes it the cache file."""
    _check(_lib().lcHipTuneCacheLoad(path.encode()))


def tune_cache_size() -> int:
    return int(_lib().lcHipTuneCacheSize())


def attention_tune_cache_save(path: str):
    """Writes the attention tune cache (#lc_tune_cache,attention,2)."""
    _check(_lib().lcHipAttentionTuneCacheSave(path.encode()))


def attention_tune_cache_load(path: str):
    _check(_lib().lcHipAttentionTuneCacheLoad(path.encode()))


def attention_reset_tuning():
    _check(_lib().lcHipAttentionResetTuning())


def attention_tune_cache_size() -> int:
    return int(_lib().lcHipAttentionTuneCacheSize())


def preload_runtime_profile_env():
    """runtime::preloadRuntimeProfileEnv (src/runtime.cpp:101-168, :421-423)."""
    _lib().lcPreloadRuntimeProfileEnv()


class HipTimer:
    """hipEvents recorded on the backend stream (the stream all kernels use)."""

    def __init__(self):
        h = ctypes.c_void_p()
        _check(_lib().lcHipTimerCreate(ctypes.byref(h)))
        self._h = h

    def start(self):
        _check(_lib().lcHipTimerStart(self._h))

    def stop(self) -> float:
        ms = ctypes.c_float()
        _check(_lib().lcHipTimerStop(self._h, ctypes.byref(ms)))
        return float(ms.value)

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            _lib().lcHipTimerDestroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
