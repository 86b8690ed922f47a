"""ctypes binding of the FP32 CPU oracle (oracle/julia1_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product path never imports
this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libjulia1_oracle.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, sz = C.c_void_p, C.c_size_t
        L.jo_create.argtypes = [vp, vp, C.c_int, C.POINTER(vp)]
        L.jo_destroy.argtypes = [vp]
        L.jo_set_threads.argtypes = [vp, C.c_int]
        L.jo_set_fault.argtypes = [C.c_int]
        L.jo_omp_threads.argtypes = [C.c_int]
        L.jo_forward.argtypes = [vp, vp, sz, vp, vp, vp, sz, vp, sz, vp]
        L.jo_encode.argtypes = [vp, vp, sz, vp, vp, sz, C.c_uint32, vp]
        for n in ("jo_exp", "jo_erf", "jo_gelu"):
            getattr(L, n).argtypes = [vp, sz, vp]
        L.jo_layer_norm.argtypes = [vp, sz, sz, vp, vp, C.c_float, vp]
        L.jo_linear.argtypes = [vp, sz, sz, vp, sz, vp, sz, sz, C.c_int, vp]
        L.jo_linear_geglu.argtypes = [vp, sz, sz, vp, sz, vp]
        L.jo_attention.argtypes = [vp, sz, sz, vp, sz, sz, sz, vp, sz, vp, sz, sz, C.c_long, C.c_float]
        L.jo_rope_table.argtypes = [C.c_float, C.c_uint32, C.c_uint32, vp, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


EPI_STORE, EPI_ADD, EPI_BIAS, EPI_BIAS_RELU, EPI_ADD_BIAS = range(5)


class OracleModel:
    """`CpuModel` restated: FP32 forward over packed batches."""

    def __init__(self, weight_set, threads: int | None = None):
        self._ws = weight_set
        threads = threads or int(os.environ.get("JULIA_CPU_THREADS", os.cpu_count() or 4))
        h = C.c_void_p()
        rc = lib().jo_create(C.addressof(weight_set.config), C.addressof(weight_set.weights), threads, C.byref(h))
        if rc != 0:
            raise ValueError(f"jo_create failed ({rc})")
        self.h = h
        self.cfg = weight_set.cfg
        self.threads = threads

    def set_threads(self, n: int):
        lib().jo_set_threads(self.h, n)
        self.threads = n

    def forward(self, b) -> np.ndarray:
        scores = np.zeros(b.marker_rows.size, dtype=np.float32)
        rc = lib().jo_forward(self.h, _p(b.ids), b.tokens, _p(b.starts), _p(b.lens), _p(b.qtypes),
                              b.lens.size, _p(b.marker_rows), b.marker_rows.size, _p(scores))
        if rc != 0:
            raise ValueError(f"jo_forward failed ({rc})")
        return scores

    def encode(self, b, layers: int) -> np.ndarray:
        x = np.zeros((b.tokens, self.cfg.hidden), dtype=np.float32)
        rc = lib().jo_encode(self.h, _p(b.ids), b.tokens, _p(b.starts), _p(b.lens), b.lens.size, layers, _p(x))
        if rc != 0:
            raise ValueError(f"jo_encode failed ({rc})")
        return x

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.jo_destroy(self.h)
            self.h = None


def omp_threads(n: int):
    """Thread count of the op-level functions below."""
    lib().jo_omp_threads(n)


def set_fault(code: int):
    """Planted mistakes for mutation tests of the oracle's checks (0 = none)."""
    lib().jo_set_fault(code)


def _unary(name, x):
    x = _f32(x)
    out = np.empty_like(x)
    getattr(lib(), name)(_p(x), x.size, _p(out))
    return out


def exp(x):
    return _unary("jo_exp", x)


def erf(x):
    return _unary("jo_erf", x)


def gelu(x):
    return _unary("jo_gelu", x)


def layer_norm(x, w, b=None, eps=1e-5):
    x = _f32(x)
    rows, width = x.shape
    out = np.empty_like(x)
    lib().jo_layer_norm(_p(x), rows, width, _p(_f32(w)), None if b is None else _p(_f32(b)), eps, _p(out))
    return out


def linear(x, w, out=None, col=0, epi=EPI_STORE, bias=None):
    """out[:, col:col+n] = epi(x · wᵀ); returns out (allocated [rows, n] if None)."""
    x, w = _f32(x), _f32(w)
    rows, k = x.shape
    n = w.shape[0]
    if out is None:
        out = np.zeros((rows, n), dtype=np.float32)
    bias = None if bias is None else _f32(bias)
    lib().jo_linear(_p(x), rows, k, _p(w), n, _p(out), out.shape[1], col, epi, _p(bias))
    return out


def linear_geglu(x, w):
    x, w = _f32(x), _f32(w)
    rows, k = x.shape
    n = w.shape[0]
    g = np.zeros((rows, n // 2), dtype=np.float32)
    lib().jo_linear_geglu(_p(x), rows, k, _p(w), n, _p(g))
    return g


def attention(q, kv, seqs, heads, window=-1, scale=0.125, ldq=None, q_off=0, k_off=None, v_off=None, ldo=None):
    """Packed attention; q [*, ldq], kv [*, ldkv]; seqs = [(q_row, nq, kv_row, len)]."""
    q, kv = _f32(q), _f32(kv)
    ldq = ldq or q.shape[1]
    ldkv = kv.shape[1]
    h = heads * 64
    k_off = h if k_off is None else k_off
    v_off = 2 * h if v_off is None else v_off
    ldo = ldo or h
    rows = max(s[0] + s[1] for s in seqs) if seqs else 0
    out = np.zeros((max(rows, q.shape[0]), ldo), dtype=np.float32)
    sq = np.ascontiguousarray(np.array(seqs, dtype=np.uint32).reshape(-1, 4))
    lib().jo_attention(_p(q), ldq, q_off, _p(kv), ldkv, k_off, v_off, _p(out), ldo, _p(sq), len(seqs), heads,
                       window, scale)
    return out


def rope_table(theta, positions, head_dim=64):
    half = head_dim // 2
    c = np.zeros((positions, half), dtype=np.float32)
    s = np.zeros((positions, half), dtype=np.float32)
    lib().jo_rope_table(theta, head_dim, positions, _p(c), _p(s))
    return c, s
