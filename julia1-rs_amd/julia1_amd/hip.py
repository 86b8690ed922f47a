"""ctypes binding of libjulia1_hip.so (include/julia1_hip.h, include/julia1_hip_ops.h).

The library must have been built (julia1-rs_amd/build.py or
__graft_entry__.build()); loading fails loudly otherwise — there is no
fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import abi

_lib = None

EXPORTS = (
    "jh_create", "jh_forward", "jh_forward_padded", "jh_stage", "jh_execute", "jh_scores", "jh_stream", "jh_submit",
    "jh_collect",
    "jh_set_graph", "jh_set_splitk", "jh_name", "jh_destroy", "jh_last_error", "jh_rope_table", "jh_debug_tokens",
    "jh_debug_encode", "jh_debug_workspace_limit", "jh_profile", "jh_profile_read", "jh_profile_replay",
    "jh_op_gemm", "jh_op_gemm_splitk", "jh_op_gemm_splitk_noalloc", "jh_op_gemm_ln", "jh_op_gemm_ws", "jh_op_pack_ws",
    "jh_op_interleave_geglu",
    "jh_op_embed_ln", "jh_op_layer_norm", "jh_op_final_norm",
    "jh_op_gather_f32", "jh_op_scorer", "jh_op_attention", "jh_op_attention_wide",
)


class KernelStat(C.Structure):
    _fields_ = [("name", C.c_char_p), ("launches", C.c_uint32), ("ms", C.c_double), ("flops", C.c_double),
                ("bytes", C.c_double)]


class HipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(abi.LIB_PATH):
            raise RuntimeError(f"{abi.LIB_PATH} is not built; run julia1-rs_amd/build.py")
        L = C.CDLL(abi.LIB_PATH)
        vp, sz, u32 = C.c_void_p, C.c_size_t, C.c_uint32
        L.jh_create.argtypes = [vp, vp, C.c_int, C.POINTER(vp)]
        L.jh_forward.argtypes = [vp, vp, sz, vp, vp, vp, sz, vp, sz, vp]
        L.jh_forward_padded.argtypes = [vp, vp, sz, sz, vp, vp, vp, vp, vp]
        L.jh_stage.argtypes = [vp, vp, sz, vp, vp, vp, sz, vp, sz]
        L.jh_execute.argtypes = [vp]
        L.jh_scores.argtypes = [vp, vp, sz]
        L.jh_submit.argtypes = [vp, vp, sz, vp, vp, vp, sz, vp, sz, C.POINTER(C.c_uint64)]
        L.jh_collect.argtypes = [vp, C.c_uint64, vp, sz]
        L.jh_stream.argtypes = [vp]
        L.jh_stream.restype = vp
        L.jh_set_graph.argtypes = [vp, C.c_int]
        L.jh_set_splitk.argtypes = [vp, C.c_int]
        L.jh_name.argtypes = [vp]
        L.jh_name.restype = C.c_char_p
        L.jh_destroy.argtypes = [vp]
        L.jh_destroy.restype = None
        L.jh_last_error.argtypes = []
        L.jh_last_error.restype = C.c_char_p
        L.jh_rope_table.argtypes = [C.c_float, u32, u32, vp, vp]
        L.jh_rope_table.restype = None
        L.jh_debug_tokens.argtypes = [vp, vp, vp, sz]
        L.jh_debug_encode.argtypes = [vp, u32, vp, sz]
        L.jh_debug_workspace_limit.argtypes = [vp, sz]
        L.jh_profile.argtypes = [vp, C.c_int]
        L.jh_profile_read.argtypes = [vp, vp, sz, C.POINTER(sz)]
        L.jh_profile_replay.argtypes = [vp, C.c_char_p, sz, C.POINTER(C.c_double)]
        L.jh_op_gemm.argtypes = [C.c_int, vp, sz, vp, sz, vp, sz, sz, vp, sz, sz, vp, vp, vp, vp, sz, vp]
        L.jh_op_gemm_splitk.argtypes = [C.c_int, vp, sz, vp, sz, vp, sz, sz, vp, sz, sz, vp, vp, vp, vp, sz, vp, sz,
                                        C.c_int, vp]
        L.jh_op_gemm_splitk_noalloc.argtypes = [C.c_int, vp, sz, vp, sz, vp, sz, sz, vp, sz, sz, vp, vp, vp, vp,
                                                sz, C.c_int, vp]
        L.jh_op_gemm_ln.argtypes = [C.c_int, vp, sz, sz, vp, sz, sz, vp, sz, sz, vp, vp, vp, sz, vp, vp, C.c_float,
                                    vp]
        L.jh_op_gemm_ws.argtypes = [C.c_int, vp, sz, sz, vp, sz, sz, vp, sz, sz, vp, vp, vp, vp, sz, vp]
        L.jh_op_pack_ws.argtypes = [vp, sz, sz, vp]
        L.jh_op_interleave_geglu.argtypes = [vp, sz, sz, vp]
        L.jh_op_interleave_geglu.restype = None
        L.jh_op_embed_ln.argtypes = [vp, sz, vp, vp, C.c_float, sz, vp, vp, vp]
        L.jh_op_layer_norm.argtypes = [vp, sz, vp, vp, C.c_float, sz, vp, vp]
        L.jh_op_final_norm.argtypes = [vp, sz, vp, vp, vp, vp, vp, C.c_float, sz, vp, vp]
        L.jh_op_gather_f32.argtypes = [vp, vp, sz, sz, vp, vp]
        L.jh_op_scorer.argtypes = [vp, sz, sz, vp, C.c_float, vp, vp]
        L.jh_op_attention.argtypes = [vp, sz, vp, vp, sz, vp, sz, vp, sz, sz, C.c_int, C.c_float, vp]
        L.jh_op_attention_wide.argtypes = L.jh_op_attention.argtypes
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise HipError(rc, lib().jh_last_error().decode())


def _p(a):
    return None if a is None else a.ctypes.data


def rope_table(theta: float, positions: int, head_dim: int = 64):
    half = head_dim // 2
    c = np.zeros((positions, half), dtype=np.float32)
    s = np.zeros((positions, half), dtype=np.float32)
    lib().jh_rope_table(theta, head_dim, positions, _p(c), _p(s))
    return c, s


class HipModel:
    """The `Backend::Hip` model: jh_create / jh_forward / jh_name / jh_destroy."""

    def __init__(self, weight_set, ordinal: int = 0):
        self._ws = weight_set
        h = C.c_void_p()
        check(lib().jh_create(C.addressof(weight_set.config), C.addressof(weight_set.weights), ordinal, C.byref(h)))
        self.h = h
        self.cfg = weight_set.cfg

    @property
    def name(self) -> str:
        return lib().jh_name(self.h).decode()

    def forward(self, b) -> np.ndarray:
        scores = np.zeros(b.marker_rows.size, dtype=np.float32)
        check(lib().jh_forward(self.h, _p(b.ids), b.tokens, _p(b.starts), _p(b.lens), _p(b.qtypes), b.lens.size,
                               _p(b.marker_rows), b.marker_rows.size, _p(scores)))
        return scores

    def forward_padded(self, ids, lens, qtypes, markers, marker_starts) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        B, L = ids.shape
        lens = np.ascontiguousarray(lens, dtype=np.uint32)
        qtypes = np.ascontiguousarray(qtypes, dtype=np.uint8)
        markers = np.ascontiguousarray(markers, dtype=np.uint32)
        marker_starts = np.ascontiguousarray(marker_starts, dtype=np.uint32)
        scores = np.zeros(int(marker_starts[-1]) if B else 0, dtype=np.float32)
        check(lib().jh_forward_padded(self.h, _p(ids), B, L, _p(lens), _p(qtypes), _p(markers), _p(marker_starts),
                                      _p(scores)))
        return scores

    def submit(self, b) -> int:
        """jh_submit: enqueue a forward without waiting; returns its ticket."""
        t = C.c_uint64(0)
        check(lib().jh_submit(self.h, _p(b.ids), b.tokens, _p(b.starts), _p(b.lens), _p(b.qtypes), b.lens.size,
                              _p(b.marker_rows), b.marker_rows.size, C.byref(t)))
        return t.value

    def collect(self, ticket: int, m: int) -> np.ndarray:
        """jh_collect: wait for a submitted forward and return its m scores."""
        out = np.zeros(m, dtype=np.float32)
        check(lib().jh_collect(self.h, ticket, _p(out), m))
        return out

    def stage(self, b):
        self._staged = b
        check(lib().jh_stage(self.h, _p(b.ids), b.tokens, _p(b.starts), _p(b.lens), _p(b.qtypes), b.lens.size,
                             _p(b.marker_rows), b.marker_rows.size))

    def execute(self):
        check(lib().jh_execute(self.h))

    def scores(self, m: int) -> np.ndarray:
        out = np.zeros(m, dtype=np.float32)
        check(lib().jh_scores(self.h, _p(out), m))
        return out

    def set_graph(self, on: bool):
        check(lib().jh_set_graph(self.h, 1 if on else 0))

    def set_splitk(self, on: bool):
        check(lib().jh_set_splitk(self.h, 1 if on else 0))

    @property
    def stream(self) -> int:
        return lib().jh_stream(self.h) or 0

    def debug_tokens(self, t: int):
        ids = np.zeros(t, dtype=np.uint32)
        pos = np.zeros(t, dtype=np.uint32)
        check(lib().jh_debug_tokens(self.h, _p(ids), _p(pos), t))
        return ids, pos

    def debug_encode(self, t: int, layers: int) -> np.ndarray:
        x = np.zeros((t, self.cfg.hidden), dtype=np.float32)
        check(lib().jh_debug_encode(self.h, layers, _p(x), t))
        return x

    def debug_workspace_limit(self, nbytes: int):
        """jh_debug_workspace_limit: later workspace growths past `nbytes` fail with JH_ERR_ALLOC (0 = off)."""
        check(lib().jh_debug_workspace_limit(self.h, nbytes))

    def profile(self, on: bool):
        check(lib().jh_profile(self.h, 1 if on else 0))

    def profile_read(self) -> list:
        """[{name, launches, ms, flops, bytes}] summed since the last read (device time from HIP events)."""
        arr = (KernelStat * 32)()
        n = C.c_size_t()
        check(lib().jh_profile_read(self.h, arr, 32, C.byref(n)))
        return [dict(name=arr[i].name.decode(), launches=arr[i].launches, ms=arr[i].ms, flops=arr[i].flops,
                     bytes=arr[i].bytes) for i in range(n.value)]

    def profile_replay(self, kernel_class: str, reps: int = 50) -> float:
        """Mean device µs of one launch of a GEMM/attention class, replayed back to back
        (see jh_profile_replay); valid right after a profiled forward."""
        us = C.c_double()
        check(lib().jh_profile_replay(self.h, kernel_class.encode(), reps, C.byref(us)))
        return us.value

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.jh_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


# ---------------------------------------------------------------- op level (device tensors via torch)

def _dp(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def op_gemm(epi, x, w, out, rows=None, gather=None, col=0, bias=None, pos=None, cos=None, sin=None, rope_cols=0,
            stream=None):
    """x, w bf16 torch tensors (2-D), out torch tensor; see jh_op_gemm."""
    rows = x.shape[0] if rows is None else rows
    n, k = w.shape
    check(lib().jh_op_gemm(epi, _dp(x), x.stride(0), _dp(gather), rows, _dp(w), n, k, _dp(out), out.stride(0), col,
                           _dp(bias), _dp(pos), _dp(cos), _dp(sin), rope_cols, stream))


def op_gemm_splitk(epi, x, w, out, workspace, splits=0, rows=None, gather=None, col=0, bias=None, pos=None, cos=None,
                   sin=None, rope_cols=0, stream=None):
    """jh_op_gemm_splitk: like op_gemm with a torch workspace tensor for the FP32 partials."""
    rows = x.shape[0] if rows is None else rows
    n, k = w.shape
    check(lib().jh_op_gemm_splitk(epi, _dp(x), x.stride(0), _dp(gather), rows, _dp(w), n, k, _dp(out), out.stride(0),
                                  col, _dp(bias), _dp(pos), _dp(cos), _dp(sin), rope_cols, _dp(workspace),
                                  workspace.numel() * workspace.element_size(), splits, stream))


def op_gemm_ln(epi, xf, w, out, ln_w, ln_b=None, eps=1e-5, rows=None, col=0, pos=None, cos=None, sin=None,
               rope_cols=0, stream=None):
    """jh_op_gemm_ln: X = bf16(LayerNorm(xf)) computed inside the GEMM; xf an FP32 torch tensor (2-D)."""
    rows = xf.shape[0] if rows is None else rows
    n, k = w.shape
    check(lib().jh_op_gemm_ln(epi, _dp(xf), xf.stride(0), rows, _dp(w), n, k, _dp(out), out.stride(0), col,
                              _dp(pos), _dp(cos), _dp(sin), rope_cols, _dp(ln_w), _dp(ln_b), eps, stream))


def op_gemm_splitk_noalloc(epi, x, w, out, splits=0, rows=None, gather=None, col=0, bias=None, pos=None, cos=None,
                           sin=None, rope_cols=0, stream=None):
    """jh_op_gemm_splitk_noalloc: op_gemm_splitk with the library's fixed scratch instead of a workspace."""
    rows = x.shape[0] if rows is None else rows
    n, k = w.shape
    check(lib().jh_op_gemm_splitk_noalloc(epi, _dp(x), x.stride(0), _dp(gather), rows, _dp(w), n, k, _dp(out),
                                          out.stride(0), col, _dp(bias), _dp(pos), _dp(cos), _dp(sin), rope_cols,
                                          splits, stream))


def pack_ws(w):
    """bf16 torch tensor [n, k] (PyTorch Linear layout; the GEGLU interleave for Wi) -> the same values on the
    device in the weight-stationary kernel's fragment order (jh_op_pack_ws)."""
    import torch
    src = w.detach().to("cpu").contiguous().view(torch.int16).numpy()
    n, k = src.shape
    dst = np.empty_like(src)
    check(lib().jh_op_pack_ws(src.ctypes.data_as(C.c_void_p), n, k, dst.ctypes.data_as(C.c_void_p)))
    return torch.from_numpy(dst).view(torch.bfloat16).cuda()


def op_gemm_ws(epi, x, w_packed, n, k, out, rows=None, col=0, bias=None, pos=None, cos=None, sin=None, rope_cols=0,
               stream=None):
    """jh_op_gemm_ws: the weight-stationary GEMM on W packed by pack_ws (K = 768 with N % 256 == 0, or K = 1152
    with N % 128 == 0 and the residual epilogue)."""
    rows = x.shape[0] if rows is None else rows
    check(lib().jh_op_gemm_ws(epi, _dp(x), x.stride(0), rows, _dp(w_packed), n, k, _dp(out), out.stride(0), col,
                              _dp(bias), _dp(pos), _dp(cos), _dp(sin), rope_cols, stream))


def interleave_geglu(wi: np.ndarray) -> np.ndarray:
    wi = np.ascontiguousarray(wi, dtype=np.float32)
    out = np.empty_like(wi)
    lib().jh_op_interleave_geglu(_p(wi), wi.shape[0] // 2, wi.shape[1], _p(out))
    return out


def op_embed_ln(ids, table, w, eps, x, xn, stream=None):
    check(lib().jh_op_embed_ln(_dp(ids), ids.numel(), _dp(table), _dp(w), eps, table.shape[1], _dp(x), _dp(xn), stream))


def op_layer_norm(x, w, b, eps, out, stream=None):
    check(lib().jh_op_layer_norm(_dp(x), x.shape[0], _dp(w), _dp(b), eps, x.shape[1], _dp(out), stream))


def op_final_norm(x, fw, type_emb, tok_meta, hw, hb, eps, out, stream=None):
    check(lib().jh_op_final_norm(_dp(x), x.shape[0], _dp(fw), _dp(type_emb), _dp(tok_meta), _dp(hw), _dp(hb), eps,
                                 x.shape[1], _dp(out), stream))


def op_gather_f32(src, idx, dst, stream=None):
    check(lib().jh_op_gather_f32(_dp(src), _dp(idx), idx.numel(), src.shape[1], _dp(dst), stream))


def op_scorer(z, w2, b2, out, stream=None):
    check(lib().jh_op_scorer(_dp(z), z.shape[0], z.shape[1], _dp(w2), b2, _dp(out), stream))


def op_attention(q, ldq, k, v, ldkv, out, ldo, tiles, heads, window, scale=0.125, stream=None, wide=False):
    """q/k/v/out torch bf16 tensors (base pointers of the first row/col); tiles torch int32 [n, 5] of at most
    128 queries each, or 256 with wide=True (eight-wave work items, jh_op_attention_wide)."""
    fn = lib().jh_op_attention_wide if wide else lib().jh_op_attention
    check(fn(_dp(q), ldq, _dp(k), _dp(v), ldkv, _dp(out), ldo, _dp(tiles), tiles.shape[0], heads, window, scale,
             stream))
