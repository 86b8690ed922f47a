"""ctypes binding of the C++ host engine (include/julia1_engine.h): the
`Engine` of the reference runtime below its text front end, on the HIP
backend.  `Engine.load(checkpoint_dir, device="hip:0")` then
`logits_encoded(items)` with items (ids, marker positions, qtype)."""
from __future__ import annotations

import ctypes as C
import json

import numpy as np

from . import hip
from .abi import JhConfig


class JeOptions(C.Structure):
    _fields_ = [("device_ordinal", C.c_int), ("max_length", C.c_uint32), ("batch_size", C.c_uint32),
                ("max_batch_tokens", C.c_uint32)]


def _lib():
    L = hip.lib()
    if not getattr(L, "_je_ready", False):
        vp, sz = C.c_void_p, C.c_size_t
        L.je_default_options.argtypes = [vp]
        L.je_default_options.restype = None
        L.je_parse_device.argtypes = [C.c_char_p, C.POINTER(C.c_int)]
        L.je_load.argtypes = [C.c_char_p, vp, C.POINTER(vp)]
        L.je_logits_encoded.argtypes = [vp, sz, vp, vp, vp, vp, vp, vp]
        L.je_config.argtypes = [vp, vp]
        L.je_get_options.argtypes = [vp, vp]
        L.je_device_name.argtypes = [vp]
        L.je_device_name.restype = C.c_char_p
        L.je_forward_count.argtypes = [vp]
        L.je_forward_count.restype = C.c_uint64
        L.je_destroy.argtypes = [vp]
        L.je_destroy.restype = None
        L.je_inspect.argtypes = [C.c_char_p, C.c_char_p, sz]
        L._je_ready = True
    return L


def parse_device(s: str) -> int:
    o = C.c_int()
    hip.check(_lib().je_parse_device(s.encode(), C.byref(o)))
    return o.value


def inspect(checkpoint_dir: str) -> dict:
    buf = C.create_string_buffer(512)
    hip.check(_lib().je_inspect(checkpoint_dir.encode(), buf, 512))
    return json.loads(buf.value.decode())


class Engine:
    def __init__(self, handle):
        self.h = handle

    @staticmethod
    def load(checkpoint_dir: str, device: str = "hip:0", max_length: int = 0, batch_size: int = 16,
             max_batch_tokens: int = 65536) -> "Engine":
        o = JeOptions()
        _lib().je_default_options(C.byref(o))
        o.device_ordinal = parse_device(device)
        o.max_length, o.batch_size, o.max_batch_tokens = max_length, batch_size, max_batch_tokens
        h = C.c_void_p()
        hip.check(_lib().je_load(checkpoint_dir.encode(), C.byref(o), C.byref(h)))
        return Engine(h)

    @property
    def device_name(self) -> str:
        return _lib().je_device_name(self.h).decode()

    @property
    def forward_count(self) -> int:
        return int(_lib().je_forward_count(self.h))

    def config(self) -> JhConfig:
        c = JhConfig()
        hip.check(_lib().je_config(self.h, C.byref(c)))
        return c

    def logits_encoded(self, items) -> list:
        """items: [(ids, markers, qtype)] -> per-item float32 logits (src/engine.rs:225-235)."""
        items = list(items)
        ids = np.ascontiguousarray(np.concatenate([np.asarray(i[0], dtype=np.uint32) for i in items])
                                   if items else np.zeros(0, np.uint32), dtype=np.uint32)
        mk = np.ascontiguousarray(np.concatenate([np.asarray(i[1], dtype=np.uint32) for i in items])
                                  if items else np.zeros(0, np.uint32), dtype=np.uint32)
        id_off = np.zeros(len(items) + 1, dtype=np.uintp)
        mk_off = np.zeros(len(items) + 1, dtype=np.uintp)
        id_off[1:] = np.cumsum([len(i[0]) for i in items])
        mk_off[1:] = np.cumsum([len(i[1]) for i in items])
        qt = np.array([int(i[2]) for i in items], dtype=np.uint8)
        out = np.zeros(int(mk_off[-1]), dtype=np.float32)
        p = lambda a: a.ctypes.data if a.size else None  # noqa: E731
        hip.check(_lib().je_logits_encoded(self.h, len(items), p(ids), id_off.ctypes.data, p(mk), mk_off.ctypes.data,
                                           p(qt) if qt.size else None, p(out)))
        return [out[int(a):int(b)] for a, b in zip(mk_off[:-1], mk_off[1:])]

    def close(self):
        if getattr(self, "h", None):
            _lib().je_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()
