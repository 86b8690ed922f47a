"""ctypes binding of the text front end (include/julia1_text.h): request rows,
pyjson, the Encoder (marker serialization with LRU caches), the legacy predict
API, named typed questions and the Router, over the HIP engine or over a
Python scorer.

The tokenizer is the `tokenizers` library on the checkpoint's tokenizer.json,
the same library the reference's `Encoder` uses (src/encode.rs:10,66-68); it
is handed to the C++ encoder as a callback.

    te = TextEngine.load("/path/to/ckpt", "hip:0")      # ckpt/tokenizer/{tokenizer,tokenizer_config}.json
    te.predict_typed("context", {"team": {"type": "choice", "instructions": "route",
                                          "criteria": {"billing": "Payments", "access": "Login"}}})
"""
from __future__ import annotations

import ctypes as C
import itertools
import json
import os
import threading

import numpy as np

from . import engine as _engine
from . import hip

ENCODE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(C.c_uint32), C.c_size_t,
                        C.POINTER(C.c_size_t))
TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_char_p, C.POINTER(C.c_uint32))
BATCH_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t),
                       C.POINTER(C.c_size_t), C.POINTER(C.POINTER(C.c_uint32)))
LOGITS_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p)


class JtTokenizer(C.Structure):
    _fields_ = [("ctx", C.c_void_p), ("encode", ENCODE_FN), ("token_to_id", TOKEN_FN), ("encode_batch", BATCH_FN)]


class JtEncoderOptions(C.Structure):
    _fields_ = [("max_length", C.c_uint32), ("head_length", C.c_uint32), ("strict", C.c_int32),
                ("token_cache", C.c_uint32), ("encoding_cache", C.c_uint32)]


EXPORTS = ("jt_free", "jt_pyjson_dumps", "jt_float_repr", "jt_default_encoder_options", "jt_encoder_create",
           "jt_encoder_destroy", "jt_encoder_clear_cache", "jt_encoder_special_ids", "jt_encode", "jt_encoding_info",
           "jt_rows_push", "jt_scorer_callback", "jt_scorer_engine", "jt_scorer_destroy", "jt_logits", "jt_predict",
           "jt_predict_typed", "jt_router_create", "jt_router_route_many", "jt_router_clear_cache",
           "jt_router_destroy", "jt_display_probabilities", "jt_confident_winner")


def _lib():
    L = hip.lib()
    if not getattr(L, "_jt_ready", False):
        vp, sz, u32 = C.c_void_p, C.c_size_t, C.c_uint32
        out = C.POINTER(C.c_void_p)
        L.jt_free.argtypes = [vp]
        L.jt_free.restype = None
        L.jt_pyjson_dumps.argtypes = [C.c_char_p, sz, out]
        L.jt_float_repr.argtypes = [C.c_double, out]
        L.jt_default_encoder_options.argtypes = [vp]
        L.jt_default_encoder_options.restype = None
        L.jt_encoder_create.argtypes = [vp, C.c_char_p, sz, vp, out]
        L.jt_encoder_destroy.argtypes = [vp]
        L.jt_encoder_destroy.restype = None
        L.jt_encoder_clear_cache.argtypes = [vp]
        L.jt_encoder_clear_cache.restype = None
        L.jt_encoder_special_ids.argtypes = [vp, C.POINTER(u32)]
        L.jt_encode.argtypes = [vp, C.c_char_p, sz, sz, out]
        L.jt_encoding_info.argtypes = [vp, C.c_char_p, sz, out]
        L.jt_rows_push.argtypes = [vp, vp, sz]
        L.jt_scorer_callback.argtypes = [LOGITS_FN, vp, out]
        L.jt_scorer_engine.argtypes = [vp, vp, out]
        L.jt_scorer_destroy.argtypes = [vp]
        L.jt_scorer_destroy.restype = None
        L.jt_logits.argtypes = [vp, C.c_char_p, sz, out]
        L.jt_predict.argtypes = [vp, C.c_char_p, sz, C.c_int, out]
        L.jt_predict_typed.argtypes = [vp, C.c_char_p, sz, C.c_char_p, sz, out]
        L.jt_router_create.argtypes = [vp, u32, u32, u32, u32, u32, out]
        L.jt_router_route_many.argtypes = [vp, C.c_char_p, sz, out]
        L.jt_router_clear_cache.argtypes = [vp]
        L.jt_router_clear_cache.restype = None
        L.jt_router_destroy.argtypes = [vp]
        L.jt_router_destroy.restype = None
        L.jt_display_probabilities.argtypes = [vp, sz, vp]
        L.jt_confident_winner.argtypes = [vp, sz, sz, C.POINTER(C.c_int)]
        L._jt_ready = True
    return L


def _call_text(fn, *args) -> str:
    """Calls a jt_* function whose last argument receives a library-allocated string."""
    p = C.c_void_p()
    hip.check(fn(*args, C.byref(p)))
    try:
        return C.string_at(p.value).decode("utf-8")
    finally:
        _lib().jt_free(p)


def _b(s: str) -> bytes:
    return s.encode("utf-8")


def jsonl(rows) -> bytes:
    return _b("\n".join(json.dumps(r, ensure_ascii=False) for r in rows))


def pyjson_dumps(text: str) -> str:
    """pyjson::dumps of a JSON document given as text."""
    b = _b(text)
    return _call_text(_lib().jt_pyjson_dumps, b, len(b))


def float_repr(v: float) -> str:
    return _call_text(_lib().jt_float_repr, float(v))


def display_probabilities(values) -> list:
    v = np.ascontiguousarray(values, dtype=np.float64)
    out = np.zeros_like(v)
    hip.check(_lib().jt_display_probabilities(v.ctypes.data if v.size else None, v.size,
                                              out.ctypes.data if v.size else None))
    return out.tolist()


def confident_winner(scores, best: int) -> bool:
    s = np.ascontiguousarray(scores, dtype=np.float32)
    o = C.c_int()
    hip.check(_lib().jt_confident_winner(s.ctypes.data, s.size, best, C.byref(o)))
    return bool(o.value)


class Tokenizer:
    """A `tokenizers.Tokenizer` (tokenizer.json) behind the jt_tokenizer callbacks, with truncation and
    padding off (src/encode.rs:67-68)."""

    def __init__(self, tok, batch: bool = True):
        tok.no_truncation()
        tok.no_padding()
        self.tok = tok
        self._encode = ENCODE_FN(self._encode_cb)
        self._token = TOKEN_FN(self._token_cb)
        # Batch tokenization (the library's parallel encode_batch_fast: ids without offsets, as the
        # reference's encode_fast); the ids handed back stay alive per thread until its next call.
        self._fast = getattr(tok, "encode_batch_fast", None) or tok.encode_batch
        self._kept = threading.local()
        self._batch = BATCH_FN(self._batch_cb) if batch else BATCH_FN()
        self.struct = JtTokenizer(None, self._encode, self._token, self._batch)

    @staticmethod
    def from_file(path: str) -> "Tokenizer":
        from tokenizers import Tokenizer as HfTokenizer
        return Tokenizer(HfTokenizer.from_file(path))

    def _encode_cb(self, ctx, text, n, ids, capacity, count):
        try:
            out = self.tok.encode(C.string_at(text, n).decode("utf-8"), add_special_tokens=False).ids
            count[0] = len(out)
            k = min(len(out), capacity)
            if k:
                a = np.asarray(out[:k], dtype=np.uint32)
                C.memmove(ids, a.ctypes.data, 4 * k)
            return 0
        except Exception:
            return 1

    def _batch_cb(self, ctx, n, texts, lens, counts, ids_out):
        try:
            encs = self._fast([C.string_at(texts[i], lens[i]).decode("utf-8") for i in range(n)],
                              add_special_tokens=False)
            for i, e in enumerate(encs):
                counts[i] = len(e.ids)
            flat = np.fromiter(itertools.chain.from_iterable(e.ids for e in encs), dtype=np.uint32)
            self._kept.ids = flat
            ids_out[0] = flat.ctypes.data_as(C.POINTER(C.c_uint32))
            return 0
        except Exception:
            return 1

    def _token_cb(self, ctx, name, out):
        try:
            i = self.tok.token_to_id(name.decode("utf-8"))
            if i is None:
                return 1
            out[0] = i
            return 0
        except Exception:
            return 1


class Encoder:
    """`Encoder` (src/encode.rs): Encoder(tokenizer, tokenizer_config_text, max_length, ...)."""

    def __init__(self, tokenizer: Tokenizer, tokenizer_config: str, max_length: int, head_length: int = 256,
                 strict: bool = False, token_cache: int = 8192, encoding_cache: int = 2048):
        self.tokenizer = tokenizer
        o = JtEncoderOptions()
        _lib().jt_default_encoder_options(C.byref(o))
        o.max_length, o.head_length, o.strict = max_length, head_length, 1 if strict else 0
        o.token_cache, o.encoding_cache = token_cache, encoding_cache
        cfg = _b(tokenizer_config)
        h = C.c_void_p()
        hip.check(_lib().jt_encoder_create(C.byref(tokenizer.struct), cfg, len(cfg), C.byref(o), C.byref(h)))
        self.h = h

    @staticmethod
    def load(tokenizer_dir: str, max_length: int, **kw) -> "Encoder":
        """`Encoder::load` (src/encode.rs:44-56): tokenizer.json + tokenizer_config.json."""
        tok = Tokenizer.from_file(os.path.join(tokenizer_dir, "tokenizer.json"))
        with open(os.path.join(tokenizer_dir, "tokenizer_config.json"), encoding="utf-8") as f:
            cfg = f.read()
        return Encoder(tok, cfg, max_length, **kw)

    @property
    def special_ids(self) -> dict:
        a = (C.c_uint32 * 4)()
        hip.check(_lib().jt_encoder_special_ids(self.h, a))
        return dict(mask=a[0], cls=a[1], sep=a[2], pad=a[3])

    def encode(self, row: dict, line: int = 1) -> dict:
        b = _b(json.dumps(row, ensure_ascii=False))
        return json.loads(_call_text(_lib().jt_encode, self.h, b, len(b), line))

    def encoding_info(self, rows) -> list:
        b = jsonl(rows)
        return json.loads(_call_text(_lib().jt_encoding_info, self.h, b, len(b)))

    def clear_cache(self):
        _lib().jt_encoder_clear_cache(self.h)

    def close(self):
        if getattr(self, "h", None):
            _lib().jt_encoder_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Scorer:
    """A `Logits` source: the engine (`EngineScorer`) or a Python function (`CallbackScorer`)."""

    h = None

    def logits(self, rows) -> list:
        b = jsonl(rows)
        return [np.asarray(z, dtype=np.float32) for z in json.loads(_call_text(_lib().jt_logits, self.h, b, len(b)))]

    def predict(self, rows, probabilities: bool = False) -> list:
        b = jsonl(rows)
        return json.loads(_call_text(_lib().jt_predict, self.h, b, len(b), 1 if probabilities else 0))

    def predict_typed(self, state, questions: dict) -> dict:
        s, q = _b(json.dumps(state, ensure_ascii=False)), _b(json.dumps(questions, ensure_ascii=False))
        return json.loads(_call_text(_lib().jt_predict_typed, self.h, s, len(s), q, len(q)))

    def close(self):
        if getattr(self, "h", None):
            _lib().jt_scorer_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class CallbackScorer(Scorer):
    """fn(rows: list[dict]) -> list of per-row logits; the reference's test doubles (tests/api.rs)."""

    def __init__(self, fn):
        self.fn = fn
        self._cb = LOGITS_FN(self._call)
        h = C.c_void_p()
        hip.check(_lib().jt_scorer_callback(self._cb, None, C.byref(h)))
        self.h = h

    def _call(self, ctx, text, n, out):
        try:
            for z in self.fn(json.loads(C.string_at(text, n).decode("utf-8"))):
                a = np.ascontiguousarray(z, dtype=np.float32)
                if _lib().jt_rows_push(out, a.ctypes.data if a.size else None, a.size) != 0:
                    return 1
            return 0
        except Exception:
            return 1


class EngineScorer(Scorer):
    """`Engine::logits`: validate, encode with `encoder`, then the HIP engine's micro-batched forward."""

    def __init__(self, engine: _engine.Engine, encoder: Encoder):
        self.engine, self.encoder = engine, encoder
        h = C.c_void_p()
        hip.check(_lib().jt_scorer_engine(engine.h, encoder.h, C.byref(h)))
        self.h = h


class Router:
    """`Router` (src/router.rs) over any scorer; defaults are the Python Router's."""

    def __init__(self, scorer: Scorer, width: int = 20, survivors: int = 2, batch_size: int = 16,
                 cache_size: int = 0, max_options: int = 4096):
        self.scorer = scorer
        h = C.c_void_p()
        hip.check(_lib().jt_router_create(scorer.h, width, survivors, batch_size, cache_size, max_options,
                                          C.byref(h)))
        self.h = h

    def route_many(self, rows) -> list:
        b = jsonl(rows)
        return json.loads(_call_text(_lib().jt_router_route_many, self.h, b, len(b)))

    def route(self, row: dict) -> dict:
        return self.route_many([row])[0]

    def clear_cache(self):
        _lib().jt_router_clear_cache(self.h)

    def close(self):
        if getattr(self, "h", None):
            _lib().jt_router_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class TextEngine(EngineScorer):
    """`Engine::load` with its encoder (src/engine.rs:89-110): the HIP engine plus the text front end read
    from <checkpoint>/tokenizer."""

    @staticmethod
    def load(checkpoint_dir: str, device: str = "hip:0", max_length: int = 0, head_length: int = 256,
             batch_size: int = 16, max_batch_tokens: int = 65536, strict_encoding: bool = False,
             encoding_cache: int = 2048, token_cache: int = 8192) -> "TextEngine":
        e = _engine.Engine.load(checkpoint_dir, device, max_length=max_length, batch_size=batch_size,
                                max_batch_tokens=max_batch_tokens)
        o = _engine.JeOptions()
        hip.check(_engine._lib().je_get_options(e.h, C.byref(o)))
        enc = Encoder.load(os.path.join(checkpoint_dir, "tokenizer"), o.max_length, head_length=head_length,
                           strict=strict_encoding, token_cache=token_cache, encoding_cache=encoding_cache)
        return TextEngine(e, enc)

    def encoding_info(self, rows) -> list:
        return self.encoder.encoding_info(rows)

    def router(self, **kw) -> Router:
        return Router(self, **kw)
