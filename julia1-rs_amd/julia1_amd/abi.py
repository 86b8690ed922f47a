"""ctypes mirror of include/julia1_hip.h (jh_config / jh_weights and friends).

The structures are shared by the HIP backend library and by the CPU oracle,
which take the same borrowed FP32 host weights.  `WeightSet` keeps the numpy
arrays alive for as long as the ctypes structures that point into them.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

from . import build_paths

LIB_DIR = os.path.dirname(build_paths.SHARED)
LIB_PATH = build_paths.SHARED

JH_OK = 0
JH_ERR_INVALID = 1
JH_ERR_DEVICE = 2
JH_ERR_ALLOC = 3
JH_ERR_NONFINITE = 4
JH_ERR_INTERNAL = 5

EPI_STORE_BF16 = 0
EPI_ROPE_BF16 = 1
EPI_GEGLU_BF16 = 2
EPI_RESID_F32 = 3
EPI_BIAS_BF16 = 4
EPI_BIAS_RELU_BF16 = 5
EPI_BIAS_F32 = 6

_f32p = C.POINTER(C.c_float)


class JhConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("intermediate", C.c_uint32), ("layers", C.c_uint32),
        ("global_", C.POINTER(C.c_uint8)), ("half_window", C.c_uint32),
        ("rope_theta", _f32p), ("norm_eps", C.c_float), ("vocab", C.c_uint32),
        ("max_positions", C.c_uint32), ("head_layers", C.c_uint32),
        ("head_heads", C.c_uint32), ("head_ff", C.c_uint32),
    ]


class JhEncoderLayer(C.Structure):
    _fields_ = [(n, _f32p) for n in ("attn_norm", "wqkv", "wo", "mlp_norm", "wi", "wo2")]


class JhHeadLayer(C.Structure):
    _fields_ = [(n, _f32p) for n in (
        "norm1_w", "norm1_b", "in_w", "in_b", "out_w", "out_b",
        "norm2_w", "norm2_b", "lin1_w", "lin1_b", "lin2_w", "lin2_b")]


class JhWeights(C.Structure):
    _fields_ = [
        ("embedding", _f32p), ("emb_norm", _f32p), ("layers", C.POINTER(JhEncoderLayer)),
        ("final_norm", _f32p), ("type_emb", _f32p), ("head", C.POINTER(JhHeadLayer)),
        ("scorer_norm_w", _f32p), ("scorer_norm_b", _f32p), ("scorer_w1", _f32p),
        ("scorer_b1", _f32p), ("scorer_w2", _f32p), ("scorer_b2", C.c_float),
    ]


class JhAttnTile(C.Structure):
    _fields_ = [("q_row", C.c_int32), ("nq", C.c_int32), ("kv_row", C.c_int32),
                ("kv_len", C.c_int32), ("q_pos", C.c_int32)]


def fptr(a: np.ndarray | None):
    if a is None:
        return _f32p()
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "weights must be contiguous float32"
    return a.ctypes.data_as(_f32p)


def u32ptr(a: np.ndarray):
    assert a.dtype == np.uint32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def u8ptr(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


@dataclass
class ModelConfig:
    """`ModelConfig` (src/config.rs:6-24) as built by `ModelConfig::from_values` (:43-96)."""
    hidden: int
    heads: int
    head_dim: int
    intermediate: int
    layers: int
    global_: list
    half_window: int
    rope_theta: list
    norm_eps: float
    vocab: int
    max_positions: int
    head_layers: int
    head_heads: int
    head_ff: int

    @staticmethod
    def from_values(julia: dict, enc: dict) -> "ModelConfig":
        """Restates src/config.rs:43-96 (same checks, same derived fields)."""
        if julia.get("format_version") != 1:
            raise ValueError("Unsupported Julia checkpoint format")
        if julia.get("weight_dtype", "float32") not in ("float32", "bfloat16"):
            raise ValueError("Only float32 Julia checkpoints are supported")
        if enc.get("model_type") != "modernbert":
            raise ValueError("Encoder must be ModernBERT")
        for key in ("attention_bias", "mlp_bias", "norm_bias"):
            if enc.get(key) is not False:
                raise ValueError(f"Unsupported encoder setting {key}")
        if enc.get("hidden_activation") != "gelu":
            raise ValueError("Unsupported encoder activation")
        hidden, heads = int(enc["hidden_size"]), int(enc["num_attention_heads"])
        layers, every = int(enc["num_hidden_layers"]), int(enc["global_attn_every_n_layers"])
        local = int(enc["local_attention"])
        if hidden % heads != 0 or hidden // heads != 64:
            raise ValueError("Runtime kernels require head_dim 64")
        types = enc.get("layer_types")
        if types is None:
            types = ["full_attention" if i % every == 0 else "sliding_attention" for i in range(layers)]
        if len(types) != layers:
            raise ValueError("layer_types must list every layer")

        def theta(kind):
            rp = enc.get("rope_parameters")
            if rp is not None and kind in rp:
                if rp[kind].get("rope_type") != "default":
                    raise ValueError("Only default RoPE is supported")
                return float(np.float32(rp[kind]["rope_theta"]))
            key = "global_rope_theta" if kind == "full_attention" else "local_rope_theta"
            return float(np.float32(enc[key]))

        return ModelConfig(
            hidden=hidden, heads=heads, head_dim=hidden // heads,
            intermediate=int(enc["intermediate_size"]), layers=layers,
            global_=[i % every == 0 for i in range(layers)], half_window=local // 2,
            rope_theta=[theta(t) for t in types],
            norm_eps=float(np.float32(enc.get("norm_eps", 1e-5))),
            vocab=int(enc["vocab_size"]), max_positions=int(enc["max_position_embeddings"]),
            head_layers=int(julia["head_layers"]), head_heads=max(hidden // 64, 1), head_ff=4 * hidden)


@dataclass
class WeightSet:
    """ctypes jh_config + jh_weights pointing into a dict of float32 arrays."""
    cfg: ModelConfig
    tensors: dict
    _keep: list = field(default_factory=list)

    def __post_init__(self):
        cfg, t = self.cfg, self.tensors
        g = np.array([1 if x else 0 for x in cfg.global_], dtype=np.uint8)
        th = np.array(cfg.rope_theta, dtype=np.float32)
        self._keep += [g, th]
        self.config = JhConfig(
            cfg.hidden, cfg.heads, cfg.head_dim, cfg.intermediate, cfg.layers,
            u8ptr(g), cfg.half_window, fptr(th), cfg.norm_eps, cfg.vocab,
            cfg.max_positions, cfg.head_layers, cfg.head_heads, cfg.head_ff)
        layers = (JhEncoderLayer * cfg.layers)()
        for l in range(cfg.layers):
            p = f"encoder.layers.{l}."
            layers[l] = JhEncoderLayer(
                fptr(t.get(p + "attn_norm.weight")), fptr(t[p + "attn.Wqkv.weight"]),
                fptr(t[p + "attn.Wo.weight"]), fptr(t[p + "mlp_norm.weight"]),
                fptr(t[p + "mlp.Wi.weight"]), fptr(t[p + "mlp.Wo.weight"]))
        head = (JhHeadLayer * cfg.head_layers)()
        for l in range(cfg.head_layers):
            p = f"head.layers.{l}."
            head[l] = JhHeadLayer(*[fptr(t[p + n]) for n in (
                "norm1.weight", "norm1.bias", "self_attn.in_proj_weight", "self_attn.in_proj_bias",
                "self_attn.out_proj.weight", "self_attn.out_proj.bias", "norm2.weight", "norm2.bias",
                "linear1.weight", "linear1.bias", "linear2.weight", "linear2.bias")])
        self._keep += [layers, head]
        self.weights = JhWeights(
            fptr(t["encoder.embeddings.tok_embeddings.weight"]), fptr(t["encoder.embeddings.norm.weight"]),
            layers, fptr(t["encoder.final_norm.weight"]), fptr(t["type_emb.weight"]), head,
            fptr(t["scorer.0.weight"]), fptr(t["scorer.0.bias"]), fptr(t["scorer.1.weight"]),
            fptr(t["scorer.1.bias"]), fptr(t["scorer.3.weight"]), float(t["scorer.3.bias"][0]))


@dataclass
class Batch:
    """`Batch` (src/model.rs:114-157): packed varlen sequences, no padding."""
    ids: np.ndarray          # uint32 [T]
    starts: np.ndarray       # uint32 [S]
    lens: np.ndarray         # uint32 [S]
    qtypes: np.ndarray       # uint8 [S]
    marker_rows: np.ndarray  # uint32 [M], absolute packed rows grouped by sequence
    marker_starts: np.ndarray  # int64 [S+1]

    @staticmethod
    def from_items(items) -> "Batch":
        """items: iterable of (ids, markers-within-sequence, qtype) — `Batch::new` (src/model.rs:127-147)."""
        ids, starts, lens, qt, rows, mst = [], [], [], [], [], [0]
        n = 0
        for it_ids, it_markers, it_q in items:
            starts.append(n)
            lens.append(len(it_ids))
            qt.append(int(it_q))
            ids.extend(int(v) for v in it_ids)
            rows.extend(n + int(m) for m in it_markers)
            mst.append(len(rows))
            n += len(it_ids)
        return Batch(np.array(ids, dtype=np.uint32), np.array(starts, dtype=np.uint32),
                     np.array(lens, dtype=np.uint32), np.array(qt, dtype=np.uint8),
                     np.array(rows, dtype=np.uint32), np.array(mst, dtype=np.int64))

    @property
    def tokens(self) -> int:
        return int(self.ids.size)

    def split_scores(self, scores):
        """Per-sequence logits (src/model.rs:154-156)."""
        return [np.asarray(scores[a:b]) for a, b in zip(self.marker_starts[:-1], self.marker_starts[1:])]

    def items(self):
        for s in range(self.lens.size):
            a, n = int(self.starts[s]), int(self.lens[s])
            m = self.marker_rows[self.marker_starts[s]:self.marker_starts[s + 1]] - a
            yield self.ids[a:a + n], m, int(self.qtypes[s])

    def subset(self, seqs) -> "Batch":
        items = list(self.items())
        return Batch.from_items([items[i] for i in seqs])
