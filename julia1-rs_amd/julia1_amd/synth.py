"""Seeded synthetic checkpoints and batches for the encoder-forward workloads.

Weights follow the checkpoint layout read by `HostWeights::load`
(src/model.rs:55-110): matrices, embeddings, type_emb, biases and scorer
weights are N(0, 0.02) float32; LayerNorm gains are 1 and LayerNorm biases 0
(N(0, 0.02) gains would collapse every activation to ~0 and tie the logits).
Token ids come from SplitMix64 so that the same seed gives the same batch on
any machine.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np

from .abi import Batch, ModelConfig

MASK64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def encoder_config(hidden=768, heads=12, intermediate=1152, layers=22, every=3, local=128,
                   global_theta=160000.0, local_theta=10000.0, vocab=50368, max_positions=8192):
    return {
        "model_type": "modernbert", "hidden_size": hidden, "num_attention_heads": heads,
        "intermediate_size": intermediate, "num_hidden_layers": layers,
        "global_attn_every_n_layers": every, "local_attention": local,
        "global_rope_theta": global_theta, "local_rope_theta": local_theta,
        "vocab_size": vocab, "max_position_embeddings": max_positions, "norm_eps": 1e-5,
        "hidden_activation": "gelu", "attention_bias": False, "mlp_bias": False, "norm_bias": False,
    }


def julia_config(head_layers=2):
    return {"format_version": 1, "weight_dtype": "float32", "head_layers": head_layers}


# Named model shapes.  "modernbert-base" is the shape of BASELINE.json's configs.  "julia1" is
# the reference's own model as its CUDA path and tests describe it: hidden 384
# (src/cuda/mod.rs:175), Wqkv [1152, 384], Wi [2304, 384] and Wo [384, 1152]
# (src/cpu/gemm.rs:380-438), 22 layers (README:212); the head-layer count is
# not published and is taken as 2.  "julia1-384" is a 6-layer cut of the
# hidden-384 shape for quick tests; "tiny" is small enough for f64 cross-checks.
SHAPES = {
    "modernbert-base": dict(enc=encoder_config(), julia=julia_config(2)),
    "julia1": dict(enc=encoder_config(hidden=384, heads=6, intermediate=1152, layers=22), julia=julia_config(2)),
    "julia1-384": dict(enc=encoder_config(hidden=384, heads=6, intermediate=576, layers=6), julia=julia_config(2)),
    "tiny": dict(enc=encoder_config(hidden=128, heads=2, intermediate=192, layers=3, local=16,
                                    vocab=512, max_positions=256), julia=julia_config(2)),
}


def model_config(shape: str) -> ModelConfig:
    s = SHAPES[shape]
    return ModelConfig.from_values(s["julia"], s["enc"])


def tensor_specs(cfg: ModelConfig):
    """(name, shape, kind) in a fixed order; kind is 'normal', 'ones' or 'zeros'."""
    h, i, ff = cfg.hidden, cfg.intermediate, cfg.head_ff
    out = [("encoder.embeddings.tok_embeddings.weight", (cfg.vocab, h), "normal"),
           ("encoder.embeddings.norm.weight", (h,), "ones")]
    for l in range(cfg.layers):
        p = f"encoder.layers.{l}."
        if l > 0:
            out.append((p + "attn_norm.weight", (h,), "ones"))
        out += [(p + "attn.Wqkv.weight", (3 * h, h), "normal"), (p + "attn.Wo.weight", (h, h), "normal"),
                (p + "mlp_norm.weight", (h,), "ones"), (p + "mlp.Wi.weight", (2 * i, h), "normal"),
                (p + "mlp.Wo.weight", (h, i), "normal")]
    out += [("encoder.final_norm.weight", (h,), "ones"), ("type_emb.weight", (3, h), "normal")]
    for l in range(cfg.head_layers):
        p = f"head.layers.{l}."
        out += [(p + "norm1.weight", (h,), "ones"), (p + "norm1.bias", (h,), "zeros"),
                (p + "self_attn.in_proj_weight", (3 * h, h), "normal"),
                (p + "self_attn.in_proj_bias", (3 * h,), "normal"),
                (p + "self_attn.out_proj.weight", (h, h), "normal"),
                (p + "self_attn.out_proj.bias", (h,), "normal"),
                (p + "norm2.weight", (h,), "ones"), (p + "norm2.bias", (h,), "zeros"),
                (p + "linear1.weight", (ff, h), "normal"), (p + "linear1.bias", (ff,), "normal"),
                (p + "linear2.weight", (h, ff), "normal"), (p + "linear2.bias", (h,), "normal")]
    out += [("scorer.0.weight", (h,), "ones"), ("scorer.0.bias", (h,), "zeros"),
            ("scorer.1.weight", (h, h), "normal"), ("scorer.1.bias", (h,), "normal"),
            ("scorer.3.weight", (1, h), "normal"), ("scorer.3.bias", (1,), "normal")]
    return out


def make_weights(cfg: ModelConfig, seed: int = 0, std: float = 0.02) -> dict:
    rng = np.random.default_rng(seed)
    t = {}
    for name, shape, kind in tensor_specs(cfg):
        if kind == "normal":
            a = rng.standard_normal(shape, dtype=np.float32)
            a *= np.float32(std)
        elif kind == "ones":
            a = np.ones(shape, dtype=np.float32)
        else:
            a = np.zeros(shape, dtype=np.float32)
        t[name] = np.ascontiguousarray(a)
    return t


def weights_sha256(t: dict) -> str:
    h = hashlib.sha256()
    for name in sorted(t):
        h.update(name.encode())
        h.update(np.ascontiguousarray(t[name]).tobytes())
    return h.hexdigest()


def write_checkpoint(root: str, shape: str, tensors: dict) -> str:
    """Checkpoint directory in the layout `Engine::load` reads (src/engine.rs:89-110)."""
    from safetensors.numpy import save_file
    s = SHAPES[shape]
    os.makedirs(os.path.join(root, "encoder"), exist_ok=True)
    with open(os.path.join(root, "julia_config.json"), "w") as f:
        json.dump(s["julia"], f)
    with open(os.path.join(root, "encoder", "config.json"), "w") as f:
        json.dump(s["enc"], f)
    save_file(tensors, os.path.join(root, "model.safetensors"))
    return root


# Special tokens of the synthetic tokenizer, in id order; tokenizer_config.json
# names them as a Julia-1 checkpoint's does (src/encode.rs:70-83).
SPECIAL_TOKENS = ("[PAD]", "[UNK]", "[CLS]", "[SEP]", "<mask>")
TOKENIZER_CONFIG = {"mask_token": "<mask>", "cls_token": "[CLS]", "sep_token": "[SEP]", "pad_token": "[PAD]",
                    "unk_token": "[UNK]"}
_WORDS = ("x", "the", "a", "to", "of", "and", "in", "is", "it", "you", "that", "for", "on", "with", "as", "player",
          "game", "turn", "card", "move", "score", "team", "route", "billing", "access", "login", "payments", "low",
          "medium", "high", "rate", "choose", "question", "choice", "noul", "true", "false", "option", "state",
          "context", "plain", "text", "word", "number", "largest", "approve", "review", "human", "run", "value")


def corpus_words() -> tuple:
    """The words of the synthetic tokenizer's training corpus (for text rows it encodes compactly)."""
    return _WORDS


def train_tokenizer(vocab_size: int = 500):
    """A byte-level BPE `tokenizers.Tokenizer` trained on a seeded synthetic corpus: the stand-in for a
    checkpoint's tokenizer.json (absent here).  " x" is a single token, as in the Julia-1 tokenizer
    (tests/checkpoint.rs:45-46)."""
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers
    rng = np.random.default_rng(1234)
    corpus = []
    for _ in range(3000):
        n = int(rng.integers(3, 14))
        words = [_WORDS[int(i)] for i in rng.integers(0, len(_WORDS), n)]
        corpus.append(" ".join(words) + ("." if rng.random() < 0.5 else ""))
        corpus.append(" ".join(["x"] * int(rng.integers(1, 6))))
        corpus.append(json.dumps({"score": int(rng.integers(0, 100)), "team": _WORDS[int(rng.integers(0, 50))]}))
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=list(SPECIAL_TOKENS), show_progress=False,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(corpus, trainer)
    return tok


def write_tokenizer(root: str, vocab_size: int = 500) -> str:
    """<root>/tokenizer/{tokenizer.json, tokenizer_config.json}, where `Engine::load` reads the encoder
    (src/engine.rs:100-107)."""
    d = os.path.join(root, "tokenizer")
    os.makedirs(d, exist_ok=True)
    train_tokenizer(vocab_size).save(os.path.join(d, "tokenizer.json"))
    with open(os.path.join(d, "tokenizer_config.json"), "w") as f:
        json.dump(TOKENIZER_CONFIG, f)
    return d


class SplitMix64:
    """SplitMix64 stream (Steele, Lea, Flood 2014), vectorised over numpy uint64."""
    GAMMA = np.uint64(0x9E3779B97F4A7C15)

    def __init__(self, seed: int):
        self.state = np.uint64(seed)
        self.count = 0

    def next_u64(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            k = np.arange(self.count + 1, self.count + n + 1, dtype=np.uint64)
            z = self.state + k * self.GAMMA
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            z = z ^ (z >> np.uint64(31))
        self.count += n
        return z

    def below(self, bound: int, n: int) -> np.ndarray:
        """n integers uniform in [0, bound) (multiply-shift on the top 32 bits)."""
        hi = self.next_u64(n) >> np.uint64(32)
        return ((hi * np.uint64(bound)) >> np.uint64(32)).astype(np.int64)


def marker_positions(length: int, n: int) -> list:
    """n option-marker positions spread over the row, clamped inside it."""
    step = max(1, (length - 2) // n)
    return [min(1 + j * step, length - 1) for j in range(n)]


def make_batch(lens, n_options, vocab: int, seed: int) -> Batch:
    """Packed batch: ids uniform in [0, vocab); qtype_s = s mod 3; n_options[s] markers per row."""
    rng = SplitMix64(seed)
    ids = rng.below(vocab, int(np.sum(lens))).astype(np.uint32)
    items, off = [], 0
    for s, (n, k) in enumerate(zip(lens, n_options)):
        items.append((ids[off:off + n], marker_positions(int(n), int(k)), s % 3))
        off += n
    return Batch.from_items(items)


def workload(name: str, vocab: int = 50368) -> Batch:
    """The BASELINE.json workloads (configs[0], [1], [3], [4]) as packed batches."""
    if name == "config0":   # 1 x 128, 4 options, seed 0
        return make_batch([128], [4], vocab, 0)
    if name == "config1":   # 32 rows, lengths U[64,512], 2-20 options, seed 1
        r = SplitMix64(1)
        lens = 64 + r.below(449, 32)
        opts = 2 + r.below(19, 32)
        return make_batch(lens, opts, vocab, 101)
    if name == "config3":   # 4 x 8192, 4 options, seed 3
        return make_batch([8192] * 4, [4] * 4, vocab, 3)
    if name == "config4":   # 256 rows, lengths U[32,1024], 20 options, seed 4
        r = SplitMix64(4)
        lens = 32 + r.below(993, 256)
        return make_batch(lens, [20] * 256, vocab, 104)
    raise KeyError(name)


def padded(batch: Batch, padded_len: int | None = None):
    """[B, Lpad] id matrix (pad id 0), row lengths, qtypes, in-row markers and marker_starts."""
    lens = batch.lens.astype(np.int64)
    L = int(padded_len or lens.max())
    B = lens.size
    ids = np.zeros((B, L), dtype=np.uint32)
    markers = []
    for s, (row_ids, m, _) in enumerate(batch.items()):
        ids[s, :row_ids.size] = row_ids
        markers.extend(int(v) for v in m)
    return (ids, batch.lens.copy(), batch.qtypes.copy(), np.array(markers, dtype=np.uint32),
            batch.marker_starts.astype(np.uint32))
