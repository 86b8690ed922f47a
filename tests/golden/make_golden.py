"""Writes whole-forward golden vectors from an independent reconstruction of
the Julia-1 decision model built from installed libraries (never from the
reference):

  tiny_forward.npz / .json   the "tiny" synthetic shape: encoder output, scores,
                             and the residual stream after the embeddings and
                             after every encoder layer (every 7th token row);
  base_forward.npz / .json   the ModernBERT-base shape of BASELINE.json with the
                             bench's weights (seed 0): configs[0] (one 128-token
                             row) and configs[1] (32 rows, 9482 tokens) scores,
                             the encoder output at configs[0]'s marker rows and
                             at the first marker row of each configs[1] sequence,
                             and configs[0]'s residual streams after layers 0, 11
                             and 22 at its marker rows.

The reconstruction:

  encoder  transformers ModernBertModel (FP32, eager attention), one sequence
           at a time so there is no padding;
  head     final_norm output + type_emb[qtype], then torch
           nn.TransformerEncoderLayer(norm_first=True, activation="relu",
           batch_first=True, dropout=0) per head layer over the whole
           sequence, then the marker rows;
  scorer   nn.Sequential(LayerNorm, Linear, GELU, Linear(h, 1)) (checkpoint keys scorer.{0,1,3}).

This is the composition the reference's CPU path implements
(src/cpu/mod.rs:201-340); the reconstruction runs the LAST head layer over
every token and gathers the markers afterwards, so it also pins the
reference's marker-only shortcut (src/cpu/mod.rs:287-321).

Run in the development container (needs torch + transformers; a few minutes on 8 CPUs):
    python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "julia1-rs_amd"))

from julia1_amd import synth  # noqa: E402

SHAPE = "tiny"
WEIGHT_SEED = 11
LENS = [40, 1, 17, 130, 3]
OPTIONS = [3, 1, 2, 5, 2]
BATCH_SEED = 5


TINY_ROW_STEP = 7            # tiny per-layer residuals: every 7th token row
BASE_LAYERS = (0, 11, 22)    # base residual streams at the marker rows after these many layers


def reconstruct(cfg, t, batch, shape, layer_rows=None):
    """Scores per marker and the final encoder output for `batch`.  With layer_rows(seq_index, length) -> row
    indices, also the residual stream after the embeddings (index 0) and after every encoder layer
    (index l + 1) at those rows, captured with forward hooks on the embedding module and the layers."""
    from transformers import ModernBertConfig, ModernBertModel

    s = synth.SHAPES[shape]["enc"]
    hf = ModernBertConfig(
        vocab_size=s["vocab_size"], hidden_size=s["hidden_size"], intermediate_size=s["intermediate_size"],
        num_hidden_layers=s["num_hidden_layers"], num_attention_heads=s["num_attention_heads"],
        global_attn_every_n_layers=s["global_attn_every_n_layers"], local_attention=s["local_attention"],
        global_rope_theta=s["global_rope_theta"], local_rope_theta=s["local_rope_theta"],
        max_position_embeddings=s["max_position_embeddings"], norm_eps=s["norm_eps"], norm_bias=False,
        attention_bias=False, mlp_bias=False, hidden_activation="gelu", embedding_dropout=0.0,
        attention_dropout=0.0, mlp_dropout=0.0, pad_token_id=0, bos_token_id=1, eos_token_id=2, cls_token_id=1,
        sep_token_id=2)
    hf._attn_implementation = "eager"
    enc = ModernBertModel(hf).eval()
    sd = {k[len("encoder."):]: torch.from_numpy(v) for k, v in t.items() if k.startswith("encoder.")}
    missing, unexpected = enc.load_state_dict(sd, strict=False)
    assert not unexpected and all("inv_freq" in m for m in missing), (missing, unexpected)

    h, ff = cfg.hidden, cfg.head_ff
    head = []
    for l in range(cfg.head_layers):
        layer = torch.nn.TransformerEncoderLayer(h, cfg.head_heads, ff, dropout=0.0, activation="relu",
                                                 batch_first=True, norm_first=True, layer_norm_eps=1e-5).eval()
        p = f"head.layers.{l}."
        layer.load_state_dict({k[len(p):]: torch.from_numpy(v) for k, v in t.items() if k.startswith(p)})
        head.append(layer)
    scorer = torch.nn.Sequential(torch.nn.LayerNorm(h, eps=1e-5), torch.nn.Linear(h, h), torch.nn.GELU(),
                                 torch.nn.Linear(h, 1)).eval()
    scorer.load_state_dict({k[len("scorer."):]: torch.from_numpy(v) for k, v in t.items()
                            if k.startswith("scorer.")})
    type_emb = torch.from_numpy(t["type_emb.weight"])

    captured = []
    hooks = [enc.embeddings.register_forward_hook(lambda mod, inp, out: captured.append(out))]
    for layer in enc.layers:
        hooks.append(layer.register_forward_hook(
            lambda mod, inp, out: captured.append(out[0] if isinstance(out, tuple) else out)))
    enc_out, scores, streams = [], [], []
    with torch.no_grad():
        for si, (ids, markers, qtype) in enumerate(batch.items()):
            captured.clear()
            ids_t = torch.from_numpy(ids.astype(np.int64))[None]
            x = enc(input_ids=ids_t, attention_mask=torch.ones_like(ids_t)).last_hidden_state
            assert len(captured) == cfg.layers + 1
            if layer_rows is not None:
                rows = torch.from_numpy(np.asarray(layer_rows(si, len(ids)), dtype=np.int64))
                streams.append(np.stack([c[0, rows].numpy() for c in captured]))
            enc_out.append(x[0].numpy().copy())
            x = x + type_emb[qtype]
            for layer in head:
                x = layer(x)
            y = x[0, torch.from_numpy(markers.astype(np.int64))]
            scores.append(scorer(y)[:, 0].numpy())
    for h_ in hooks:
        h_.remove()
    layers = np.concatenate(streams, axis=1) if streams else None
    return np.concatenate(enc_out), np.concatenate(scores), layers


SOURCE = "transformers ModernBertModel (eager, FP32) + torch TransformerEncoderLayer head + scorer"


def tiny():
    cfg = synth.model_config(SHAPE)
    t = synth.make_weights(cfg, seed=WEIGHT_SEED)
    batch = synth.make_batch(LENS, OPTIONS, cfg.vocab, BATCH_SEED)
    step_rows = lambda si, n: np.arange(0, n, TINY_ROW_STEP)
    enc_out, scores, layers = reconstruct(cfg, t, batch, SHAPE, step_rows)
    # packed row index of every captured row, in capture order
    rows = np.concatenate([int(a) + step_rows(i, int(n)) for i, (a, n) in enumerate(zip(batch.starts, batch.lens))])
    meta = dict(shape=SHAPE, weight_seed=WEIGHT_SEED, weights_sha256=synth.weights_sha256(t), lens=LENS,
                options=OPTIONS, batch_seed=BATCH_SEED, layer_row_step=TINY_ROW_STEP,
                ids_sha256=hashlib.sha256(batch.ids.tobytes()).hexdigest(), source=SOURCE)
    np.savez_compressed(os.path.join(HERE, "tiny_forward.npz"), encoder_out=enc_out.astype(np.float32),
                        scores=scores.astype(np.float32), ids=batch.ids, marker_rows=batch.marker_rows,
                        layer_rows=rows.astype(np.int64), layers=layers.astype(np.float32))
    with open(os.path.join(HERE, "tiny_forward.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("tiny: wrote", enc_out.shape, layers.shape, scores)


def base():
    """configs[0] and configs[1] at the ModernBERT-base shape with the bench's weights (seed 0)."""
    cfg = synth.model_config("modernbert-base")
    t = synth.make_weights(cfg, seed=0)
    out, meta = {}, dict(shape="modernbert-base", weight_seed=0, weights_sha256=synth.weights_sha256(t),
                         base_layers=list(BASE_LAYERS), source=SOURCE)
    for wl in ("config0", "config1"):
        batch = synth.workload(wl)
        mk = [np.asarray(m, dtype=np.int64) for _, m, _ in batch.items()]
        enc_out, scores, layers = reconstruct(cfg, t, batch, "modernbert-base", lambda si, n: mk[si])
        out[f"{wl}_scores"] = scores.astype(np.float32)
        # encoder output and residual streams at each sequence's first marker row (configs[0]: every marker
        # row), so the fixture stays small
        sel = np.arange(batch.marker_rows.size) if wl == "config0" else batch.marker_starts[:-1].astype(np.int64)
        out[f"{wl}_rows"] = batch.marker_rows[sel]
        out[f"{wl}_encoder_out"] = enc_out[batch.marker_rows[sel].astype(np.int64)].astype(np.float32)
        if wl == "config0":
            out[f"{wl}_layers"] = layers[list(BASE_LAYERS)][:, sel].astype(np.float32)
        meta[wl] = dict(tokens=batch.tokens, markers=int(batch.marker_rows.size),
                        ids_sha256=hashlib.sha256(batch.ids.tobytes()).hexdigest())
        print(f"base {wl}: {batch.tokens} tokens, {scores.size} scores, first {scores[:4]}", flush=True)
    np.savez_compressed(os.path.join(HERE, "base_forward.npz"), **out)
    with open(os.path.join(HERE, "base_forward.json"), "w") as f:
        json.dump(meta, f, indent=1)


def main():
    torch.manual_seed(0)
    torch.set_num_threads(max(1, os.cpu_count() or 1))
    which = sys.argv[1:] or ["tiny", "base"]
    if "tiny" in which:
        tiny()
    if "base" in which:
        base()


if __name__ == "__main__":
    main()
