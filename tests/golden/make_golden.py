"""Writes tests/golden/tiny_forward.npz: whole-forward golden vectors for the
"tiny" synthetic shape from an independent reconstruction of the Julia-1
decision model built from installed libraries (never from the reference):

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

Run in the development container (needs torch + transformers):
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


def reconstruct(cfg, t, batch):
    from transformers import ModernBertConfig, ModernBertModel

    s = synth.SHAPES[SHAPE]["enc"]
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

    enc_out, scores = [], []
    with torch.no_grad():
        for ids, markers, qtype in batch.items():
            ids_t = torch.from_numpy(ids.astype(np.int64))[None]
            x = enc(input_ids=ids_t, attention_mask=torch.ones_like(ids_t)).last_hidden_state
            enc_out.append(x[0].numpy().copy())
            x = x + type_emb[qtype]
            for layer in head:
                x = layer(x)
            y = x[0, torch.from_numpy(markers.astype(np.int64))]
            scores.append(scorer(y)[:, 0].numpy())
    return np.concatenate(enc_out), np.concatenate(scores)


def main():
    torch.manual_seed(0)
    cfg = synth.model_config(SHAPE)
    t = synth.make_weights(cfg, seed=WEIGHT_SEED)
    batch = synth.make_batch(LENS, OPTIONS, cfg.vocab, BATCH_SEED)
    enc_out, scores = reconstruct(cfg, t, batch)
    meta = dict(shape=SHAPE, weight_seed=WEIGHT_SEED, weights_sha256=synth.weights_sha256(t), lens=LENS,
                options=OPTIONS, batch_seed=BATCH_SEED,
                ids_sha256=hashlib.sha256(batch.ids.tobytes()).hexdigest(),
                source="transformers ModernBertModel (eager, FP32) + torch TransformerEncoderLayer head + scorer")
    np.savez_compressed(os.path.join(HERE, "tiny_forward.npz"), encoder_out=enc_out.astype(np.float32),
                        scores=scores.astype(np.float32), ids=batch.ids, marker_rows=batch.marker_rows)
    with open(os.path.join(HERE, "tiny_forward.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("wrote", enc_out.shape, scores)


if __name__ == "__main__":
    main()
