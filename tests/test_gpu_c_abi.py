"""The C-ABI from a plain C99 program linked against the static library.

tests/c_abi/jh_caller.c includes only include/julia1_hip.h and is linked by
julia1-rs_amd/build.py against libjulia1_hip.a with the system toolchain and
the HIP runtime, as a Rust `Backend::Hip` arm's build.rs would link it
(src/engine.rs:67-71, 158-169 select the backend; build.rs:11-32 builds the
CUDA one).  It runs in a fresh child process: jh_create on the synthetic tiny
checkpoint's weights, jh_name, jh_forward, a rejected batch, jh_forward
again, jh_destroy.  Its scores are held to the same gates as the ctypes path
against the FP32 CPU oracle.
"""
import os
import subprocess

import numpy as np
import pytest

from julia1_amd import abi, build_paths, synth
from julia1_amd import parity as par
from oracle import oracle

pytestmark = pytest.mark.gpu


def write_weights(path, ws):
    """The caller's weight file: 4-byte words, u32 config fields then f32 tensors (see jh_caller.c)."""
    c, t = ws.cfg, ws.tensors
    words = [np.array([0x3157484A, c.hidden, c.heads, c.head_dim, c.intermediate, c.layers, c.half_window, c.vocab,
                       c.max_positions, c.head_layers, c.head_heads, c.head_ff], dtype=np.uint32),
             np.array([c.norm_eps, t["scorer.3.bias"][0]], dtype=np.float32),
             np.array([1 if g else 0 for g in c.global_], dtype=np.uint32),
             np.array(c.rope_theta, dtype=np.float32),
             t["encoder.embeddings.tok_embeddings.weight"], t["encoder.embeddings.norm.weight"]]
    for l in range(c.layers):
        p = f"encoder.layers.{l}."
        an = t.get(p + "attn_norm.weight")
        words.append(np.array([0 if an is None else 1], dtype=np.uint32))
        if an is not None:
            words.append(an)
        words += [t[p + n] for n in ("attn.Wqkv.weight", "attn.Wo.weight", "mlp_norm.weight", "mlp.Wi.weight",
                                     "mlp.Wo.weight")]
    words += [t["encoder.final_norm.weight"], t["type_emb.weight"]]
    for l in range(c.head_layers):
        p = f"head.layers.{l}."
        words += [t[p + n] for n in ("norm1.weight", "norm1.bias", "self_attn.in_proj_weight",
                                     "self_attn.in_proj_bias", "self_attn.out_proj.weight", "self_attn.out_proj.bias",
                                     "norm2.weight", "norm2.bias", "linear1.weight", "linear1.bias", "linear2.weight",
                                     "linear2.bias")]
    words += [t[n] for n in ("scorer.0.weight", "scorer.0.bias", "scorer.1.weight", "scorer.1.bias",
                             "scorer.3.weight")]
    with open(path, "wb") as f:
        for a in words:
            a = np.ascontiguousarray(a)
            assert a.dtype.itemsize == 4
            f.write(a.tobytes())


def write_batch(path, b):
    with open(path, "wb") as f:
        f.write(np.array([0x3142484A, b.tokens, b.lens.size, b.marker_rows.size], dtype=np.uint32).tobytes())
        for a in (b.ids, b.starts, b.lens, b.qtypes.astype(np.uint32), b.marker_rows):
            f.write(np.ascontiguousarray(a, dtype=np.uint32).tobytes())


@pytest.mark.parametrize("shape", ["tiny", "julia1-384"])
def test_c_caller_static_library(tmp_path, shape):
    assert os.access(build_paths.CALLER, os.X_OK), "run julia1-rs_amd/build.py first"
    cfg = synth.model_config(shape)
    ws = abi.WeightSet(cfg, synth.make_weights(cfg, seed=5))
    b = synth.make_batch([61, 130, 9, 200], [3, 5, 2, 4], cfg.vocab, seed=6)
    wpath, bpath, spath = (str(tmp_path / n) for n in ("w.bin", "b.bin", "s.bin"))
    write_weights(wpath, ws)
    write_batch(bpath, b)
    print(f"running {build_paths.CALLER} on {shape}", flush=True)
    r = subprocess.run([build_paths.CALLER, wpath, bpath, spath], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert "name=hip:0 (" in r.stdout
    assert "rejected=token id out of vocabulary" in r.stdout
    got = np.fromfile(spath, dtype=np.float32)
    assert got.size == b.marker_rows.size and np.all(np.isfinite(got))
    ref = oracle.OracleModel(ws, threads=4).forward(b)
    s = par.report(b.split_scores(got), b.split_scores(ref))
    print(s)
    par.check_gates(s)
