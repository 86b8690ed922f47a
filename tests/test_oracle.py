"""Pins the FP32 CPU oracle (oracle/julia1_oracle.cpp) before it is trusted as
the parity reference.  CPU only.

What pins what:
  fastmath exp/erf/gelu   against libm / math.erf in f64 (src/cpu/fastmath.rs:55-77)
  linear (5 epilogues),   against f64 brute force on the reference's own unit-test
  linear_geglu            shapes and LCG (src/cpu/gemm.rs:358-426)
  layer_norm              against the f64 closed form, incl. widths with a tail
  rope_table              bit-exact against glibc powf/cosf/sinf, and against
                          the product library's table builder
  attention               against f64 softmax(0.125·QKᵀ)·V with varlen, windows
                          and the reductions a window >= len and len = 1 imply
  whole forward           against golden vectors of an independent
                          torch/transformers reconstruction (tests/golden)
  invariants              batching invariance (tests/checkpoint.rs:91-105)
Planted mistakes (jo_set_fault) must each fail the check that covers them.
"""
import ctypes
import hashlib
import json
import math
import os

import numpy as np
import pytest

from julia1_amd import abi, synth
from oracle import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def lcg_stream(seed, n):
    """rnd() of src/cpu/gemm.rs:362-365: u32 LCG, (seed >> 8) / 2^24 - 0.5."""
    out = np.empty(n, dtype=np.float32)
    s = seed
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32((s >> 8) / float(1 << 24) - 0.5)
    return out, s


def test_exp_close_to_libm():
    x = np.arange(-87.0, 88.0, 0.0013, dtype=np.float64).astype(np.float32)
    got = oracle.exp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert np.max(np.abs((got - ref) / ref)) < 3e-7
    assert oracle.exp(np.array([-np.inf], dtype=np.float32))[0] < 1e-37


def test_erf_and_gelu_close_to_libm():
    x = np.arange(-6.0, 6.0, 0.0007, dtype=np.float64).astype(np.float32)
    erf = np.vectorize(math.erf)
    assert np.max(np.abs(oracle.erf(x) - erf(x.astype(np.float64)))) < 1e-6
    g64 = 0.5 * x.astype(np.float64) * (1 + erf(x.astype(np.float64) / math.sqrt(2)))
    assert np.max(np.abs(oracle.gelu(x) - g64)) < 3e-6


@pytest.mark.parametrize("rows,n,k", [(1, 32, 7), (13, 96, 384), (70, 40, 300), (129, 1152, 384)])
def test_linear_matches_naive(rows, n, k):
    seed = 1
    x, seed = lcg_stream(seed, rows * k)
    w, seed = lcg_stream(seed, n * k)
    bias, seed = lcg_stream(seed, n)
    x, w = x.reshape(rows, k), w.reshape(n, k)
    ldo = n + 5
    base, seed = lcg_stream(seed, rows * ldo)
    base = base.reshape(rows, ldo)
    prod = x.astype(np.float64) @ w.astype(np.float64).T
    b64 = bias.astype(np.float64)
    for mode in range(5):
        out = base.copy()
        oracle.linear(x, w, out=out, col=3, epi=mode, bias=bias)
        old = base[:, 3:3 + n].astype(np.float64)
        expect = [prod, old + prod, prod + b64, np.maximum(prod + b64, 0), old + prod + b64][mode]
        assert np.max(np.abs(out[:, 3:3 + n] - expect)) < 1e-4, mode
        assert np.array_equal(out[:, :3], base[:, :3]) and np.array_equal(out[:, 3 + n:], base[:, 3 + n:])


@pytest.mark.parametrize("rows,inter,k", [(1, 64, 384), (21, 128, 100), (300, 1152, 384)])
def test_geglu_matches_naive(rows, inter, k):
    seed = 7
    x, seed = lcg_stream(seed, rows * k)
    w, seed = lcg_stream(seed, 2 * inter * k)
    x, w = x.reshape(rows, k), w.reshape(2 * inter, k)
    prod = x.astype(np.float64) @ w.astype(np.float64).T
    u, v = prod[:, :inter], prod[:, inter:]
    expect = 0.5 * u * (1 + np.vectorize(math.erf)(u / math.sqrt(2))) * v
    assert np.max(np.abs(oracle.linear_geglu(x, w) - expect)) < 1e-4


def test_linear_thread_count_does_not_change_results():
    r = np.random.default_rng(0)
    x = r.standard_normal((77, 256), dtype=np.float32)
    w = r.standard_normal((192, 256), dtype=np.float32)
    oracle.omp_threads(8)
    a = oracle.linear(x, w)
    oracle.omp_threads(1)
    b = oracle.linear(x, w)
    oracle.omp_threads(os.cpu_count() or 4)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("width", [768, 384, 100, 7])
def test_layer_norm_closed_form(width):
    r = np.random.default_rng(width)
    x = (r.standard_normal((50, width)) * 3 + 2).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(width)).astype(np.float32)
    b = (0.1 * r.standard_normal(width)).astype(np.float32)
    x64 = x.astype(np.float64)
    ln = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5)
    assert np.max(np.abs(oracle.layer_norm(x, w, b, 1e-5) - (ln * w + b))) < 2e-5
    assert np.max(np.abs(oracle.layer_norm(x, w, None, 1e-5) - ln * w)) < 2e-5


def test_planted_layer_norm_fault_is_caught():
    r = np.random.default_rng(3)
    x = (r.standard_normal((8, 100)) * 3 + 2).astype(np.float32)
    w = np.ones(100, dtype=np.float32)
    x64 = x.astype(np.float64)
    ln = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5)
    oracle.set_fault(5)
    try:
        bad = oracle.layer_norm(x, w, None, 1e-5)
    finally:
        oracle.set_fault(0)
    assert np.max(np.abs(bad - ln)) > 1e-3


def _libm():
    m = ctypes.CDLL("libm.so.6")
    for f in ("powf", "cosf", "sinf"):
        getattr(m, f).restype = ctypes.c_float
    m.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    m.cosf.argtypes = m.sinf.argtypes = [ctypes.c_float]
    return m


@pytest.mark.parametrize("theta", [10000.0, 160000.0])
def test_rope_table_bit_exact(theta):
    m = _libm()
    c, s = oracle.rope_table(theta, 8192)
    inv = [np.float32(1.0) / np.float32(m.powf(theta, np.float32(2 * i) / np.float32(64))) for i in range(32)]
    for p in list(range(0, 70)) + [1000, 4095, 8191]:
        for i in range(32):
            f = np.float32(inv[i] * np.float32(p))
            assert np.float32(m.cosf(f)).view(np.uint32) == c[p, i].view(np.uint32)
            assert np.float32(m.sinf(f)).view(np.uint32) == s[p, i].view(np.uint32)
    # the product's device tables are built by the same arithmetic
    from julia1_amd import hip
    c2, s2 = hip.rope_table(theta, 8192)
    assert np.array_equal(c.view(np.uint32), c2.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), s2.view(np.uint32))


def _attn64(q, kv, seqs, heads, window, h):
    out = np.zeros((q.shape[0], h))
    for q_row, nq, kv_row, ln in seqs:
        for hh in range(heads):
            sl = slice(hh * 64, hh * 64 + 64)
            Q = q[q_row:q_row + nq, sl].astype(np.float64)
            K = kv[kv_row:kv_row + ln, h + hh * 64:h + hh * 64 + 64].astype(np.float64)
            V = kv[kv_row:kv_row + ln, 2 * h + hh * 64:2 * h + hh * 64 + 64].astype(np.float64)
            sc = 0.125 * Q @ K.T
            if window >= 0:
                i = np.arange(nq)[:, None]
                j = np.arange(ln)[None, :]
                sc = np.where(np.abs(i - j) <= window, sc, -np.inf)
            sc -= sc.max(1, keepdims=True)
            p = np.exp(sc)
            out[q_row:q_row + nq, sl] = (p / p.sum(1, keepdims=True)) @ V
    return out


@pytest.mark.parametrize("window", [-1, 64, 8, 0])
def test_attention_matches_f64(window):
    r = np.random.default_rng(11)
    heads, h = 2, 128
    lens = [1, 5, 33, 64, 65, 130]
    t = sum(lens)
    qkv = r.standard_normal((t, 3 * h), dtype=np.float32)
    seqs, st = [], 0
    for ln in lens:
        seqs.append((st, ln, st, ln))
        st += ln
    got = oracle.attention(qkv, qkv, seqs, heads, window, ldq=3 * h)
    assert np.max(np.abs(got - _attn64(qkv, qkv, seqs, heads, window, h))) < 1e-5


def test_attention_special_cases():
    r = np.random.default_rng(12)
    heads, h = 1, 64
    qkv = r.standard_normal((100, 3 * h), dtype=np.float32)
    seqs = [(0, 100, 0, 100)]
    # a window covering the whole sequence is global attention
    assert np.array_equal(oracle.attention(qkv, qkv, seqs, heads, 100, ldq=3 * h),
                          oracle.attention(qkv, qkv, seqs, heads, -1, ldq=3 * h))
    # a one-token sequence returns its own value row
    one = oracle.attention(qkv[:1], qkv[:1], [(0, 1, 0, 1)], heads, -1, ldq=3 * h)
    assert np.allclose(one[0], qkv[0, 2 * h:3 * h], atol=1e-7)
    # window 0 is each token's own value row
    w0 = oracle.attention(qkv, qkv, seqs, heads, 0, ldq=3 * h)
    assert np.allclose(w0, qkv[:, 2 * h:3 * h], atol=1e-6)


@pytest.fixture(scope="module")
def golden():
    meta = json.load(open(os.path.join(GOLDEN, "tiny_forward.json")))
    g = np.load(os.path.join(GOLDEN, "tiny_forward.npz"))
    cfg = synth.model_config(meta["shape"])
    t = synth.make_weights(cfg, seed=meta["weight_seed"])
    assert synth.weights_sha256(t) == meta["weights_sha256"], "synthetic weight generator drifted"
    b = synth.make_batch(meta["lens"], meta["options"], cfg.vocab, meta["batch_seed"])
    assert np.array_equal(b.ids, g["ids"]) and np.array_equal(b.marker_rows, g["marker_rows"])
    ws = abi.WeightSet(cfg, t)
    return dict(cfg=cfg, t=t, b=b, g=g, ws=ws, model=oracle.OracleModel(ws, threads=4))


def _golden_tol(g):
    return 1e-6 + 1e-4 * np.abs(g["scores"]).max()


def test_forward_matches_golden(golden):
    m, b, g = golden["model"], golden["b"], golden["g"]
    x = m.encode(b, golden["cfg"].layers)
    enc = oracle.layer_norm(x, golden["t"]["encoder.final_norm.weight"], None, 1e-5)
    assert np.max(np.abs(enc - g["encoder_out"])) < 5e-6
    assert np.max(np.abs(m.forward(b) - g["scores"])) < _golden_tol(g)


def test_tiny_layerwise_matches_golden(golden):
    """The residual stream after the embeddings and after every encoder layer, at every 7th token row, against
    the reconstruction's layer outputs (forward hooks on ModernBertModel's embeddings and layers)."""
    m, b, g = golden["model"], golden["b"], golden["g"]
    rows = g["layer_rows"]
    for l in range(golden["cfg"].layers + 1):
        assert np.max(np.abs(m.encode(b, l)[rows] - g["layers"][l])) < 5e-6, l


@pytest.fixture(scope="module")
def base_golden():
    """configs[0] and configs[1] at the ModernBERT-base shape (22 layers, hidden 768, vocab 50368, head_layers 2)
    with the bench's weights (seed 0), against the same independent reconstruction (tests/golden/make_golden.py)."""
    meta = json.load(open(os.path.join(GOLDEN, "base_forward.json")))
    g = np.load(os.path.join(GOLDEN, "base_forward.npz"))
    cfg = synth.model_config(meta["shape"])
    t = synth.make_weights(cfg, seed=meta["weight_seed"])
    assert synth.weights_sha256(t) == meta["weights_sha256"], "synthetic weight generator drifted"
    model = oracle.OracleModel(abi.WeightSet(cfg, t), threads=min(8, os.cpu_count() or 1))
    return dict(cfg=cfg, t=t, g=g, meta=meta, model=model)


def test_base_config0_matches_golden(base_golden):
    bg = base_golden
    m, g, cfg = bg["model"], bg["g"], bg["cfg"]
    b = synth.workload("config0")
    assert hashlib.sha256(b.ids.tobytes()).hexdigest() == bg["meta"]["config0"]["ids_sha256"]
    rows = g["config0_rows"].astype(np.int64)
    for i, l in enumerate(bg["meta"]["base_layers"]):
        assert np.max(np.abs(m.encode(b, l)[rows] - g["config0_layers"][i])) < 2e-5, l
    enc = oracle.layer_norm(m.encode(b, cfg.layers), bg["t"]["encoder.final_norm.weight"], None, cfg.norm_eps)
    assert np.max(np.abs(enc[rows] - g["config0_encoder_out"])) < 2e-5
    assert np.max(np.abs(m.forward(b) - g["config0_scores"])) < 1e-5


def test_base_config1_matches_golden(base_golden):
    bg = base_golden
    m, g, cfg = bg["model"], bg["g"], bg["cfg"]
    b = synth.workload("config1")
    assert hashlib.sha256(b.ids.tobytes()).hexdigest() == bg["meta"]["config1"]["ids_sha256"]
    assert np.max(np.abs(m.forward(b) - g["config1_scores"])) < 1e-5
    enc = oracle.layer_norm(m.encode(b, cfg.layers), bg["t"]["encoder.final_norm.weight"], None, cfg.norm_eps)
    assert np.max(np.abs(enc[g["config1_rows"].astype(np.int64)] - g["config1_encoder_out"])) < 2e-5


@pytest.mark.parametrize("fault", [1, 2, 3, 4])
def test_planted_faults_caught_at_base_shape(base_golden, fault):
    """1 drop type_emb, 2 RoPE sign, 3 window one wider, 4 skip final norm: each moves configs[0]'s scores far
    outside the golden tolerance at the full shape too."""
    b = synth.workload("config0")
    oracle.set_fault(fault)
    try:
        s = base_golden["model"].forward(b)
    finally:
        oracle.set_fault(0)
    assert np.max(np.abs(s - base_golden["g"]["config0_scores"])) > 1e-3


@pytest.mark.parametrize("fault", [1, 2, 3, 4])
def test_planted_forward_faults_are_caught(golden, fault):
    """1 drop type_emb, 2 RoPE sign, 3 window one wider, 4 skip final norm."""
    m, b, g = golden["model"], golden["b"], golden["g"]
    oracle.set_fault(fault)
    try:
        s = m.forward(b)
    finally:
        oracle.set_fault(0)
    assert np.max(np.abs(s - g["scores"])) > _golden_tol(g)


def test_batching_invariance(golden):
    m, b = golden["model"], golden["b"]
    together = b.split_scores(m.forward(b))
    for i in range(b.lens.size):
        assert np.array_equal(m.forward(b.subset([i])), together[i])


def test_oracle_rejects_bad_batches(golden):
    m, b = golden["model"], golden["b"]
    bad = abi.Batch(b.ids.copy(), b.starts, b.lens, b.qtypes, b.marker_rows, b.marker_starts)
    bad.ids[0] = golden["cfg"].vocab
    with pytest.raises(ValueError):
        m.forward(bad)
