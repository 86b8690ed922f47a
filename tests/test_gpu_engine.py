"""The C++ host engine on the GPU: Engine::load of a checkpoint directory and
logits_encoded with length-sorted micro-batching, against the CPU oracle on
the same weights (src/engine.rs:89-235)."""
import numpy as np
import pytest

from julia1_amd import abi, engine, synth
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("ckpt"))
    cfg = synth.model_config("tiny")
    t = synth.make_weights(cfg, seed=21)
    synth.write_checkpoint(root, "tiny", t)
    return root, cfg, oracle.OracleModel(abi.WeightSet(cfg, t), threads=4)


def test_engine_matches_oracle(setup):
    root, cfg, orc = setup
    e = engine.Engine.load(root, "hip:0")
    assert e.device_name.startswith("hip:0 (")
    c = e.config()
    assert (c.hidden, c.layers, c.head_layers, c.max_positions) == (128, 3, 2, 256)
    b = synth.make_batch([50, 3, 200, 17, 90, 64, 1, 130], [2, 1, 6, 3, 4, 5, 1, 20], cfg.vocab, 12)
    items = list(b.items())
    got = e.logits_encoded(items)
    ref = b.split_scores(orc.forward(b))
    for g, r in zip(got, ref):
        assert g.shape == r.shape
        assert np.abs(g - r).max() <= 2e-2
        assert np.argmax(g) == np.argmax(r)


def test_micro_batching_does_not_change_results(setup):
    root, cfg, _ = setup
    b = synth.make_batch([50, 3, 200, 17, 90, 64, 1, 130], [2, 1, 6, 3, 4, 5, 1, 20], cfg.vocab, 13)
    items = list(b.items())
    big = engine.Engine.load(root, batch_size=16)
    small = engine.Engine.load(root, batch_size=3, max_batch_tokens=256)
    a = big.logits_encoded(items)
    s = small.logits_encoded(items)
    assert big.forward_count == 1 and small.forward_count >= 3
    for x, y in zip(a, s):
        assert np.abs(x - y).max() <= 1e-5


def test_engine_rejects_rows_over_max_length(setup):
    root, cfg, _ = setup
    e = engine.Engine.load(root, max_length=64)
    from julia1_amd import hip
    with pytest.raises(hip.HipError, match="longer than max_length"):
        e.logits_encoded([(np.zeros(65, dtype=np.uint32), [0], 0)])
    assert e.logits_encoded([]) == []


def test_bf16_checkpoint_gives_identical_logits(setup, tmp_path):
    """A weight_dtype "bfloat16" checkpoint (matrices stored as their BF16
    rounding, FP32-resident tensors kept F32) loads to the same device weights
    as the F32 checkpoint it came from: logits are bit-identical.  Rounding the
    FP32-resident tensors too moves the logits by that rounding only."""
    from julia1_amd import checkpoint
    root, cfg, orc = setup
    half = checkpoint.convert_to_bf16(root, str(tmp_path / "bf16"))
    every = checkpoint.convert_to_bf16(root, str(tmp_path / "all"), all_tensors=True)
    b = synth.make_batch([50, 3, 200, 17, 90, 64, 1, 130], [2, 1, 6, 3, 4, 5, 1, 20], cfg.vocab, 14)
    items = list(b.items())
    want = engine.Engine.load(root).logits_encoded(items)
    got = engine.Engine.load(half).logits_encoded(items)
    rough = engine.Engine.load(every).logits_encoded(items)
    ref = b.split_scores(orc.forward(b))
    for w, g, r, o in zip(want, got, rough, ref):
        assert np.array_equal(w.view(np.uint32), g.view(np.uint32))
        assert np.abs(r - o).max() <= 2e-2


def test_nonfinite_logits_drain_pipelined_batches(setup, tmp_path):
    """Engine::forward's nonfinite check (src/engine.rs:212-223) with micro-batches submitted
    ahead: the error surfaces, the batches still in flight are collected and dropped, and the
    engine keeps working (a second call fails the same way rather than on leaked tickets)."""
    from julia1_amd import hip
    root, cfg, _ = setup
    t = synth.make_weights(cfg, seed=21)
    t["scorer.3.weight"] = np.full_like(t["scorer.3.weight"], np.nan)
    bad = str(tmp_path / "nan")
    synth.write_checkpoint(bad, "tiny", t)
    e = engine.Engine.load(bad, batch_size=2)
    b = synth.make_batch([50, 3, 200, 17, 90, 64, 1, 130], [2, 1, 6, 3, 4, 5, 1, 20], cfg.vocab, 15)
    items = list(b.items())
    for _ in range(2):
        with pytest.raises(hip.HipError, match="nonfinite"):
            e.logits_encoded(items)
    good = engine.Engine.load(root, batch_size=2)
    assert len(good.logits_encoded(items)) == len(items)
