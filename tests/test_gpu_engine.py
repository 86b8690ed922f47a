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
