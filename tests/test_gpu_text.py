"""The text front end over the HIP engine, end to end: TextEngine.load of a
checkpoint directory with a tokenizer (the synthetic byte-level BPE of
synth.write_tokenizer), then Engine::logits, predict_typed, the legacy predict
and the Router on text, against the CPU oracle fed the same encodings
(tests: |dlogit| <= 2e-2, |dsoftmax| <= 1e-2, the parity gates of the forward)."""
import numpy as np
import pytest

from julia1_amd import abi, synth, text
from oracle import oracle
from oracle import text_oracle as TO

pytestmark = pytest.mark.gpu

QTYPE = {"choice": 0, "score": 1, "noul": 2}


@pytest.fixture(scope="module")
def setup(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("ckpt_text"))
    cfg = synth.model_config("tiny")
    t = synth.make_weights(cfg, seed=41)
    synth.write_checkpoint(root, "tiny", t)
    synth.write_tokenizer(root, vocab_size=500)
    te = text.TextEngine.load(root, "hip:0", head_length=64, batch_size=3)
    te.root = root
    return te, oracle.OracleModel(abi.WeightSet(cfg, t), threads=4)


def oracle_logits(te, orc, rows):
    encs = [te.encoder.encode(r, i + 1) for i, r in enumerate(rows)]
    b = abi.Batch.from_items((e["ids"], e["markers"], QTYPE[e["qtype"]]) for e in encs)
    return b.split_scores(orc.forward(b))


ROWS = [
    dict(state="the player has one card left", question="choose the move", options=["play the card", "pass"]),
    dict(state={"turn": 3, "scores": [1.5, -2], "log": ["x x x"]}, question="rate the turn", type="score",
         options=["low", "medium", "high", "very high"]),
    dict(state="x " * 180, question="approve?", type="noul", options=["no", "yes"]),
    dict(state="context", question="route the ticket", options=[f"team {k}" for k in range(12)]),
]


def decided(r, margin=1e-3):
    """The oracle's top choice is decided by more than bf16 round-off (random weights give near-ties)."""
    s = np.sort(np.asarray(r))
    return s.size < 2 or s[-1] - s[-2] > margin


def test_text_logits_match_oracle(setup):
    te, orc = setup
    got = te.logits(ROWS)
    ref = oracle_logits(te, orc, ROWS)
    assert te.engine.forward_count >= 2  # batch_size 3: micro-batched and pipelined
    for g, r in zip(got, ref):
        assert g.shape == r.shape
        assert np.abs(g - r).max() <= 2e-2
        assert np.argmax(g) == np.argmax(r) or not decided(r)


def test_predict_typed_on_text_matches_oracle(setup):
    te, orc = setup
    questions = {
        "team": {"type": "choice", "instructions": "route", "criteria": {"billing": "Payments", "access": "Login"}},
        "severity": {"type": "score", "instructions": "rate", "criteria": ["low", "medium", "high"]},
        "approved": {"type": "noul", "instructions": "approve?"},
    }
    state = {"ticket": "cannot log in", "tries": 3}
    got = te.predict_typed(state, questions)["answers"]
    rows, meta = TO.typed_rows(TO.state_from_value(state), questions)
    plain = [dict(state=r["state"][1], question=r["question"], options=r["options"], type=r["qtype"]) for r in rows]
    want = TO.answers_from_logits(meta, oracle_logits(te, orc, plain))["answers"]
    assert list(got) == list(want)
    for k in want:
        g = np.array(list(got[k]["probabilities"].values()))
        w = np.array(list(want[k]["probabilities"].values()))
        assert np.abs(g - w).max() <= 1e-2


def test_legacy_predict_and_router_on_text(setup):
    te, orc = setup
    pred = te.predict(ROWS, probabilities=True)
    ref = oracle_logits(te, orc, ROWS)
    assert all(p["index"] == int(np.argmax(r)) or not decided(r) for p, r in zip(pred, ref))
    router = te.router(width=5, survivors=2, batch_size=4)
    row = dict(state="the player has one card left", question="choose the move",
               options=[f"card {k}" for k in range(23)])
    res = router.route(row)
    assert res["hierarchical"] and res["index"] in res["candidates"] and res["model_rows"] >= 6
    assert abs(sum(res["probabilities"]) - 1.0) < 1e-9


def test_strict_text_engine_audit(setup):
    """Engine::encoding_info (src/engine.rs:261-280) needs strict encoding; a strict engine rejects a
    marker in the text before any forward."""
    te, _ = setup
    rows = [dict(state="plain text", question="choose", options=["a", "b b"])]
    with pytest.raises(Exception, match="strict_encoding=True"):
        te.encoding_info(rows)
    strict = text.TextEngine.load(te.root, "hip:0", head_length=64, strict_encoding=True)
    info = strict.encoding_info(rows)
    enc = strict.encoder.encode(rows[0])
    assert info == [{"tokens": len(enc["ids"]), "optionTokens": enc["option_tokens"], "headLength": 64,
                     "stateTruncated": False, "optionsTruncated": False}]
    n = strict.engine.forward_count
    with pytest.raises(Exception, match="Reserved model marker"):
        strict.logits([dict(rows[0], state="a <mask> b")])
    assert strict.engine.forward_count == n
