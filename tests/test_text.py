"""Text front end and callers (include/julia1_text.h, host/text.cpp) on the CPU.

Checked against the reference's own tests (tests/api.rs, the pyjson tests of
src/pyjson.rs:120-156, the tokenizer-level cases of tests/checkpoint.rs:41-74),
against Python's json module (the contract pyjson restates), and against the
pure-Python restatement oracle/text_oracle.py on randomized inputs.  The engine
is replaced by scorer callbacks, as the reference's model-free tests do; the
tokenizer is a byte-level BPE trained by synth.train_tokenizer (the real
checkpoint's tokenizer.json is not available here).
"""
import json
import math
import random
import struct
import zlib

import numpy as np
import pytest

from julia1_amd import hip, synth, text
from oracle import text_oracle as TO

# ------------------------------------------------------------------ pyjson

FLOAT_KATS = [  # src/pyjson.rs:124-139
    (1e16, "1e+16"), (1e15, "1000000000000000.0"), (1e-5, "1e-05"), (1.5e-5, "1.5e-05"), (0.0001, "0.0001"),
    (32.5, "32.5"), (0.1, "0.1"), (-2.0, "-2.0"), (123456789012345678.0, "1.2345678901234568e+17"),
    (1.7976931348623157e308, "1.7976931348623157e+308"), (5e-324, "5e-324"),
]


def test_float_repr_reference_vectors():
    for v, s in FLOAT_KATS:
        assert text.float_repr(v) == s == repr(v)
    assert [text.float_repr(v) for v in (math.nan, math.inf, -math.inf, 0.0, -0.0)] == \
        ["NaN", "Infinity", "-Infinity", "0.0", "-0.0"]


def test_float_repr_matches_python_on_random_doubles():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2**64, 20000, dtype=np.uint64)
    vals = [struct.unpack("<d", struct.pack("<Q", int(b)))[0] for b in bits]
    vals += [float(x) for x in rng.standard_normal(5000) * 10.0 ** rng.integers(-30, 30, 5000)]
    vals += [float(10**k) for k in range(-8, 25)] + [1e16 - 2, 1e16 + 2, 9999999999999998.0, 0.00009999999]
    for v in vals:
        if math.isfinite(v):
            assert text.float_repr(v) == repr(v), v


def test_dumps_reference_vector():
    src = r'{"b": [1, 2.50, -0, 1E5, "é\n\u0001\"\\"], "a": {}, "c": [], "d": null, "e": true}'
    want = r'{"b": [1, 2.5, 0, 100000.0, "é\n\u0001\"\\"], "a": {}, "c": [], "d": null, "e": true}'
    assert text.pyjson_dumps(src) == want == json.dumps(json.loads(src), ensure_ascii=False)


def _random_value(rng, depth=0):
    k = rng.randrange(9 if depth < 4 else 6)
    if k == 0:
        return None
    if k == 1:
        return rng.random() < 0.5
    if k == 2:
        return rng.choice([0, -1, 7, 2**63, -(2**70), 10**30, rng.randrange(-10**6, 10**6)])
    if k == 3:
        return rng.choice([0.5, -0.0, 1e-7, 1e16, 1.5e300, 2.5e-310, rng.uniform(-1e6, 1e6),
                           rng.uniform(-1, 1) * 10.0 ** rng.randrange(-40, 40)])
    if k in (4, 5):
        alphabet = "ab é世\n\t\"\\/\x01\x1f\x7f😀 "
        return "".join(rng.choice(alphabet) for _ in range(rng.randrange(8)))
    if k in (6, 7):
        return [_random_value(rng, depth + 1) for _ in range(rng.randrange(4))]
    return {_random_value(rng, 9) if rng.random() < 0.9 else "k": _random_value(rng, depth + 1)
            for _ in range(rng.randrange(4))}


def test_dumps_matches_python_json_on_random_documents():
    rng = random.Random(11)
    for _ in range(1500):
        v = {"v": _random_value(rng)}
        src = json.dumps(v, ensure_ascii=rng.random() < 0.5, indent=rng.choice([None, 2]))
        assert text.pyjson_dumps(src) == json.dumps(json.loads(src), ensure_ascii=False), src
    for lit in ["1E5", "-0", "2.50", "1e400", "-1e400", "1e-400", "0.1e1", "123456789012345678901234567890",
                "-0.0", "1.0E+2", "5e-324", "[1,2 ,3]", ' {"a" : 1 , "a": 2, "b": 3} ', '"\\u00e9\\ud83d\\ude00"',
                '"\\/"']:
        assert text.pyjson_dumps(lit) == json.dumps(json.loads(lit), ensure_ascii=False), lit


@pytest.mark.parametrize("bad", ["", "{", "[1,]", "01", "1.", ".5", "+1", "NaN", "Infinity", '"\x01"',
                                 '"\\ud800"', '"\\udc00x"', "tru", '{"a" 1}', '{"a":1,}', "[1] 2", "\"abc",
                                 "[" * 129 + "]" * 129])
def test_dumps_rejects_invalid_json(bad):
    with pytest.raises(hip.HipError):
        text.pyjson_dumps(bad)


def test_nesting_limit_is_128():
    assert text.pyjson_dumps("[" * 128 + "]" * 128) == "[" * 128 + "]" * 128


# ------------------------------------------------------------------ scorers (the reference's test doubles)

class Fixed:
    """Returns fixed logits and records the rows it was asked to score (tests/api.rs:10-26)."""

    def __init__(self, logits):
        self.logits, self.calls = logits, []
        self.scorer = text.CallbackScorer(self)

    def __call__(self, rows):
        self.calls.append(rows)
        return self.logits


class Numeric:
    """The logit of an option is its numeric label times `scale` (tests/api.rs:144-156)."""

    def __init__(self, scale):
        self.scale, self.batches = scale, []
        self.scorer = text.CallbackScorer(self)

    def __call__(self, rows):
        self.batches.append(rows)
        return [[np.float32(self.scale) * np.float32(o) for o in r["options"]] for r in rows]


def row_dict(state="context", question="Choose", options=("A", "B"), **kw):
    return dict(state=state, question=question, options=list(options), **kw)


# ------------------------------------------------------------------ requests (tests/api.rs:107-142)

MALFORMED = [
    None, [], row_dict(teacher_logits="bad"), row_dict(teacher_logits=[True, 0.0]), row_dict(options=["A"]),
    row_dict(options=["A", ""]), row_dict(state=3), row_dict(type="other"),
    row_dict(type="noul", options=["a", "b", "c"]), row_dict(target=2),
    # beyond the reference's list: the remaining branches of Request::from_value
    row_dict(question=None), {"question": "q", "options": ["a", "b"]}, row_dict(options=["a"] * 21),
    row_dict(type=None), row_dict(target=-1), row_dict(target=1.0), row_dict(target=None), row_dict(target=True),
    row_dict(teacher_logits=[1, 2, 3]), row_dict(options=["a", 3]),
]


@pytest.mark.parametrize("i", range(len(MALFORMED)))
def test_rejects_malformed_rows(i):
    f = Fixed([[0.0, 1.0]])
    with pytest.raises(hip.HipError, match="JSONL line 1: "):
        f.scorer.logits([MALFORMED[i]])
    with pytest.raises(TO.FrontEndError):
        TO.request_from_value(MALFORMED[i], 1)
    assert not f.calls


def test_valid_rows_and_big_literals_accepted():
    f = Fixed([[0.0, 1.0]])
    for r in [row_dict(), row_dict(type="noul"), row_dict(target=1, teacher_logits=[0, 1.5]),
              row_dict(state={"a": [1, 2.5]}), row_dict(teacher_logits=None), row_dict(state=[])]:
        assert f.scorer.logits([r])[0].tolist() == [0.0, 1.0]
        TO.request_from_value(r, 1)
    from julia1_amd.text import _call_text, _lib
    raw = b'{"state": "s", "question": "q", "options": ["a", "b"], "teacher_logits": [0, 1e400]}'
    with pytest.raises(hip.HipError, match="teacher logits must be finite"):
        _call_text(_lib().jt_logits, f.scorer.h, raw, len(raw))
    big = b'{"state": "s", "question": "q", "options": ["a", "b"], "target": 18446744073709551616}'
    with pytest.raises(hip.HipError, match="target must index"):
        _call_text(_lib().jt_logits, f.scorer.h, big, len(big))


def test_jsonl_line_numbers_and_blank_lines():
    f = Fixed([[0.0, 1.0], [1.0, 0.0]])
    good = json.dumps(row_dict())
    doc = "\n".join([good, "", "   　", good]).encode()
    from julia1_amd.text import _call_text, _lib
    out = json.loads(_call_text(_lib().jt_logits, f.scorer.h, doc, len(doc)))
    assert len(out) == 2 and len(f.calls[0]) == 2
    bad = "\n".join([good, "", "{oops"]).encode()
    with pytest.raises(hip.HipError, match=r"\] line 3: invalid JSON$"):
        _call_text(_lib().jt_logits, f.scorer.h, bad, len(bad))
    with pytest.raises(TO.FrontEndError, match="line 3: invalid JSON"):
        TO.parse_rows(bad.decode())
    bad2 = "\n".join([good, json.dumps(row_dict(options=["a"]))]).encode()
    with pytest.raises(hip.HipError, match="JSONL line 2: options"):
        _call_text(_lib().jt_logits, f.scorer.h, bad2, len(bad2))


# ------------------------------------------------------------------ typed questions (tests/api.rs:33-96)

def test_named_questions_keep_ids_and_full_probabilities():
    f = Fixed([[0.0, 2.0], [0.0, 0.0, 0.0], [0.0, 0.0]])
    questions = {
        "team": {"type": "choice", "instructions": "route", "criteria": {"billing": "Payments", "access": "Login"}},
        "severity": {"type": "score", "instructions": "rate", "criteria": ["low", "medium", "high"]},
        "approved": {"type": "noul", "instructions": "approve?"},
    }
    out = f.scorer.predict_typed("context", questions)
    a = out["answers"]
    assert list(a) == ["team", "severity", "approved"]
    assert a["team"]["choice"] == "access"
    assert abs(a["severity"]["score"] - 1.0) < 1e-12
    assert a["approved"]["noul"] == 0.5
    assert abs(sum(a["team"]["probabilities"].values()) - 1.0) < 1e-12
    assert f.calls[0][0]["options"] == ["Payments", "Login"]
    assert "max_probability" not in a["approved"] and isinstance(a["severity"]["max_probability"], float)
    assert list(a["team"]) == ["type", "probabilities", "choice", "max_probability"]
    rows, meta = TO.typed_rows(TO.state_from_value("context"), questions)
    assert out == TO.answers_from_logits(meta, f.logits)


def test_invalid_questions_rejected_before_inference():
    f = Fixed([])
    many = {str(i): str(i) for i in range(21)}
    for q in [{}, {"q": {"type": "choice", "instructions": "q", "criteria": {"a": "a"}}},
              {"q": {"type": "choice", "instructions": "q", "criteria": many}},
              {"q": {"type": "other", "instructions": "q", "criteria": {"a": "a", "b": "b"}}},
              {"q": {"type": "choice", "criteria": {"a": "a", "b": "b"}}},
              {"q": {"type": "choice", "instructions": "q", "criteria": {"": "a", "b": "b"}}},
              {"q": {"type": "score", "instructions": "q", "criteria": {"a": "a"}}},
              {"": {"type": "noul", "instructions": "q"}}, {"q": "not an object"}, []]:
        with pytest.raises(hip.HipError):
            f.scorer.predict_typed("s", q)
        with pytest.raises(TO.FrontEndError):
            TO.typed_rows(TO.state_from_value("s"), q)
    assert not f.calls
    with pytest.raises(hip.HipError, match="state must be text/JSON"):
        f.scorer.predict_typed(3, {"q": {"type": "noul", "instructions": "q"}})


def test_noul_preserves_descriptions_in_false_true_order():
    f = Fixed([[0.0, 2.0]])
    q = {"review": {"type": "noul", "instructions": "Needs human review?",
                    "criteria": {"true": "A human should inspect this run.",
                                 "false": "No human attention is warranted."}}}
    out = f.scorer.predict_typed({"turn": 3, "scores": [1.5, -0.0]}, q)
    assert f.calls[0][0]["options"] == ["No human attention is warranted.", "A human should inspect this run."]
    assert f.calls[0][0]["state"] == {"turn": 3, "scores": [1.5, -0.0]}
    assert list(out["answers"]["review"]["probabilities"]) == ["false", "true"]
    assert out["answers"]["review"]["noul"] > 0.5


def test_noul_rejects_invalid_criteria_before_inference():
    f = Fixed([[0.0, 2.0]])
    for c in [{}, {"true": "yes"}, {"false": "no", "true": "yes", "other": "maybe"}, ["no", "yes"],
              {"false": "", "true": "yes"}]:
        with pytest.raises(hip.HipError):
            f.scorer.predict_typed("context", {"q": {"type": "noul", "instructions": "q", "criteria": c}})
    assert not f.calls


def test_typed_answers_check_model_output():
    for logits in ([[0.0, 1.0]], [[0.0, 1.0], [1.0]], [[0.0, float("nan")]]):
        f = Fixed(logits)
        q = {"a": {"type": "noul", "instructions": "q"}, "b": {"type": "noul", "instructions": "q"}}
        with pytest.raises(hip.HipError, match="answer count|Invalid model scores"):
            f.scorer.predict_typed("s", q)


def test_typed_random_against_restatement():
    rng = random.Random(3)
    for _ in range(200):
        qs, logits = {}, []
        for j in range(rng.randrange(1, 6)):
            kind = rng.choice(["choice", "score", "noul"])
            n = 2 if kind == "noul" else rng.randrange(2, 21)
            if kind == "choice":
                crit = {f"id{k}": f"desc {k}" for k in range(n)}
            elif kind == "score":
                crit = [f"level {k}" for k in range(n)]
            else:
                crit = rng.choice([None, {"false": "no", "true": "yes"}])
            qs[f"q{j}"] = {"type": kind, "instructions": "do it", "criteria": crit}
            logits.append([float(np.float32(rng.gauss(0, 3))) for _ in range(n)])
        f = Fixed(logits)
        assert f.scorer.predict_typed("ctx", qs) == TO.answers_from_logits(TO.typed_rows(("t", "ctx"), qs)[1],
                                                                              logits)


# ------------------------------------------------------------------ legacy predict + display

def test_display_rounds_decisive_answer_and_redistributes_small_values():
    assert text.display_probabilities([0.955, 0.044, 0.001]) == [1.0, 0.0, 0.0]
    assert text.display_probabilities([0.951, 0.049]) != [1.0, 0.0]
    r = text.display_probabilities([0.6, 0.395, 0.005])
    assert r[2] == 0.0 and abs(sum(r) - 1.0) < 1e-12 and abs(r[0] / r[1] - 0.6 / 0.395) < 1e-12
    rng = random.Random(4)
    for _ in range(500):
        v = [rng.random() ** 3 for _ in range(rng.randrange(1, 8))]
        s = sum(v)
        v = [x / s for x in v]
        assert text.display_probabilities(v) == TO.display_probabilities(v)
    assert text.display_probabilities([]) == []


def test_predict_legacy_against_restatement():
    rng = np.random.default_rng(8)
    logits = [rng.standard_normal(int(rng.integers(2, 21))).astype(np.float32) * 4 for _ in range(50)]
    logits.append(np.array([3.0, 3.0, -1.0], dtype=np.float32))  # first-max rule
    f = Fixed([z.tolist() for z in logits])
    rows = [row_dict(options=[f"o{k}" for k in range(z.size)]) for z in logits]
    got = f.scorer.predict(rows, probabilities=True)
    want = TO.predict(logits, True)
    assert [g["index"] for g in got] == [w["index"] for w in want]
    assert got[-1]["index"] == 0
    for g, w in zip(got, want):
        # f32 softmax: glibc expf here, numpy's float32 exp in the restatement (both within 1 ulp)
        assert np.allclose(g["probabilities"], w["probabilities"], rtol=1e-5, atol=1e-7)
    assert "probabilities" not in Fixed([logits[0].tolist()]).scorer.predict(rows[:1])[0]


# ------------------------------------------------------------------ router (tests/api.rs:158-211)

def request(n, qtype="choice"):
    return dict(state="Olá, 世界", question="Choose the largest number", options=[str(i) for i in range(n)],
                type=qtype)


def test_router_direct_and_hierarchical():
    e = Numeric(1.0)
    router = text.Router(e.scorer, 20, 2, 3, 0, 4096)
    res = router.route_many([request(n) for n in (2, 20, 21, 77, 4096)])
    assert [r["index"] for r in res] == [1, 19, 20, 76, 4095]
    for r in res:
        assert abs(sum(r["probabilities"]) - 1.0) < 1e-9
        assert r["index"] in r["candidates"]
    assert res[0]["probability_scope"] == "all_options" and res[4]["probability_scope"] == "final_candidates"
    assert all(len(b) <= 3 for b in e.batches)
    assert all(2 <= len(r["options"]) <= 20 for b in e.batches for r in b)
    assert router.route_many([]) == []


def test_router_confident_group_shortcut():
    assert text.confident_winner([0.0, 4.0, -3.0], 1) and TO.confident_winner([0.0, 4.0, -3.0], 1)
    assert not text.confident_winner([0.0, 3.0, -3.0], 1) and not TO.confident_winner([0.0, 3.0, -3.0], 1)
    e = Numeric(10.0)
    r = text.Router(e.scorer).route(request(2001))
    assert (r["index"], r["rounds"], r["model_rows"]) == (2000, 3, 106)


def test_router_cache_and_dedup():
    e = Numeric(1.0)
    router = text.Router(e.scorer, 20, 2, 16, 1, 4096)
    res = router.route_many([request(5), request(5)])
    assert (res[0]["model_rows"], res[0]["cache_hits"]) == (1, 1)
    assert router.route(request(5))["model_rows"] == 0
    router.clear_cache()
    assert router.route(request(5))["model_rows"] == 1
    router.route(request(6))
    assert router.route(request(5))["model_rows"] == 1


def test_router_rejects_invalid_and_bad_engines():
    e = Numeric(1.0)
    router = text.Router(e.scorer)
    for r in [request(1), request(30, "score"), request(3, "noul"), dict(request(4), options=["1", "", "2", "3"])]:
        with pytest.raises(hip.HipError):
            router.route(r)
    bad = Fixed([[0.0]])
    with pytest.raises(hip.HipError, match="finite and match option count"):
        text.Router(bad.scorer).route(request(4))
    for args in [(1, 0), (21, 2), (20, 20), (20, 0)]:
        with pytest.raises(hip.HipError, match="width"):
            text.Router(e.scorer, *args)
    with pytest.raises(hip.HipError, match="capacity"):
        text.Router(e.scorer, 20, 2, 16, 0, 19)


def test_router_random_against_restatement():
    rng = random.Random(9)

    def fn(rows):
        # deterministic pseudo-logits per (option text, question) so dedup and caching see equal rows equal
        return [[float(np.float32(((zlib.crc32((o + r["question"]).encode()) % 2003) - 1000) / 97.0))
                 for o in r["options"]] for r in rows]

    for _ in range(40):
        width = rng.randrange(2, 21)
        survivors = rng.randrange(1, width)
        batch = rng.randrange(1, 9)
        rows = [dict(state=rng.choice(["s", {"k": [1, 2.5]}]), question=f"q{rng.randrange(3)}",
                     options=[f"opt{rng.randrange(400)}" for _ in range(rng.randrange(2, 300))])
                for _ in range(rng.randrange(1, 4))]
        s = text.CallbackScorer(fn)
        got = text.Router(s, width, survivors, batch, 0, 4096).route_many(rows)
        want = TO.route_many(fn, rows, width, survivors, batch)
        assert got == want


# ------------------------------------------------------------------ encoder (src/encode.rs)

@pytest.fixture(scope="module")
def tok():
    return text.Tokenizer(synth.train_tokenizer())


CFG = json.dumps(synth.TOKENIZER_CONFIG)


def special_of(enc):
    s = enc.special_ids
    return dict(mask_token="<mask>", mask=s["mask"], cls=s["cls"], sep=s["sep"])


def oracle_encode(tok, enc, max_length, head_length, strict, row):
    t = lambda s: tok.tok.encode(s, add_special_tokens=False).ids  # noqa: E731
    return TO.sequence(t, special_of(enc), max_length, head_length, strict, TO.request_from_value(row, 1))


def test_encoder_special_tokens_and_config_errors(tok):
    enc = text.Encoder(tok, CFG, 512)
    assert enc.special_ids == dict(mask=4, cls=2, sep=3, pad=0)
    with pytest.raises(hip.HipError, match="tokenizer lacks cls_token"):
        text.Encoder(tok, json.dumps({"mask_token": "<mask>"}), 512)
    with pytest.raises(hip.HipError, match="unknown sep_token <nope>"):
        text.Encoder(tok, json.dumps(dict(synth.TOKENIZER_CONFIG, sep_token="<nope>")), 512)
    with pytest.raises(hip.HipError, match="max_length must leave room"):
        text.Encoder(tok, CFG, 260, head_length=256)


def _random_row(rng, allow_mask=True, option_words=70):
    words = ["x", "the", "player", "turn", "card", "score", "é", "世界", "choose", "1.5", "\n", "  "]
    if allow_mask:
        words.append("<mask>")
    say = lambda k: " ".join(rng.choice(words) for _ in range(k))  # noqa: E731
    n = rng.randrange(2, 21)
    kind = rng.choice(["choice", "score", "noul"])
    if kind == "noul":
        n = 2
    state = rng.choice([say(rng.randrange(0, 400)), {"turn": rng.randrange(50), "log": [say(5), 2.5, None]},
                        [say(3), {"x": "<mask>" if allow_mask else "y"}]])
    return dict(state=state, question=say(rng.randrange(0, 60)), options=[say(rng.randrange(1, option_words)) or "o"
                                                                         for _ in range(n)], type=kind)


@pytest.mark.parametrize("max_length,head_length,strict", [(512, 256, False), (128, 32, False), (64, 24, False),
                                                           (1024, 256, True), (300, 64, True)])
def test_encoder_matches_restatement(tok, max_length, head_length, strict):
    enc = text.Encoder(tok, CFG, max_length, head_length=head_length, strict=strict)
    rng = random.Random(max_length * 7 + head_length)
    ok = err = 0
    for _ in range(150):
        row = _random_row(rng, allow_mask=not strict or rng.random() < 0.1, option_words=12 if strict else 70)
        try:
            want = oracle_encode(tok, enc, max_length, head_length, strict, row)
        except TO.FrontEndError as e:
            with pytest.raises(hip.HipError, match=str(e).split(";")[0]):
                enc.encode(row)
            err += 1
            continue
        got = enc.encode(row)
        assert got == want
        assert len(got["ids"]) <= max_length
        assert all(got["ids"][m] == enc.special_ids["mask"] for m in got["markers"])
        ok += 1
    assert ok >= (5 if strict else 20)


def test_full_budget_and_strict_overflow(tok):
    """tests/checkpoint.rs:41-50 on the synthetic tokenizer (" x" is one token)."""
    enc = text.Encoder(tok, CFG, 8192, head_length=256, strict=True, token_cache=0, encoding_cache=0)
    row = lambda s: dict(state=s, question="choose", options=["a", "b"])  # noqa: E731
    overhead = len(enc.encode(row(""))["ids"])
    fill = lambda n: " ".join(["x"] * n)  # noqa: E731
    assert len(enc.encode(row(fill(8192 - overhead)))["ids"]) == 8192
    with pytest.raises(hip.HipError, match="lossless context budget"):
        enc.encode(row(fill(8193 - overhead)))


def test_batch_tokenization_matches_per_text(tok):
    """Engine::encode (src/engine.rs:183-188) encodes rows in parallel with encode_fast; here every distinct
    segment the uncached rows need goes to one batch-tokenizer call. The encodings equal those of per-text
    calls, and rows or segments already cached are not tokenized again."""
    per = text.Encoder(text.Tokenizer(tok.tok, batch=False), CFG, 1024, head_length=256, strict=True)
    rng = random.Random(5)
    rows = []
    while len(rows) < 40:
        r = _random_row(rng, allow_mask=False, option_words=12)
        try:
            per.encode(r)
        except hip.HipError:
            continue
        rows.append(r)
    rows += rows[:5]  # repeated rows
    bt = text.Tokenizer(tok.tok)
    calls, fast = [], bt._fast
    bt._fast = lambda texts, **kw: (calls.append(list(texts)), fast(texts, **kw))[1]  # noqa: E731
    bat = text.Encoder(bt, CFG, 1024, head_length=256, strict=True)
    assert bat.encoding_info(rows) == per.encoding_info(rows)
    assert len(calls) == 1 and len(set(calls[0])) == len(calls[0])
    assert bat.encoding_info(rows) == per.encoding_info(rows) and len(calls) == 1  # all cached now
    for r in rows:
        assert bat.encode(r) == per.encode(r)
    # without caches every row is assembled from the one batch call
    calls.clear()
    nocache = text.Encoder(bt, CFG, 1024, head_length=256, strict=True, token_cache=0, encoding_cache=0)
    assert nocache.encoding_info(rows) == per.encoding_info(rows) and len(calls) == 1
    # a single row keeps the per-text calls
    assert nocache.encoding_info(rows[:1]) == per.encoding_info(rows[:1]) and len(calls) == 1


class CountingTokenizer(text.Tokenizer):
    calls = 0

    def _encode_cb(self, *a):
        CountingTokenizer.calls += 1
        return super()._encode_cb(*a)


def test_strict_encoding_rejects_markers_and_loss_and_caches():
    """tests/checkpoint.rs:52-74 on the synthetic tokenizer; cache reuse is seen as no tokenizer calls."""
    tok = CountingTokenizer(synth.train_tokenizer())
    enc = text.Encoder(tok, CFG, 1024, head_length=256, strict=True, token_cache=16, encoding_cache=16)
    row = lambda s: dict(state=s, question="choose", options=["a", "b"])  # noqa: E731
    first = enc.encode(row("plain text"))
    n = CountingTokenizer.calls
    assert enc.encode(row("plain text")) == first and CountingTokenizer.calls == n
    assert len(first["markers"]) == 2 and all(first["ids"][m] == 4 for m in first["markers"])
    for bad in [row("<mask>"), dict(row(""), state={"value": "<mask>"}), dict(row("x"), options=["word " * 49, "b"]),
                row("x " * 2000)]:
        with pytest.raises(hip.HipError):
            enc.encode(bad)
    enc.clear_cache()
    enc.encode(row("plain text"))
    assert CountingTokenizer.calls > n
    lax = text.Encoder(tok, CFG, 64, head_length=32, strict=False, token_cache=0, encoding_cache=0)
    e = lax.encode(row("<mask> " + "x " * 200))
    assert e["truncated"] and len(e["ids"]) == 64 and e["ids"].count(4) == 2


def test_encoding_info_requires_strict(tok):
    rows = [dict(state="plain text", question="choose", options=["a", "bb b"])]
    with pytest.raises(hip.HipError, match="strict_encoding=True"):
        text.Encoder(tok, CFG, 512).encoding_info(rows)
    info = text.Encoder(tok, CFG, 512, strict=True).encoding_info(rows)
    want = oracle_encode(tok, text.Encoder(tok, CFG, 512), 512, 256, True, rows[0])
    assert info == [{"tokens": len(want["ids"]), "optionTokens": want["option_tokens"], "headLength": 256,
                     "stateTruncated": False, "optionsTruncated": False}]


def test_tokenizer_failure_is_reported(tok):
    class Broken(text.Tokenizer):
        def _encode_cb(self, *a):
            return 1

    enc = text.Encoder(Broken(synth.train_tokenizer()), CFG, 512)
    with pytest.raises(hip.HipError, match="tokenizer failed"):
        enc.encode(row_dict())


def test_invalid_utf8_rejected(tok):
    enc = text.Encoder(tok, CFG, 512)
    from julia1_amd.text import _call_text, _lib
    b = b'{"state": "\xff", "question": "q", "options": ["a", "b"]}'
    with pytest.raises(hip.HipError, match="UTF-8"):
        _call_text(_lib().jt_encode, enc.h, b, len(b), 1)
