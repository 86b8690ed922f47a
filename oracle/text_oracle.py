"""Pure-Python restatement of the reference's text front end and callers.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the C++ front
end (julia1-rs_amd/host/text.cpp, include/julia1_text.h).  The product path
never imports this module.

Each function follows the reference's Rust (file:line in its docstring) on
Python JSON values (json.loads with insertion-ordered dicts: ints for literals
without '.', 'e' or 'E', floats otherwise, which is also how the reference's
pyjson reads numbers).  pyjson itself needs no restatement: its contract is
Python's own json.dumps(value, ensure_ascii=False) and float.__repr__, which
the tests call directly.

Pinned by tests/test_text.py against the reference's own tests
(tests/api.rs, the pyjson tests in src/pyjson.rs:120-156, the tokenizer-level
cases of tests/checkpoint.rs:41-74) and by hand-computed budget cases.
"""
from __future__ import annotations

import json
import math

import numpy as np

OPTION_TOKENS = 48  # src/encode.rs:12
QTYPES = ("choice", "score", "noul")


class FrontEndError(ValueError):
    pass


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _is_number(v) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def dumps(v) -> str:
    """pyjson::dumps (src/pyjson.rs:7-49): Python's json.dumps(ensure_ascii=False)."""
    return json.dumps(v, ensure_ascii=False)


def state_from_value(v):
    """State::from_value (src/request.rs:41-47): ("t", text) or ("j", object/array)."""
    if isinstance(v, str):
        return ("t", v)
    if isinstance(v, (dict, list)):
        return ("j", v)
    return None


def render(state) -> str:
    """State::render (src/request.rs:51-56)."""
    return state[1] if state[0] == "t" else dumps(state[1])


def request_from_value(row, line: int) -> dict:
    """Request::from_value (src/request.rs:90-130)."""
    prefix = f"JSONL line {line}: "
    if not isinstance(row, dict):
        raise FrontEndError(prefix + "request must be a JSON object")
    state = state_from_value(row["state"]) if "state" in row else None
    question = row.get("question")
    if state is None or not isinstance(question, str):
        raise FrontEndError(prefix + "state must be text/JSON and question must be text")
    options = row.get("options")
    if not isinstance(options, list) or not all(isinstance(x, str) and x for x in options) \
            or not 2 <= len(options) <= 20:
        raise FrontEndError(prefix + "options must contain 2–20 nonempty rendered descriptions")
    qtype = "choice"
    if "type" in row:
        if row["type"] not in QTYPES:
            raise FrontEndError(prefix + "type must be choice, score, or noul")
        qtype = row["type"]
    if qtype == "noul" and len(options) != 2:
        raise FrontEndError(prefix + "noul options must be ordered [false, true]")
    if "target" in row:
        t = row["target"]
        if not (_is_int(t) and 0 <= t < len(options)):
            raise FrontEndError(prefix + "target must index the supplied option list")
    teacher = row.get("teacher_logits")
    if teacher is not None:
        def finite(x):
            try:
                return _is_number(x) and math.isfinite(float(x))
            except OverflowError:
                return False
        if not (isinstance(teacher, list) and len(teacher) == len(options) and all(finite(x) for x in teacher)):
            raise FrontEndError(prefix + "teacher logits must be finite and match option count/order")
    return dict(state=state, question=question, options=list(options), qtype=qtype)


def parse_rows(text: str) -> list:
    """parse_rows (src/engine.rs:298-307): JSONL, blank lines skipped, 1-based line numbers."""
    rows = []
    for i, line in enumerate(text.split("\n")):
        if line.endswith("\r"):
            line = line[:-1]
        if not line.strip():
            continue
        try:
            v = json.loads(line)
        except ValueError:
            raise FrontEndError(f"line {i + 1}: invalid JSON")
        rows.append(request_from_value(v, i + 1))
    return rows


def sequence(tokenize, special: dict, max_length: int, head_length: int, strict: bool, row: dict) -> dict:
    """Encoder::sequence (src/encode.rs:137-195).  tokenize(text) -> list of ids; special holds the
    mask token text and the mask/cls/sep ids."""
    state = render(row["state"])
    mask = special["mask_token"]
    if strict and any(mask in t for t in [state, row["question"], *row["options"]]):
        raise FrontEndError("Reserved model marker in request")
    clean = lambda t: t.replace(mask, " ")  # noqa: E731
    head = tokenize(f"{row['qtype']} question: {clean(row['question'])}")
    option_ids = [tokenize(" " + clean(x)) for x in row["options"]]
    if strict and any(len(x) > OPTION_TOKENS for x in option_ids):
        raise FrontEndError("Option exceeds 48-token model contract")
    options = [[special["mask"]] + list(x[:OPTION_TOKENS]) for x in option_ids]
    budget = head_length - sum(len(o) for o in options)
    if budget < 16:
        per_option = max((head_length - 16) // len(options), 4)
        options = [o[:per_option] for o in options]
        budget = head_length - sum(len(o) for o in options)
    if strict and (len(head) > budget or any(len(o) != len(x) + 1 for o, x in zip(options, option_ids))):
        raise FrontEndError("Question/options exceed lossless head budget")
    ids = [special["cls"]] + list(head[:min(len(head), max(budget, 8))]) + [special["sep"]]
    markers = []
    for o in options:
        markers.append(len(ids))
        ids += o
    ids.append(special["sep"])
    state_ids = tokenize(clean(state))
    room = max_length - len(ids) - 1
    if room < 1:
        raise FrontEndError("Question/options exceed sequence budget; shorten descriptions")
    if strict and len(state_ids) > room:
        raise FrontEndError("Game state exceeds lossless context budget")
    ids += list(state_ids[:room]) + [special["sep"]]
    return dict(ids=ids, markers=markers, qtype=row["qtype"], truncated=len(state_ids) > room,
                option_tokens=[len(x) for x in option_ids] if strict else [])


def argmax(values) -> int:
    """argmax (src/request.rs:164-172): first index of the maximum."""
    best = 0
    for i, v in enumerate(values):
        if v > values[best]:
            best = i
    return best


def display_probabilities(values) -> list:
    """display_probabilities (src/request.rs:150-161)."""
    if len(values) == 0:
        return []
    w = argmax(values)
    if values[w] > 0.95 and all(i == w or v < 0.045 for i, v in enumerate(values)):
        return [1.0 if i == w else 0.0 for i in range(len(values))]
    visible = [v if v >= 0.01 else 0.0 for v in values]
    total = 0.0
    for v in visible:
        total += v
    return [v / total for v in visible]


def softmax_f32(values) -> np.ndarray:
    """softmax_f32 (src/request.rs:175-180), float32 arithmetic throughout."""
    z = np.asarray(values, dtype=np.float32)
    e = np.exp(z - np.float32(z.max()), dtype=np.float32)
    total = np.float32(0)
    for x in e:
        total = np.float32(total + x)
    return (e / total).astype(np.float32)


def predict(logits, probabilities: bool) -> list:
    """Engine::predict (src/engine.rs:247-258)."""
    out = []
    for z in logits:
        p = {"index": argmax(list(z))}
        if probabilities:
            p["probabilities"] = display_probabilities([float(x) for x in softmax_f32(z)])
        out.append(p)
    return out


def typed_rows(state, questions):
    """typed_rows (src/typed.rs:65-112) -> (rows, [(id, qtype, keys)])."""
    if not isinstance(questions, dict) or not questions:
        raise FrontEndError("questions must be a nonempty mapping")
    rows, meta = [], []
    for qid, q in questions.items():
        if not isinstance(q, dict) or not qid:
            raise FrontEndError("Questions require nonempty string IDs and question objects")
        kind = q.get("type") if q.get("type") in QTYPES else None
        criteria = q.get("criteria")
        if kind == "choice":
            if not isinstance(criteria, dict) or not all(criteria.keys()):
                raise FrontEndError("Choice criteria must map nonempty IDs to descriptions")
            keys, labels = list(criteria.keys()), list(criteria.values())
        elif kind == "score":
            if not isinstance(criteria, list):
                raise FrontEndError("Score requires an ordered rubric")
            keys, labels = [str(i) for i in range(len(criteria))], list(criteria)
        elif kind == "noul":
            keys = ["false", "true"]
            if criteria is None:
                labels = ["false", "true"]
            elif isinstance(criteria, dict) and len(criteria) == 2 and "false" in criteria and "true" in criteria:
                labels = [criteria["false"], criteria["true"]]
            else:
                raise FrontEndError("Noul criteria must map false and true to descriptions")
        else:
            raise FrontEndError("Unsupported question type")
        row = {"state": state[1], "question": q.get("instructions"), "type": kind, "options": labels}
        rows.append(request_from_value(row, len(rows) + 1))
        meta.append((qid, kind, keys))
    return rows, meta


def answers_from_logits(meta, scores) -> dict:
    """answers_from_logits + answers_to_json (src/typed.rs:37-62, 115-131), float64 softmax."""
    if len(scores) != len(meta):
        raise FrontEndError("Model returned an incorrect answer count")
    answers = {}
    for (qid, kind, keys), z in zip(meta, scores):
        z = [float(np.float32(v)) for v in z]
        if len(z) != len(keys) or not all(math.isfinite(v) for v in z):
            raise FrontEndError("Invalid model scores")
        mx = max(z)
        e = [math.exp(v - mx) for v in z]
        total = 0.0
        for x in e:
            total += x
        p = [x / total for x in e]
        a = {"type": kind, "probabilities": dict(zip(keys, p))}
        if kind == "choice":
            a["choice"] = keys[argmax(p)]
        elif kind == "score":
            s = 0.0
            for i, x in enumerate(p):
                s += i * x
            a["score"] = s
        else:
            a["noul"] = p[1]
        if kind != "noul":
            a["max_probability"] = max(p)
        answers[qid] = a
    return {"answers": answers}


def confident_winner(scores, best: int) -> bool:
    """Router::confident_winner (src/router.rs:132-142)."""
    s = [float(np.float32(x)) for x in scores]
    runner_up = max((v for i, v in enumerate(s) if i != best), default=-math.inf)
    if runner_up - s[best] >= math.log(0.045 / 0.95):
        return False
    total = 0.0
    for v in s:
        total += math.exp(v - s[best])
    return 1.0 / total > 0.95 and math.exp(runner_up - s[best]) / total < 0.045


def route_many(logits_fn, rows, width=20, survivors=2, batch_size=16, max_options=4096, cache=None) -> list:
    """Router::route_many + score (src/router.rs:88-210); rows are dicts with state (JSON value), question,
    options and type; logits_fn(list of rows) -> list of logit lists; cache: dict or None (unbounded)."""
    for r in rows:
        n = len(r["options"])
        if not 2 <= n <= max_options:
            raise FrontEndError(f"Expected 2–{max_options} options")
        if any(not o for o in r["options"]):
            raise FrontEndError("Options must be nonempty strings")
        if r.get("type", "choice") == "noul" and n != 2:
            raise FrontEndError("noul requires [false, true]")
        if r.get("type", "choice") != "choice" and n > width:
            raise FrontEndError("Hierarchical routing supports choice decisions only")

    def key(r):
        return "\0".join([dumps(r["state"]), r["question"], r.get("type", "choice"), "\0".join(r["options"])])

    def score(jobs):
        values, missing, index, hits = [None] * len(jobs), [], {}, 0
        for i, r in enumerate(jobs):
            k = key(r)
            if cache is not None and k in cache:
                values[i] = cache[k]
                hits += 1
                continue
            if k in index:
                missing[index[k]][1].append(i)
                hits += 1
            else:
                index[k] = len(missing)
                missing.append((k, [i]))
        for c in range(0, len(missing), batch_size):
            chunk = missing[c:c + batch_size]
            out = logits_fn([jobs[idx[0]] for _, idx in chunk])
            if len(out) != len(chunk):
                raise FrontEndError("Engine returned the wrong number of rows")
            for (k, idx), z in zip(chunk, out):
                z = [float(np.float32(v)) for v in z]
                if len(z) != len(jobs[idx[0]]["options"]) or not all(math.isfinite(v) for v in z):
                    raise FrontEndError("Engine logits must be finite and match option count")
                for i in idx:
                    values[i] = z
                if cache is not None:
                    cache[k] = z
        return values, len(missing), hits

    candidates = [list(range(len(r["options"]))) for r in rows]
    results, rounds = [None] * len(rows), [0] * len(rows)
    model_rows = hits = 0
    while any(r is None for r in results):
        jobs, layout = [], []
        for i, r in enumerate(rows):
            if results[i] is not None:
                continue
            rounds[i] += 1
            current, candidates[i] = candidates[i], []
            last = len(current) <= width
            for c in range(0, len(current), width):
                group = current[c:c + width]
                if len(group) == 1:
                    candidates[i] += group
                    continue
                jobs.append(dict(r, options=[r["options"][k] for k in group]))
                layout.append((i, group, last))
        scored, used, cached = score(jobs)
        model_rows += used
        hits += cached
        for (i, group, last), s in zip(layout, scored):
            best = argmax(s)
            if last:
                mx = max(s)
                w = [math.exp(x - mx) for x in s]
                total = 0.0
                for x in w:
                    total += x
                hier = len(rows[i]["options"]) > width
                results[i] = dict(index=group[best], candidates=group,
                                  probabilities=display_probabilities([x / total for x in w]), rounds=rounds[i],
                                  hierarchical=hier, probability_scope="final_candidates" if hier else "all_options")
            elif confident_winner(s, best):
                candidates[i].append(group[best])
            else:
                remaining, chosen = list(range(len(group))), []
                for _ in range(min(survivors, len(group))):
                    a = argmax([s[k] for k in remaining])
                    chosen.append(group[remaining.pop(a)])
                candidates[i] += sorted(chosen)
    for r in results:
        r["model_rows"], r["cache_hits"] = model_rows, hits
    return results
