"""Parity report of one backend's option logits against another's, per row.

The reference's `julia1 check` compares its logits with a reference dump row
by row: argmax agreement (first-max rule, src/request.rs:164-172) and
max/mean |Δlogit| over all options (src/bin/julia1.rs:197-237).  This adds
what a random-weights comparison needs to be read correctly:

- max |Δsoftmax| with the f64 softmax of the typed answers
  (src/typed.rs:115-131);
- the distribution of the reference row's top-2 logit gap, and how many rows
  have a gap below the observed max |Δlogit| (on those, argmax agreement is
  not decided by the backend's accuracy);
- argmax agreement restricted to rows whose gap exceeds twice max |Δlogit|,
  where a disagreement is a real divergence, not a near-tie.
"""
from __future__ import annotations

import numpy as np

# top-2 gap histogram edges (logit units)
GAP_EDGES = (0.0, 1e-3, 3e-3, 1e-2, 3e-2, 1e-1, 3e-1, float("inf"))


def argmax_first(v) -> int:
    """Index of the first maximum (src/request.rs:164-172); -1 for an empty row."""
    v = np.asarray(v)
    return int(np.argmax(v)) if v.size else -1


def softmax64(z) -> np.ndarray:
    z = np.asarray(z, dtype=np.float64)
    e = np.exp(z - z.max())
    return e / e.sum()


def top2_gap(v) -> float:
    s = np.sort(np.asarray(v, dtype=np.float64))
    return float(s[-1] - s[-2])


def report(rows_got, rows_ref) -> dict:
    """rows_got / rows_ref: per-row arrays of option logits (same shapes).  Returns a JSON-able dict."""
    if len(rows_got) != len(rows_ref):
        raise ValueError("row count mismatch")
    dl_max, dl_sum, n_opt, dp_max = 0.0, 0.0, 0, 0.0
    agree, rows, gaps, pairs = 0, 0, [], []
    for a, b in zip(rows_got, rows_ref):
        a = np.asarray(a, dtype=np.float64)
        b = np.asarray(b, dtype=np.float64)
        if a.shape != b.shape:
            raise ValueError("option count mismatch")
        if not a.size:
            continue
        d = np.abs(a - b)
        dl_max = max(dl_max, float(d.max()))
        dl_sum += float(d.sum())
        n_opt += a.size
        dp_max = max(dp_max, float(np.abs(softmax64(a) - softmax64(b)).max()))
        rows += 1
        same = argmax_first(a) == argmax_first(b)
        agree += int(same)
        if b.size > 1:
            gaps.append(top2_gap(b))
            pairs.append((gaps[-1], same))
    gaps_arr = np.array(gaps)
    hist = np.histogram(gaps_arr, bins=np.array(GAP_EDGES))[0] if gaps else np.zeros(len(GAP_EDGES) - 1, int)
    robust = [same for gap, same in pairs if gap > 2 * dl_max]
    return dict(rows=rows, options=n_opt, max_dlogit=dl_max, mean_dlogit=dl_sum / max(n_opt, 1),
                max_dsoftmax=dp_max, argmax_agree=agree,
                min_gap=float(gaps_arr.min()) if gaps else None,
                gap_hist=dict(edges=[e if np.isfinite(e) else "inf" for e in GAP_EDGES], counts=[int(c) for c in hist]),
                rows_gap_below_dlogit=int((gaps_arr < dl_max).sum()) if gaps else 0,
                robust_rows=len(robust), robust_agree=int(sum(robust)))


def check_gates(s: dict, dlogit=2e-2, dsoftmax=1e-2, argmax_frac=0.999) -> None:
    """The north-star gates: |Δlogit| <= 2e-2, |Δsoftmax| <= 1e-2, argmax agreement >= 99.9% of rows, and
    no disagreement on a row whose top-2 gap exceeds twice the max |Δlogit|."""
    assert s["max_dlogit"] <= dlogit, s
    assert s["max_dsoftmax"] <= dsoftmax, s
    assert s["argmax_agree"] >= argmax_frac * s["rows"] or s["argmax_agree"] == s["rows"], s
    assert s["robust_agree"] == s["robust_rows"], s
