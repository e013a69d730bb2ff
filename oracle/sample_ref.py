"""Next-token sampling, restated from SwiftletSession.sample
(SwiftletSession.swift:226-273) — TEST INFRASTRUCTURE ONLY (tests/ import it
as the checker of swq_sample; the product path never does).

The reference draws its uniform number with Float.random; here it is the
argument u in [0, 1), so a draw is reproducible.  Everything else follows
the Swift code step by step in float32: penalties (:227-236), greedy first
maximum (:238-242), the partial top-k candidate scan (:244-252), the sort
by logit (:253; Swift's sort is not stable, so the order of exactly equal
logits is unspecified there; here they keep the lower id first, the order
the device uses), p = exp((l - l0) / T) (:254), the top-p cut (:256-265) and
the subtraction walk (:266-271)."""

from __future__ import annotations

import numpy as np

f32 = np.float32


def penalise(logits, seen: dict[int, int], banned, presence: float, frequency: float) -> np.ndarray:
    """SwiftletSession.swift:227-236: banned ids to -inf, then the presence
    and frequency penalties of the seen tokens."""
    lg = np.array(logits, dtype=f32, copy=True)
    for t in banned:
        lg[t] = -np.inf
    if presence != 0 or frequency != 0:
        for t, n in seen.items():
            lg[t] = f32(lg[t] - (f32(presence) + f32(frequency) * f32(n)))
    return lg


def sample(logits, temperature: float, top_k: int, top_p: float, presence: float = 0.0,
           frequency: float = 0.0, seen: dict[int, int] | None = None, banned=(), u: float = 0.0) -> int:
    lg = penalise(logits, seen or {}, banned, presence, frequency)
    vocab = lg.shape[0]
    if temperature <= 0:
        best = 0
        for v in range(1, vocab):
            if lg[v] > lg[best]:
                best = v
        return best
    k = max(1, min(top_k, vocab))
    cand = list(range(k))
    min_pos = 0
    for i in range(1, k):
        if lg[cand[i]] < lg[cand[min_pos]]:
            min_pos = i
    # the scan of :248-252, vectorised: only logits above the running minimum matter
    for v in np.nonzero(lg[k:] > np.min(lg[:k]))[0] + k:
        v = int(v)
        if lg[v] > lg[cand[min_pos]]:
            cand[min_pos] = v
            min_pos = 0
            for i in range(1, k):
                if lg[cand[i]] < lg[cand[min_pos]]:
                    min_pos = i
    top = sorted(((c, lg[c]) for c in cand), key=lambda p: (-float(p[1]), p[0]))
    t = f32(temperature)
    probs = [f32(np.exp(f32(f32(l - top[0][1]) / t))) for _, l in top]
    s = f32(0)
    for p in probs:
        s = f32(s + p)
    if top_p < 1:
        cum = f32(0)
        cut = len(probs)
        for i, p in enumerate(probs):
            cum = f32(cum + f32(p / s))
            if cum >= f32(top_p):
                cut = i + 1
                break
        top, probs = top[:cut], probs[:cut]
        s = f32(0)
        for p in probs:
            s = f32(s + p)
    r = f32(f32(u) * s)
    for i, p in enumerate(probs):
        r = f32(r - p)
        if r <= 0:
            return top[i][0]
    return top[0][0]
