"""Next-token sampling on the device (swq_sample) against the oracle
(oracle/sample_ref.py, SwiftletSession.sample, SwiftletSession.swift:226-273):
the same token, bit for bit, for the same logits, options, penalties and
uniform number u — greedy, Qwen's default settings (T 0.7, top-k 20, top-p
0.8, presence 1.5, frequency 0.5), no cut, the widest top-k (64), exact
ties, banned ids, at the 35B vocabulary (248,320) and small ones; a call
without penalties after one with them matches the oracle without (nothing
of a call's penalties stays in the workspace).  Every logit equal is the
selection's widest case (keys order by id alone, so the last workgroup
ranks ~k^2 candidates: 4,033 at top-k 64); the tokens still match."""

import numpy as np
import pytest

from oracle import sample_ref as S
from swiftlet_amd.engine import HipEngine

pytestmark = pytest.mark.gpu

QWEN = dict(temperature=0.7, top_k=20, top_p=0.8, presence=1.5, frequency=0.5)


@pytest.fixture(scope="module")
def eng():
    return HipEngine()


@pytest.mark.parametrize("vocab", [248320, 1000, 128, 65])
def test_sample_matches_oracle(eng, vocab):
    import torch
    rng = np.random.default_rng(vocab)
    ws = eng.new_sample_workspace(vocab)
    print(f"sample vocab {vocab}", flush=True)
    for trial in range(12):
        lg = (rng.standard_normal(vocab) * 2.5).astype(np.float32)
        if trial % 3 == 2:  # exact ties at the top
            top = int(np.argmax(lg))
            lg[rng.choice(vocab, 3, replace=False)] = lg[top]
        seen = {int(t): int(rng.integers(1, 4)) for t in rng.choice(vocab, min(40, vocab // 2), replace=False)}
        banned = [int(t) for t in rng.choice(vocab, 3, replace=False)]
        opts = [dict(temperature=0.0, top_k=20, top_p=0.8, presence=0.0, frequency=0.0), QWEN,
                dict(temperature=1.0, top_k=64, top_p=1.0, presence=0.3, frequency=0.0),
                dict(temperature=0.5, top_k=1, top_p=0.9, presence=0.0, frequency=0.0)]
        d = torch.from_numpy(lg).cuda()
        for o in opts:
            for u in (0.0, 0.37, 0.999):
                want = S.sample(lg, o["temperature"], o["top_k"], o["top_p"], o["presence"], o["frequency"],
                                seen, banned, u)
                got = eng.sample(d, o["temperature"], o["top_k"], o["top_p"], o["presence"], o["frequency"],
                                 seen, banned, u, ws=ws)
                assert got == want, (vocab, trial, o, u)
        # no penalties now
        got = eng.sample(d, 0.7, 20, 0.8, u=0.5, ws=ws)
        assert got == S.sample(lg, 0.7, 20, 0.8, u=0.5), (vocab, trial)


@pytest.mark.parametrize("vocab", [248320, 3000])
def test_sample_all_logits_equal(eng, vocab):
    import torch
    rng = np.random.default_rng(vocab + 1)
    ws = eng.new_sample_workspace(vocab)
    print(f"equal logits, vocab {vocab}", flush=True)
    lg = np.zeros(vocab, dtype=np.float32)
    d = torch.from_numpy(lg).cuda()
    seen = {int(t): 1 for t in rng.choice(40, 6, replace=False)}  # some of the lowest ids
    for o in [dict(temperature=0.0, top_k=20, top_p=0.8, presence=0.0, frequency=0.0), QWEN,
              dict(temperature=1.0, top_k=64, top_p=1.0, presence=0.0, frequency=0.0),
              dict(temperature=0.9, top_k=64, top_p=0.5, presence=0.7, frequency=0.2)]:
        for u in (0.0, 0.37, 0.999):
            want = S.sample(lg, o["temperature"], o["top_k"], o["top_p"], o["presence"], o["frequency"], seen, [3], u)
            got = eng.sample(d, o["temperature"], o["top_k"], o["top_p"], o["presence"], o["frequency"], seen, [3], u,
                             ws=ws)
            assert got == want, (vocab, o, u)
