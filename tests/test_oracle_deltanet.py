"""The DeltaNet oracle (oracle/deltanet_ref.py, QwenCPUModel.deltaNetForward,
QwenCPUModel.swift:371-496) beyond the mlx fixtures that already run the tiny
model through it (tests/test_oracle_fixtures.py):

- carrying (conv tail, state) token by token equals the whole-sequence call
  (the reference's DecodeState continuation, :420-435, :452-479);
- closed forms of the recurrence from a fresh state with an identity conv:
  after one token o = beta1 (k1.q1) v1, after a second token whose key is
  orthogonal to the first o = g2 beta1 (k1.q2) v1 + beta2 (k2.q2) v2, with
  q and k normalised and scaled by 1/dk and 1/sqrt(dk) and the gated norm on
  top — computed here in float64 from those formulas, not from the
  oracle's code;
- a planted mistake (q and k exchanged) fails the closed form."""

import numpy as np
import pytest

from oracle import deltanet_ref as D
from oracle.qwen_tiny import TinyQwen
from tests.test_oracle_fixtures import G


def _random_params(rng, nk, nv, dk, dv, K):
    convD = 2 * nk * dk + nv * dv
    return dict(conv_w=(rng.standard_normal((convD, K)) * 0.5).astype(np.float32),
                a_log=(rng.standard_normal(nv) * 0.5).astype(np.float32),
                dt_bias=(rng.standard_normal(nv) * 0.5).astype(np.float32),
                norm_w=(1 + 0.2 * rng.standard_normal(dv)).astype(np.float32),
                nk=nk, nv=nv, dk=dk, dv=dv, eps=1e-6)


@pytest.mark.parametrize("shape", ["tiny", "35b"])
def test_token_by_token_equals_sequence(shape):
    rng = np.random.default_rng(3)
    if shape == "tiny":
        prm = TinyQwen(G / "tiny-model-q4").deltanet_params(0)
        S = 9
    else:
        prm = _random_params(rng, 16, 32, 128, 128, 4)
        S = 4
    convD = 2 * prm["nk"] * prm["dk"] + prm["nv"] * prm["dv"]
    mixed = rng.standard_normal((S, convD)).astype(np.float32)
    z = rng.standard_normal((S, prm["nv"] * prm["dv"])).astype(np.float32)
    b = rng.standard_normal((S, prm["nv"])).astype(np.float32)
    a = rng.standard_normal((S, prm["nv"])).astype(np.float32)
    y_all, tail_all, st_all = D.deltanet_core(mixed, z, b, a, **prm)
    tail = st = None
    for s in range(S):
        y, tail, st = D.deltanet_core(mixed[s:s + 1], z[s:s + 1], b[s:s + 1], a[s:s + 1], conv_tail=tail,
                                      state=st, **prm)
        np.testing.assert_allclose(y[0], y_all[s], rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(tail, tail_all)
    np.testing.assert_allclose(st, st_all, rtol=1e-6, atol=1e-7)


def _closed_form_case(swap_qk=False):
    """Two tokens, nk = 1, nv = 2, dk = dv = 4, identity conv (K = 4, weight 1
    on the newest row), keys with disjoint supports."""
    nk, nv, dk, dv, K = 1, 2, 4, 4, 4
    conv_w = np.zeros((2 * dk + nv * dv, K), np.float32)
    conv_w[:, K - 1] = 1.0
    prm = dict(conv_w=conv_w, a_log=np.array([0.3, -0.4], np.float32), dt_bias=np.array([0.1, 0.2], np.float32),
               norm_w=np.array([1.0, 0.5, 2.0, 1.5], np.float32), nk=nk, nv=nv, dk=dk, dv=dv, eps=1e-6)
    q = np.array([[0.9, 0.3, 0.0, 1.2], [0.5, 1.1, 0.7, 0.0]], np.float32)
    k = np.array([[1.3, 0.0, 0.0, 0.8], [0.0, 0.6, 1.7, 0.0]], np.float32)  # disjoint: silu(0) = 0
    v = np.array([[[0.4, -1.0, 2.0, 0.3], [1.5, 0.2, -0.7, 0.9]],
                  [[-0.6, 0.8, 0.1, 1.1], [0.3, -1.2, 0.5, 0.4]]], np.float32)
    z = np.array([[0.5, -0.3, 1.0, 0.2, 0.7, 0.1, -0.9, 1.3], [1.1, 0.4, -0.2, 0.6, -0.5, 0.9, 0.3, 0.8]],
                 np.float32)
    b = np.array([[0.2, -0.5], [1.0, 0.4]], np.float32)
    a = np.array([[-0.3, 0.6], [0.5, -1.0]], np.float32)
    qq, kk = (k, q) if swap_qk else (q, k)
    mixed = np.concatenate([qq, kk, v.reshape(2, nv * dv)], axis=1)
    y, _, _ = D.deltanet_core(mixed, z, b, a, **prm)

    # the formulas, in float64
    silu = lambda x: x / (1 + np.exp(-x))
    sig = lambda x: 1 / (1 + np.exp(-x))
    f = lambda x: np.asarray(x, np.float64)
    qh = [silu(f(q[t])) / np.sqrt(np.mean(silu(f(q[t])) ** 2) + 1e-6) / dk for t in range(2)]
    kh = [silu(f(k[t])) / np.sqrt(np.mean(silu(f(k[t])) ** 2) + 1e-6) / np.sqrt(dk) for t in range(2)]
    vs = silu(f(v))
    beta = sig(f(b))
    sp = np.log1p(np.exp(f(a) + f(prm["dt_bias"])))
    g = np.exp(-np.exp(f(prm["a_log"])) * sp)
    assert abs(kh[0] @ kh[1]) == 0.0
    want = np.zeros((2, nv * dv))
    for hv in range(nv):
        o1 = beta[0, hv] * (kh[0] @ qh[0]) * vs[0, hv]
        o2 = g[1, hv] * beta[0, hv] * (kh[0] @ qh[1]) * vs[0, hv] + beta[1, hv] * (kh[1] @ qh[1]) * vs[1, hv]
        for t, o in enumerate((o1, o2)):
            n = o / np.sqrt(np.mean(o ** 2) + 1e-6) * f(prm["norm_w"])
            want[t, hv * dv:(hv + 1) * dv] = n * silu(f(z[t, hv * dv:(hv + 1) * dv]))
    return y, want


def test_two_step_closed_form():
    y, want = _closed_form_case()
    np.testing.assert_allclose(y, want, rtol=2e-5, atol=1e-6)


def test_planted_mistake_fails_closed_form():
    y, want = _closed_form_case(swap_qk=True)
    assert not np.allclose(y, want, rtol=2e-5, atol=1e-6)


def test_deinterleave_places_every_channel():
    """Each value of the fused projections lands at its [q|k|v], z, b, a slot
    (QwenCPUModel.swift:386-410), checked by tagging values with their source."""
    nk, nv, dk, dv = 2, 6, 3, 2
    rep = nv // nk
    chunk = 2 * dk + 2 * rep * dv
    qkvz = np.arange(nk * chunk, dtype=np.float32)[None]
    ba = 1000 + np.arange(2 * nv, dtype=np.float32)[None]
    mixed, z, b, a = D.deinterleave(qkvz, ba, nk, nv, dk, dv)
    for hk in range(nk):
        base = hk * chunk
        assert mixed[0, hk * dk:(hk + 1) * dk].tolist() == list(range(base, base + dk))
        assert mixed[0, nk * dk + hk * dk:nk * dk + (hk + 1) * dk].tolist() == list(range(base + dk, base + 2 * dk))
        for ri in range(rep):
            hv = hk * rep + ri
            vs = base + 2 * dk + ri * dv
            assert mixed[0, 2 * nk * dk + hv * dv:2 * nk * dk + (hv + 1) * dv].tolist() == list(range(vs, vs + dv))
            zs = base + 2 * dk + rep * dv + ri * dv
            assert z[0, hv * dv:(hv + 1) * dv].tolist() == list(range(zs, zs + dv))
            assert b[0, hv] == 1000 + hk * 2 * rep + ri and a[0, hv] == 1000 + hk * 2 * rep + rep + ri
