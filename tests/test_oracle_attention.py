"""The attention oracle (oracle/attention_ref.py, QwenCPUModel.
attentionForward + applyRope, QwenCPUModel.swift:285-367) beyond the mlx
fixtures that already run the tiny model through it:

- a cache carried token by token equals the whole-sequence call;
- closed forms: the first token attends only to itself (out = v *
  sigmoid(gate) whatever q and k are); with no rotary dims and equal keys
  every cached position gets the same weight (out = mean of the group's v
  rows * sigmoid(gate)), each query head reading its own kv head
  (head // (H / KVH)); RoPE preserves each rotated pair's norm and makes
  q.k depend only on the position difference;
- a planted mistake (the query and gate halves of q_proj swapped) fails the
  equal-keys form."""

import numpy as np
import pytest

from oracle import attention_ref as A
from oracle import moe_ref as R
from oracle.qwen_tiny import TinyQwen
from tests.test_oracle_fixtures import G

f32 = np.float32


def _params(H, KVH, hd, rot, rng, theta=1e7):
    return dict(q_norm_w=(1 + 0.2 * rng.standard_normal(hd)).astype(f32),
                k_norm_w=(1 + 0.2 * rng.standard_normal(hd)).astype(f32),
                H=H, KVH=KVH, hd=hd, rot=rot, theta=theta, eps=1e-6)


@pytest.mark.parametrize("shape", ["tiny", "35b"])
def test_cache_carry_equals_sequence(shape):
    rng = np.random.default_rng(4)
    prm = TinyQwen(G / "tiny-model-q4").attention_params(3) if shape == "tiny" else _params(16, 2, 256, 64, rng)
    H, KVH, hd = prm["H"], prm["KVH"], prm["hd"]
    S = 9
    q = rng.standard_normal((S, H * 2 * hd)).astype(f32)
    k = rng.standard_normal((S, KVH * hd)).astype(f32)
    v = rng.standard_normal((S, KVH * hd)).astype(f32)
    want, ck_all, cv_all = A.attention_core(q, k, v, **prm)
    ck = cv = None
    for s in range(S):
        out, ck, cv = A.attention_core(q[s:s + 1], k[s:s + 1], v[s:s + 1], cache_k=ck, cache_v=cv, **prm)
        np.testing.assert_allclose(out[0], want[s], rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(ck, ck_all)
    np.testing.assert_array_equal(cv, cv_all)


def test_first_token_attends_to_itself():
    rng = np.random.default_rng(5)
    prm = _params(8, 2, 64, 16, rng)
    q = rng.standard_normal((1, 8 * 2 * 64)).astype(f32)
    k = rng.standard_normal((1, 2 * 64)).astype(f32)
    v = rng.standard_normal((1, 2 * 64)).astype(f32)
    out, _, _ = A.attention_core(q, k, v, **prm)
    gate = q.reshape(8, 2, 64)[:, 1, :]
    want = np.stack([v.reshape(2, 64)[h // 4] for h in range(8)]) * R.sigmoid(gate)
    np.testing.assert_allclose(out.reshape(8, 64), want, rtol=1e-6)


def _equal_keys_case(mistake=False):
    rng = np.random.default_rng(6)
    H, KVH, hd, S = 8, 2, 32, 5
    prm = _params(H, KVH, hd, 0, rng)  # no rotary dims
    q = rng.standard_normal((S, H * 2 * hd)).astype(f32)
    k = np.tile(rng.standard_normal((1, KVH * hd)).astype(f32), (S, 1))
    v = rng.standard_normal((S, KVH * hd)).astype(f32)
    qin = q.reshape(S, H, 2, hd)[:, :, ::-1].reshape(S, -1) if mistake else q  # query and gate halves swapped
    out, _, _ = A.attention_core(np.ascontiguousarray(qin), k, v, **prm)
    vv = v.reshape(S, KVH, hd).astype(np.float64)
    gate = q.reshape(S, H, 2 * hd)[..., hd:]
    want = np.zeros((S, H, hd))
    for s in range(S):
        for h in range(H):
            want[s, h] = vv[:s + 1, h // (H // KVH)].mean(axis=0) * R.sigmoid(gate[s, h])
    return out.reshape(S, H, hd), want


def test_equal_keys_give_the_mean_of_the_group_values():
    out, want = _equal_keys_case()
    np.testing.assert_allclose(out, want, rtol=2e-5, atol=1e-6)


def test_planted_mistake_fails_equal_keys():
    out, want = _equal_keys_case(mistake=True)
    assert not np.allclose(out, want, rtol=2e-5, atol=1e-6)


def test_rope_norms_and_relative_positions():
    rng = np.random.default_rng(8)
    hd, rot = 64, 32
    x = rng.standard_normal((1, 3, hd)).astype(f32)
    y = A.apply_rope(x, [17], rot, 1e4)
    half = rot // 2
    n0 = x[..., :half] ** 2 + x[..., half:rot] ** 2
    n1 = y[..., :half] ** 2 + y[..., half:rot] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)
    np.testing.assert_array_equal(y[..., rot:], x[..., rot:])  # dims past rot untouched
    np.testing.assert_array_equal(A.apply_rope(x, [0], rot, 1e4), x)  # position 0: identity
    q = rng.standard_normal((1, 1, hd)).astype(f32)
    k = rng.standard_normal((1, 1, hd)).astype(f32)
    d1 = float(np.dot(A.apply_rope(q, [7], rot, 1e4)[0, 0], A.apply_rope(k, [3], rot, 1e4)[0, 0]))
    d2 = float(np.dot(A.apply_rope(q, [12], rot, 1e4)[0, 0], A.apply_rope(k, [8], rot, 1e4)[0, 0]))
    assert abs(d1 - d2) < 1e-4 * max(1.0, abs(d1))
