"""Gated GQA attention decode on the device (swq_attention_step) against the
oracle (oracle/attention_ref.py, QwenCPUModel.attentionForward + applyRope,
QwenCPUModel.swift:285-367).

Bar: fp32, sums and the softmax in another order (split positions, online
maxima) — each token's output within 1e-5 of the oracle's (max abs error
over max abs value); the cache rows the step appends within the same bound
(normalised, rotated k; v bit-exact).  Cases: the tiny model's attention
shape (hd 16, 4 heads over 2 kv heads, 4 rotary dims) token by token; the
35B / 80B shape (16 heads over 2 kv heads, hd 256, 64 rotary dims, theta
1e7) token by token across the 64-position split boundary, and single steps
at positions 1000 and 5000 over a random cache (several splits, chunks
above the minimum); and the reference's tiny 4-bit qwen3_next model run
entirely on the device — embedding rows, every norm, DeltaNet and attention
block (input norm fused into the projections' launch), MoE block and the
lm_head — against mlx's logits (2e-3,
FixtureForwardTests.swift:94-95) and greedy ids."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import attention_ref as A
from oracle.qwen_tiny import TinyQwen
from swiftlet_amd.attention import AttentionGPU, attention_from_checkpoint

pytestmark = pytest.mark.gpu

G = Path(__file__).resolve().parent / "golden" / "swiftlet_fixtures"
f32 = np.float32


def _rel(got, want):
    return float(np.abs(np.asarray(got) - want).max() / max(np.abs(want).max(), 1e-30))


def _block(prm, max_positions):
    return AttentionGPU(prm["H"], prm["KVH"], prm["hd"], prm["rot"], prm["theta"], prm["eps"], max_positions,
                        prm["q_norm_w"], prm["k_norm_w"])


def _sequence(prm, S, seed):
    import torch
    rng = np.random.default_rng(seed)
    H, KVH, hd = prm["H"], prm["KVH"], prm["hd"]
    blk = _block(prm, 256)
    cache, ws = blk.new_cache(), blk.new_workspace()
    q = rng.standard_normal((S, H * 2 * hd)).astype(f32)
    k = rng.standard_normal((S, KVH * hd)).astype(f32)
    v = rng.standard_normal((S, KVH * hd)).astype(f32)
    want, ck, cv = A.attention_core(q, k, v, **prm)
    worst = 0.0
    for s in range(S):
        out = blk.step(*(torch.from_numpy(t[s]).cuda() for t in (q, k, v)), cache, ws, s)
        torch.cuda.synchronize()
        worst = max(worst, _rel(out.cpu().numpy(), want[s]))
    gk, gv = blk.cache_views(cache)
    assert _rel(gk[:S].cpu().numpy(), ck) < 1e-5
    assert np.array_equal(gv[:S].cpu().numpy(), cv)
    return worst


def test_tiny_model_shape():
    err = _sequence(TinyQwen(G / "tiny-model-q4").attention_params(3), S=12, seed=2)
    print(f"tiny: {err:.2e}", flush=True)
    assert err < 1e-5


def _big_params(rng):
    return dict(q_norm_w=(1 + 0.2 * rng.standard_normal(256)).astype(f32),
                k_norm_w=(1 + 0.2 * rng.standard_normal(256)).astype(f32),
                H=16, KVH=2, hd=256, rot=64, theta=1e7, eps=1e-6)


def test_real_shape_sequence_across_splits():
    err = _sequence(_big_params(np.random.default_rng(3)), S=70, seed=4)
    print(f"35B shape, 70 tokens: {err:.2e}", flush=True)
    assert err < 1e-5


@pytest.mark.parametrize("position", [1000, 5000])
def test_real_shape_long_cache(position):
    import torch
    rng = np.random.default_rng(position)
    prm = _big_params(rng)
    blk = _block(prm, 6000)
    cache, ws = blk.new_cache(), blk.new_workspace()
    gk, gv = blk.cache_views(cache)
    # a cache of unit-scale rows, as normalised keys are
    ck = (rng.standard_normal((position, 2, 256)) * 0.5).astype(f32)
    cv = rng.standard_normal((position, 2, 256)).astype(f32)
    gk[:position].copy_(torch.from_numpy(ck))
    gv[:position].copy_(torch.from_numpy(cv))
    q = rng.standard_normal((1, 16 * 2 * 256)).astype(f32)
    k = rng.standard_normal((1, 2 * 256)).astype(f32)
    v = rng.standard_normal((1, 2 * 256)).astype(f32)
    want, _, _ = A.attention_core(q, k, v, cache_k=ck, cache_v=cv, **prm)
    print(f"position {position}", flush=True)
    out = blk.step(*(torch.from_numpy(t[0]).cuda() for t in (q, k, v)), cache, ws, position)
    torch.cuda.synchronize()
    err = _rel(out.cpu().numpy(), want[0])
    print(f"error {err:.2e}", flush=True)
    assert err < 1e-5


def test_tiny_q4_model_entirely_on_the_device_matches_mlx():
    import torch
    from safetensors.numpy import load_file
    from swiftlet_amd.checkpoint import Checkpoint, moe_layer_from_checkpoint
    from swiftlet_amd.deltanet import deltanet_from_checkpoint
    from swiftlet_amd.engine import HipEngine
    eng = HipEngine()
    d = G / "tiny-model-q4"
    cfg = json.loads((d / "config.json").read_text())
    ck = Checkpoint(d)
    eps = cfg["rms_norm_eps"]
    fx = load_file(str(G / "tiny_forward_q4.safetensors"))
    toks = fx["input_ids"][0]
    S = len(toks)
    emb = ck.gpu_linear("model.embed_tokens")
    hd = torch.cat([eng.dequantize(emb, int(t), 1) for t in toks])
    interval = cfg["full_attention_interval"]
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        w_in = ck.load(p + "input_layernorm.weight")  # the input norm runs inside the projections' launch
        if (i + 1) % interval != 0:
            blk = deltanet_from_checkpoint(ck, i, cfg)
            state = blk.new_state()
            att = torch.stack([blk.forward_token(eng, hd[t], state, t, norm_weight=w_in, eps=eps) for t in range(S)])
        else:
            blk = attention_from_checkpoint(ck, i, cfg, max_positions=64)
            cache, ws = blk.new_cache(), blk.new_workspace()
            att = torch.stack([blk.forward_token(eng, hd[t], cache, ws, t, norm_weight=w_in, eps=eps)
                               for t in range(S)])
        x2 = eng.rms_norm(hd, ck.load(p + "post_attention_layernorm.weight"), eps, residual=att.contiguous())
        moe_layer_from_checkpoint(ck, i, cfg).decode(x2, out=hd, accumulate=True)
        torch.cuda.synchronize()
    hn = eng.rms_norm(hd, ck.load("model.norm.weight"), eps)
    head = ck.gpu_linear("lm_head")
    logits = torch.empty((S, head.out_dim), dtype=torch.float32, device="cuda")
    for t in range(S):
        eng.encode_gemv(head, hn[t], logits[t])
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    diff = np.abs(got - fx["logits"][0]).max()
    print(f"max |logit - mlx| = {diff:.3g}", flush=True)
    assert diff < 2e-3, diff
    want = json.loads((G / "tiny_forward_q4.json").read_text())["greedy_next_tokens"]
    assert np.argmax(got, axis=-1).tolist() == want
