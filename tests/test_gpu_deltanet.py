"""The gated DeltaNet decode step on the device (swq_deltanet_step) against
the oracle (oracle/deltanet_ref.py, QwenCPUModel.deltaNetForward,
QwenCPUModel.swift:371-496).

Bar: fp32 throughout, sums in another order than the reference's serial
loops — every token's output within 1e-5 of the oracle's (max abs error
over max abs value), and the recurrent state after the run within 1e-5 the
same way; the conv ring holds exactly the inputs (bit-exact).  Cases: the
tiny model's DeltaNet parameters (interleaved layout, dk 8), both layouts at
the 35B / 80B shapes (nk 16, nv 32, dk = dv = 128, K 4) from a fresh session
and from a random state at a position past the ring's wrap, and the tiny
4-bit qwen3_next model with every DeltaNet layer (projections, step,
out_proj), post-attention norm, MoE block and lm_head on the device
(attention on the host) against mlx's logits (2e-3,
FixtureForwardTests.swift:94-95) and greedy ids; the tiny f32 qwen3_5 model
(split projections, nested config, "language_model." names) with every
DeltaNet step on the device, its parameters read through the library's
checkpoint loader, against mlx's per-layer outputs and greedy ids
(FixtureForwardTests.swift:55-82).  That model's weights are f32: its
projections, attention and MoE blocks (quantized-only on the device) run in
the oracle."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import deltanet_ref as D
from oracle.qwen_tiny import TinyQwen
from swiftlet_amd._lib import SWQ_DELTA_INTERLEAVED, SWQ_DELTA_SPLIT
from swiftlet_amd.deltanet import DeltaNetGPU, deltanet_from_checkpoint

pytestmark = pytest.mark.gpu

G = Path(__file__).resolve().parent / "golden" / "swiftlet_fixtures"


def _rel(got, want):
    return float(np.abs(np.asarray(got) - want).max() / max(np.abs(want).max(), 1e-30))


def _interleave(mixed, z, b, a, nk, nv, dk, dv):
    """Inverse of the oracle's deinterleave: the fused projections' order."""
    rep = nv // nk
    keyD = nk * dk
    S = mixed.shape[0]
    chunk = 2 * dk + 2 * rep * dv
    qkvz = np.zeros((S, nk * chunk), np.float32)
    ba = np.zeros((S, 2 * nv), np.float32)
    for hk in range(nk):
        c = hk * chunk
        qkvz[:, c:c + dk] = mixed[:, hk * dk:(hk + 1) * dk]
        qkvz[:, c + dk:c + 2 * dk] = mixed[:, keyD + hk * dk:keyD + (hk + 1) * dk]
        for ri in range(rep):
            hv = hk * rep + ri
            qkvz[:, c + 2 * dk + ri * dv:c + 2 * dk + (ri + 1) * dv] = mixed[:, 2 * keyD + hv * dv:2 * keyD + (hv + 1) * dv]
            o = c + 2 * dk + rep * dv + ri * dv
            qkvz[:, o:o + dv] = z[:, hv * dv:(hv + 1) * dv]
        ba[:, hk * 2 * rep:hk * 2 * rep + rep] = b[:, hk * rep:(hk + 1) * rep]
        ba[:, hk * 2 * rep + rep:(hk + 1) * 2 * rep] = a[:, hk * rep:(hk + 1) * rep]
    return qkvz, ba


def _run(prm, K, layout, S, seed, start=None):
    """S tokens through the device step and the oracle; returns the worst
    per-token output error and the final-state error."""
    import torch
    rng = np.random.default_rng(seed)
    nk, nv, dk, dv = prm["nk"], prm["nv"], prm["dk"], prm["dv"]
    convD, valD = 2 * nk * dk + nv * dv, nv * dv
    blk = DeltaNetGPU(nk, nv, dk, dv, K, layout, prm["eps"], prm["conv_w"], prm["a_log"], prm["dt_bias"],
                      prm["norm_w"])
    state = blk.new_state()
    ring, rec = blk.state_views(state)
    pos0, tail, st = 0, None, None
    if start is not None:  # a session in progress: random history and state
        pos0 = start
        ring.copy_(torch.from_numpy((rng.standard_normal((K, convD))).astype(np.float32)))
        rec.copy_(torch.from_numpy((rng.standard_normal((nv, dv, dk)) * 0.05).astype(np.float32)))
        r_h = ring.cpu().numpy()
        tail = np.stack([r_h[(pos0 - (K - 1) + j) % K] for j in range(K - 1)])
        st = rec.cpu().numpy().copy()
    mixed = rng.standard_normal((S, convD)).astype(np.float32)
    z = rng.standard_normal((S, valD)).astype(np.float32)
    b = rng.standard_normal((S, nv)).astype(np.float32)
    a = rng.standard_normal((S, nv)).astype(np.float32)
    if layout == SWQ_DELTA_SPLIT:
        qkvz, ba = np.concatenate([mixed, z], axis=1), np.concatenate([b, a], axis=1)
    else:
        qkvz, ba = _interleave(mixed, z, b, a, nk, nv, dk, dv)
    want, _, st_want = D.deltanet_core(mixed, z, b, a, conv_tail=tail, state=st, **prm)
    worst = 0.0
    for s in range(S):
        y = blk.step(torch.from_numpy(qkvz[s]).cuda(), torch.from_numpy(ba[s]).cuda(), state, pos0 + s)
        torch.cuda.synchronize()
        worst = max(worst, _rel(y.cpu().numpy(), want[s]))
    ring_h = ring.cpu().numpy()
    for s in range(max(0, S - K), S):  # the last K inputs sit in their slots
        assert np.array_equal(ring_h[(pos0 + s) % K], mixed[s])
    return worst, _rel(rec.cpu().numpy(), st_want)


def test_tiny_model_parameters():
    prm = TinyQwen(G / "tiny-model-q4").deltanet_params(0)
    err, st_err = _run(prm, 4, SWQ_DELTA_INTERLEAVED, S=11, seed=1)
    print(f"tiny: y {err:.2e}, state {st_err:.2e}", flush=True)
    assert err < 1e-5 and st_err < 1e-5


@pytest.mark.parametrize("layout", [SWQ_DELTA_SPLIT, SWQ_DELTA_INTERLEAVED], ids=["split", "interleaved"])
@pytest.mark.parametrize("start", [None, 37], ids=["fresh", "pos37"])
def test_real_shapes(layout, start):
    rng = np.random.default_rng(7)
    nk, nv, dk, dv, K = 16, 32, 128, 128, 4
    convD = 2 * nk * dk + nv * dv
    prm = dict(conv_w=(rng.standard_normal((convD, K)) * 0.5).astype(np.float32),
               a_log=(rng.standard_normal(nv) * 0.5).astype(np.float32),
               dt_bias=(rng.standard_normal(nv) * 0.5).astype(np.float32),
               norm_w=(1 + 0.2 * rng.standard_normal(dv)).astype(np.float32), nk=nk, nv=nv, dk=dk, dv=dv, eps=1e-6)
    print(f"layout {layout}, start {start}", flush=True)
    err, st_err = _run(prm, K, layout, S=6, seed=11, start=start)
    print(f"y {err:.2e}, state {st_err:.2e}", flush=True)
    assert err < 1e-5 and st_err < 1e-5


def test_tiny_q4_model_with_device_deltanet_matches_mlx():
    import torch
    from safetensors.numpy import load_file
    from swiftlet_amd.checkpoint import Checkpoint, moe_layer_from_checkpoint
    from swiftlet_amd.engine import HipEngine
    eng = HipEngine()
    d = G / "tiny-model-q4"
    cfg = json.loads((d / "config.json").read_text())
    ck, m = Checkpoint(d), TinyQwen(d)
    fx = load_file(str(G / "tiny_forward_q4.safetensors"))
    toks = fx["input_ids"][0]
    S = len(toks)
    emb = ck.gpu_linear("model.embed_tokens")
    hd = torch.cat([eng.dequantize(emb, int(t), 1) for t in toks])
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        xin = eng.rms_norm(hd.clone(), ck.load(p + "input_layernorm.weight"), m.eps)
        if m.is_linear(i):
            blk = deltanet_from_checkpoint(ck, i, cfg)
            state = blk.new_state()
            att = torch.stack([blk.forward_token(eng, xin[t], state, t) for t in range(S)])
        else:
            att = torch.from_numpy(m.attention_forward(xin.cpu().numpy(), i)).cuda()
        x2 = eng.rms_norm(hd, ck.load(p + "post_attention_layernorm.weight"), m.eps, residual=att.contiguous())
        moe_layer_from_checkpoint(ck, i, cfg).decode(x2, out=hd, accumulate=True)
        torch.cuda.synchronize()
    hn = eng.rms_norm(hd, ck.load("model.norm.weight"), m.eps)
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


def test_tiny_q35_model_with_device_deltanet_matches_mlx():
    import torch
    from safetensors.numpy import load_file
    from oracle.qwen_tiny import rms_norm, text_config
    from oracle import moe_ref as R
    from swiftlet_amd.checkpoint import Checkpoint
    d = G / "tiny-model-q35"
    c = text_config(json.loads((d / "config.json").read_text()))
    ck, m = Checkpoint(d), TinyQwen(d)
    assert c["split_layout"] and m.split
    fx = load_file(str(G / "tiny_forward_q35.safetensors"))
    toks = fx["input_ids"][0]
    S = len(toks)
    h = fx["embed"][0].astype(np.float32)
    for i in range(m.L):
        x = rms_norm(h, m.ck.tensor(f"model.layers.{i}.input_layernorm.weight"), m.eps)
        if m.is_linear(i):
            p = f"model.layers.{i}.linear_attn."
            # unprefixed names, resolved by the library to language_model.*
            blk = DeltaNetGPU(c["linear_num_key_heads"], c["linear_num_value_heads"], c["linear_key_head_dim"],
                              c["linear_value_head_dim"], c["linear_conv_kernel_dim"], SWQ_DELTA_SPLIT,
                              c["rms_norm_eps"], *(ck.load(p + n).float() for n in
                                                   ("conv1d.weight", "A_log", "dt_bias", "norm.weight")))
            mixed, z, b, a = m.deltanet_inputs(x, i)
            qkvz = torch.from_numpy(np.ascontiguousarray(np.concatenate([mixed, z], -1), np.float32)).cuda()
            ba = torch.from_numpy(np.ascontiguousarray(np.concatenate([b, a], -1), np.float32)).cuda()
            state = blk.new_state()
            y = torch.stack([blk.step(qkvz[t], ba[t], state, t) for t in range(S)])
            torch.cuda.synchronize()
            want, _, _ = D.deltanet_core(mixed, z, b, a, **m.deltanet_params(i))
            err = _rel(y.cpu().numpy(), want)
            print(f"q35 layer {i}: device DeltaNet vs oracle {err:.2e}", flush=True)
            assert err < 1e-5, (i, err)
            r = (y.cpu().numpy() @ m.ck.module_weight(p + "out_proj").T).astype(np.float32)
        else:
            r = m.attention_forward(x, i)
        h = (h + r).astype(np.float32)
        x2 = rms_norm(h, m.ck.tensor(f"model.layers.{i}.post_attention_layernorm.weight"), m.eps)
        h = (h + R.moe_forward(x2, m.moe_layer(i))[0]).astype(np.float32)
        diff = np.abs(h - fx[f"layer_{i:02d}"][0]).max()
        assert diff < 5e-4, (i, diff)  # chained from mlx's embedding (the oracle alone: 1.3e-5 at layer 7)
    logits = (rms_norm(h, m.final_norm, m.eps) @ m.lm_head.T).astype(np.float32)
    assert np.abs(logits - fx["logits"][0]).max() < 0.05
    want = json.loads((G / "tiny_forward_q35.json").read_text())["greedy_next_tokens"]
    assert np.argmax(logits, axis=-1).tolist() == want
