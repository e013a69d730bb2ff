"""The layer tail on the device: the attention branch's residual add and the
post-attention RMSNorm (swq_rmsnorm, QwenCPUModel.swift:47-59, :276-277;
Kernels.metal.txt:425-452), then the MoE step adding into the residual
stream (swq_moe_decode with SWQ_MOE_ACCUMULATE, :278-279).

Bar: h after the residual add is bit-identical to the oracle's (the same one
addition); the normalised rows are within 2e-6 relative of the oracle's
(fp32 sums in another order); bf16 outputs are the round-to-nearest-even of
values within that bound.  End to end, the reference's tiny 4-bit qwen3_next
model (tests/golden/swiftlet_fixtures, mlx's own quantized weights and
outputs) runs with every post-attention norm, MoE block, residual add, the
final norm and the lm_head on the device (attention and DeltaNet by the
oracle on the host): its logits match mlx's within the oracle's own bar
(2e-3, FixtureForwardTests.swift:94-95) and its greedy tokens exactly."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import moe_ref as R
from oracle.qwen_tiny import TinyQwen, rms_norm
from swiftlet_amd import _lib
from swiftlet_amd.engine import GPULinear, HipEngine
from swiftlet_amd.moe import MoELayerGPU

pytestmark = pytest.mark.gpu

G = Path(__file__).resolve().parent / "golden" / "swiftlet_fixtures"
EPS = 1e-6


@pytest.fixture(scope="module")
def eng():
    return HipEngine()


@pytest.mark.parametrize("rows,dim,wdt,residual", [
    (1, 2048, "f32", True), (5, 2048, "bf16", True), (3, 64, "f32", False), (2, 1000, "f16", True),
    (1, 4096, None, False),
])
def test_rmsnorm_matches_oracle(eng, rows, dim, wdt, residual):
    import torch
    rng = np.random.default_rng(rows * 7919 + dim)
    h = rng.standard_normal((rows, dim)).astype(np.float32) * 3.0
    r = rng.standard_normal((rows, dim)).astype(np.float32) if residual else None
    w = (rng.standard_normal(dim) * 0.5 + 1.0).astype(np.float32)
    tw = None
    if wdt is not None:
        tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[wdt]
        tw = torch.from_numpy(w).to(tdt).cuda()
        w = tw.float().cpu().numpy()  # the weight as the device holds it
    hd = torch.from_numpy(h).cuda()
    rd = torch.from_numpy(r).cuda() if residual else None
    out = eng.rms_norm(hd, tw, EPS, residual=rd)
    out16 = eng.rms_norm(hd.clone(), tw, EPS, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    h_ref = (h + r).astype(np.float32) if residual else h
    x_ref = rms_norm(h_ref, w if wdt is not None else None, EPS)
    assert np.array_equal(hd.cpu().numpy(), h_ref)
    got = out.cpu().numpy()
    rel = np.abs(got - x_ref).max() / np.abs(x_ref).max()
    assert rel < 2e-6, rel
    g16 = R.bf16_bits_to_f32(out16.view(torch.int16).cpu().numpy().view(np.uint16))
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(x_ref), 1e-30))) - 7)
    assert np.all(np.abs(g16 - x_ref) <= ulp * 0.5 + 2e-6 * np.abs(x_ref).max())


def _moe_gpu(m: TinyQwen, i: int) -> MoELayerGPU:
    """Layer i's MoE block with mlx's packed weights uploaded as they are."""
    ck = m.ck
    p = f"model.layers.{i}.mlp."

    def lin(path):
        w, s, b, bits, group = ck.quantized(path)
        return GPULinear.from_host(w, s.astype(np.float32), b.astype(np.float32), group, bits, _lib.SWQ_F32)

    return MoELayerGPU(lin(p + "gate"), lin(p + "switch_mlp.gate_proj"), lin(p + "switch_mlp.up_proj"),
                       lin(p + "switch_mlp.down_proj"), lin(p + "shared_expert.gate_proj"),
                       lin(p + "shared_expert.up_proj"), lin(p + "shared_expert.down_proj"),
                       lin(p + "shared_expert_gate"), top_k=m.c["num_experts_per_tok"],
                       norm_topk_prob=bool(m.c.get("norm_topk_prob", False)))


def test_tiny_q4_model_with_device_layer_tails_matches_mlx(eng):
    import torch
    from safetensors.numpy import load_file
    m = TinyQwen(G / "tiny-model-q4")
    fx = load_file(str(G / "tiny_forward_q4.safetensors"))
    toks = fx["input_ids"][0]
    ck = m.ck
    h = m.embed[toks].astype(np.float32)
    S = h.shape[0]
    print(f"tiny q4 model, {S} tokens, {m.L} layers", flush=True)
    hd = torch.from_numpy(h).cuda()
    for i in range(m.L):
        p = f"model.layers.{i}."
        x = rms_norm(hd.cpu().numpy(), ck.tensor(p + "input_layernorm.weight"), m.eps)
        r = m.deltanet_forward(x, i) if m.is_linear(i) else m.attention_forward(x, i)
        post = torch.from_numpy(ck.tensor(p + "post_attention_layernorm.weight")).cuda()
        x2 = eng.rms_norm(hd, post, m.eps, residual=torch.from_numpy(np.ascontiguousarray(r, np.float32)).cuda())
        layer = _moe_gpu(m, i)
        layer.decode(x2, out=hd, accumulate=True)
        torch.cuda.synchronize()
    hn = eng.rms_norm(hd, torch.from_numpy(m.final_norm).cuda(), m.eps)
    w, s, b, bits, group = ck.quantized("lm_head")
    head = GPULinear.from_host(w, s.astype(np.float32), b.astype(np.float32), group, bits, _lib.SWQ_F32)
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


@pytest.mark.parametrize("name,with_residual,shared", [
    ("qwen3.6-35b-a3b-q4", True, True), ("qwen3.6-35b-a3b-q4", False, True), ("qwen3.6-35b-a3b-q4", True, False),
    ("qwen3-next-80b-a3b-q4", True, True),  # top-10 of 512: the picks past the eighth as split slots
])
def test_moe_decode_with_folded_norm(eng, name, with_residual, shared):
    """swq_moe_decode_norm: the residual add and the post-attention RMSNorm in
    the MoE step's launch.  out - (h + r) is the MoE output of the
    normalised input: the oracle's expert ids exactly (the input's top-k
    margin checked first), the MoE output within the decode bar (1e-3
    relative L2, fp32 sums in another order), and within 1e-4 of swq_rmsnorm
    followed by swq_moe_decode (the sum of squares is taken in another
    order, so x differs in the last bits).  h and r are left as they were."""
    import torch
    from swiftlet_amd import moe, synth
    from tests import helpers
    shape = synth.SHAPES[name]
    print(f"folded norm: {name} residual {with_residual} shared {shared}", flush=True)
    if not shared:  # has_shared = 0 (QwenCPUModel.swift:559-566 skips the shared expert)
        shape = synth.MoEShape("no-shared", 2048, 256, 8, 512, 0, 4)
    layer = moe.synth_layer(shape, helpers.SEED, 0, "cuda")
    ref_layer = helpers.ref_layer(shape, helpers.SEED, 0)
    rng = np.random.default_rng(31)
    checked = 0
    w16 = (1 + 0.1 * rng.standard_normal(shape.hidden)).astype(np.float32)
    wt = torch.from_numpy(w16).to(torch.bfloat16).cuda()
    w_dev = wt.float().cpu().numpy()
    for trial in range(8):
        h = (rng.standard_normal(shape.hidden) * 2).astype(np.float32)
        r = rng.standard_normal(shape.hidden).astype(np.float32) if with_residual else None
        h1 = (h + r).astype(np.float32) if with_residual else h
        x = rms_norm(h1[None], w_dev, EPS)
        if R.router_margin(x, ref_layer)[0] <= 1e-3:
            continue
        ref_m, picks, ref_w = R.moe_forward(x, ref_layer)
        hd = torch.from_numpy(h).cuda()
        rd = torch.from_numpy(r).cuda() if with_residual else None
        out, ids, wts = layer.decode_norm(hd, wt, EPS, residual=rd)
        # the separate launches
        hs = hd.clone()
        x_sep = eng.rms_norm(hs, wt, EPS, residual=rd)
        sep, sep_ids, _ = layer.decode(x_sep, out=hs, accumulate=True)
        torch.cuda.synchronize()
        print(f"trial {trial}", flush=True)
        assert np.array_equal(hd.cpu().numpy(), h)  # inputs untouched
        assert ids.cpu().numpy()[0].tolist() == [e for e, _ in picks[0]]
        assert np.allclose(wts.cpu().numpy()[0], ref_w[0], rtol=1e-5, atol=1e-7)
        got_m = out.cpu().numpy() - h1
        assert R.rel_l2(got_m[None], ref_m) < 1e-3
        assert torch.equal(ids, sep_ids)
        sep_h = sep.cpu().numpy().reshape(-1)
        assert np.abs(out.cpu().numpy() - sep_h).max() <= 1e-4 * np.abs(sep_h).max()
        checked += 1
    assert checked >= 6, checked  # trials inside the top-k margin guard are skipped


def test_moe_decode_norm_limits(eng):
    """A layer outside the single launch (f32 scales, the tiny fixture
    model) returns SWQ_ERR_LIMIT: the caller falls back to the separate
    launches."""
    import torch
    m = TinyQwen(G / "tiny-model-q4")
    layer = _moe_gpu(m, 0)
    h = torch.zeros(m.c["hidden_size"], dtype=torch.float32, device="cuda")
    w = torch.ones(m.c["hidden_size"], dtype=torch.float32, device="cuda")
    with pytest.raises(_lib.SwqError) as e:
        layer.decode_norm(h, w, EPS)
    assert e.value.code == _lib.SWQ_ERR_LIMIT
