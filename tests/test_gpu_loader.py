"""Checkpoint and .qpack loading into HBM (swq_checkpoint_load /
swq_checkpoint_linear / swq_qpack_load_experts / swq_qpack_expert_linear).

Bar: every byte that reaches the device equals the file's (tensors, whole
layer files, expert ranges, a tensor larger than the two 16 MiB staging
buffers so the copy cycles through both several times); the MoE block built
from qpack blobs resident in HBM and addressed in place gives the same ids
and bit-identical outputs as the block built from the stacked switch_mlp
tensors, and both agree with the oracle's MoE forward; the reference's tiny
4-bit qwen3_next model with every device weight loaded by the library (MoE
experts from the container) matches mlx's logits (2e-3,
FixtureForwardTests.swift:94-95) and greedy ids, as QpackTests'
streamingInstallMatchesRepacker runs the model from a container
(QpackTests.swift:66-121)."""

import json
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import moe_ref as R
from oracle import qpack_ref as Q
from oracle.qwen_tiny import TinyQwen, rms_norm
from swiftlet_amd.checkpoint import Checkpoint, QpackExpertReader, moe_layer_from_checkpoint
from swiftlet_amd.engine import HipEngine

pytestmark = pytest.mark.gpu

FIXTURES = Path(__file__).resolve().parent / "golden" / "swiftlet_fixtures"
Q4 = FIXTURES / "tiny-model-q4"


@pytest.fixture(scope="module")
def container(tmp_path_factory):
    out = tmp_path_factory.mktemp("qpack") / "tiny-q4.qpack"
    Q.repack(Q4, out)
    return out


def _bytes(t) -> bytes:
    import torch
    return t.contiguous().view(torch.uint8).cpu().numpy().tobytes()


def test_tensor_and_layer_bytes_reach_the_device(container):
    import torch
    c = Checkpoint(Q4)
    for name in ("model.embed_tokens.weight", "model.layers.0.mlp.gate.weight", "lm_head.scales",
                 "model.layers.3.self_attn.q_norm.weight"):
        t = c.load(name)
        torch.cuda.synchronize()
        assert _bytes(t) == c.raw_tensor(name), name
        assert tuple(t.shape) == c.info(name).shape
    r = QpackExpertReader(container)
    for layer in (0, r.layer_count - 1):
        blobs = r.load_experts(layer)
        torch.cuda.synchronize()
        f = (container / "packed_experts" / f"layer_{layer:02d}.bin").read_bytes()
        assert _bytes(blobs) == f, layer
        part = r.load_experts(layer, first=3, count=2)
        torch.cuda.synchronize()
        assert _bytes(part) == f[3 * r.expert_stride:5 * r.expert_stride]


def test_large_tensor_cycles_the_staging_buffers(tmp_path):
    import torch
    rng = np.random.default_rng(11)
    n = 40 * (1 << 20) + 4 * 12345  # 2.5 staging buffers, not a multiple of the chunk
    raw = rng.integers(0, 2**32, n // 4, dtype=np.uint32).tobytes()
    Q.write_safetensors(tmp_path / "model.safetensors",
                        [("small", "F32", [3], struct.pack("<3f", 1, 2, 3)), ("big", "U32", [n // 4], raw)])
    c = Checkpoint(tmp_path)
    print(f"loading {n} bytes", flush=True)
    t = c.load("big")
    torch.cuda.synchronize()
    assert _bytes(t) == raw
    assert c.load("small").cpu().tolist() == [1.0, 2.0, 3.0]


def test_moe_from_qpack_equals_moe_from_stacked_tensors(container):
    import torch
    cfg = json.loads((Q4 / "config.json").read_text())
    ck, packed, r = Checkpoint(Q4), Checkpoint(container), QpackExpertReader(container)
    tiny = TinyQwen(Q4)
    rng = np.random.default_rng(5)
    for layer in range(cfg["num_hidden_layers"]):
        print(f"layer {layer}", flush=True)
        a = moe_layer_from_checkpoint(ck, layer, cfg)
        b = moe_layer_from_checkpoint(packed, layer, cfg, qpack=r)
        assert b.gate.expert_stride_w == r.expert_stride and b.num_experts == cfg["num_experts"]
        x = rng.standard_normal((3, cfg["hidden_size"])).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        oa, ia, wa = a.decode(xd)
        ob, ib, wb = b.decode(xd)
        torch.cuda.synchronize()
        assert torch.equal(ia, ib) and torch.equal(wa, wb)
        assert torch.equal(oa, ob), layer
        ref, picks, _ = R.moe_forward(x, tiny.moe_layer(layer))
        assert ia.cpu().numpy().tolist() == [[e for e, _ in p] for p in picks]
        assert R.rel_l2(ob.cpu().numpy(), ref) < 1e-5


def test_tiny_q4_model_loaded_by_the_library_matches_mlx(container):
    import torch
    from safetensors.numpy import load_file
    eng = HipEngine()
    cfg = json.loads((Q4 / "config.json").read_text())
    packed, r = Checkpoint(container), QpackExpertReader(container)
    m = TinyQwen(Q4)  # attention and DeltaNet on the host
    fx = load_file(str(FIXTURES / "tiny_forward_q4.safetensors"))
    toks = fx["input_ids"][0]
    emb = packed.gpu_linear("model.embed_tokens")  # the embedding rows, dequantised on the device
    hd = torch.cat([eng.dequantize(emb, int(t), 1) for t in toks])
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        x = rms_norm(hd.cpu().numpy(), packed.load(p + "input_layernorm.weight").cpu().numpy(), m.eps)
        att = m.deltanet_forward(x, i) if m.is_linear(i) else m.attention_forward(x, i)
        x2 = eng.rms_norm(hd, packed.load(p + "post_attention_layernorm.weight"), m.eps,
                          residual=torch.from_numpy(np.ascontiguousarray(att, np.float32)).cuda())
        moe_layer_from_checkpoint(packed, i, cfg, qpack=r).decode(x2, out=hd, accumulate=True)
        torch.cuda.synchronize()
    hn = eng.rms_norm(hd, packed.load("model.norm.weight"), m.eps)
    head = packed.gpu_linear("lm_head")
    logits = torch.empty((len(toks), head.out_dim), dtype=torch.float32, device="cuda")
    for t in range(len(toks)):
        eng.encode_gemv(head, hn[t], logits[t])
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    diff = np.abs(got - fx["logits"][0]).max()
    print(f"max |logit - mlx| = {diff:.3g}", flush=True)
    assert diff < 2e-3, diff
    want = json.loads((FIXTURES / "tiny_forward_q4.json").read_text())["greedy_next_tokens"]
    assert np.argmax(got, axis=-1).tolist() == want
