"""MoE-layer decode on the device against the oracle (QwenCPUModel.moeForward,
QwenCPUModel.swift:500-569), at the benchmark shapes and at odd ones.

Bar: expert ids equal the oracle's wherever the router's k-th/(k+1)-th
logit gap exceeds 1e-3 (f32 summation-order noise of the router GEMV is
~1e-6 here); combine weights within 1e-5; layer output within 1e-3
relative L2 of the f32 oracle (the observed error is ~1e-6)."""

import numpy as np
import pytest

from oracle import moe_ref as R
from swiftlet_amd import moe, synth
from tests import helpers

pytestmark = pytest.mark.gpu

REL_L2_BAR = 1e-3
MARGIN = 1e-3


def _run(shape, batch, x_dtype="bf16", out_dtype="f32", seed=helpers.SEED, layer=0, gpu=None, path="auto"):
    import torch
    from swiftlet_amd import _lib
    gpu = gpu or moe.synth_layer(shape, seed, layer)
    xb = synth.activations_bf16(seed + 1000 * layer + batch, batch, shape.hidden)
    xf = synth.bf16_to_f32(xb)
    if x_dtype == "bf16":
        x = helpers.bf16_bits_to_torch(xb)
    else:
        x = torch.from_numpy(xf).cuda()
    odt = torch.float32 if out_dtype == "f32" else torch.bfloat16
    ws = gpu.new_workspace(batch)
    out, ids, w = gpu.decode(x, out_dtype=odt, ws=ws, path=path)
    torch.cuda.synchronize()
    # every bounded wait of the call completed (the single launch at batch 1)
    assert gpu.workspace_status(ws) == _lib.SWQ_OK
    return gpu, xf, out, ids.cpu().numpy(), w.cpu().numpy()


def _check_against_oracle(shape, xf, out, ids, w, seed=helpers.SEED, layer=0):
    import torch
    ref_layer = helpers.ref_layer(shape, seed, layer)
    ref_out, picks, ref_w = R.moe_forward(xf, ref_layer)
    margin = R.router_margin(xf, ref_layer)
    B = xf.shape[0]
    checked = 0
    for b in range(B):
        ref_ids = [e for e, _ in picks[b]]
        if margin[b] > MARGIN:
            assert list(ids[b]) == ref_ids, (b, ids[b], ref_ids)
            assert np.allclose(w[b], ref_w[b], rtol=1e-5, atol=1e-7)
            checked += 1
    # the selection was actually compared: at most one token of a batch may
    # fall inside the margin guard (none does for the seeds used here)
    assert checked >= max(1, B - 1), (checked, B, margin)
    if out.dtype == torch.bfloat16:
        got = R.bf16_bits_to_f32(helpers.torch_bf16_to_bits(out))
        ref_b = R.bf16_bits_to_f32(R.f32_to_bf16_bits_rne(ref_out))
        assert R.rel_l2(got, ref_b) < REL_L2_BAR
        # bf16 of an f32 output whose error is ~1e-6 of the output's rms: at
        # most one ulp from the oracle's rounding wherever the value is at least
        # 1% of the rms (there a bf16 ulp, >= 2^-8 |v|, exceeds that error), and
        # everywhere within the rounding (<= 2^-8 |v|) plus 2e-5 of the rms
        ref = ref_out.astype(np.float64)
        rms = float(np.sqrt(np.mean(ref ** 2)))
        ulp = np.abs(helpers.torch_bf16_to_bits(out).astype(np.int32)
                     - R.f32_to_bf16_bits_rne(ref_out).astype(np.int32))
        assert ulp[np.abs(ref) >= 1e-2 * rms].max() <= 1
        assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 2e-5 * rms)
    else:
        got = out.cpu().numpy()
        err = R.rel_l2(got, ref_out)
        assert err < REL_L2_BAR, err
        assert err < 1e-5, err  # fp32 accumulation throughout: far inside the bar
    return ref_out


@pytest.mark.parametrize("name,batch", [
    ("qwen3.6-35b-a3b-q4", 1),
    ("qwen3-next-80b-a3b-q4", 1),
    ("qwen3.6-35b-a3b-q8", 1),
    ("qwen3.6-35b-a3b-q8", 4),   # one launch, token-major slots
    ("qwen3.6-35b-a3b-q4", 4),
    ("qwen3-next-80b-a3b-q4", 2),
    ("qwen3.6-35b-a3b-q4", 3),   # three launches
])
def test_moe_decode_matches_oracle(name, batch):
    shape = synth.SHAPES[name]
    gpu, xf, out, ids, w = _run(shape, batch)
    _check_against_oracle(shape, xf, out, ids, w)


def test_moe_decode_bf16_out_and_f32_x():
    shape = synth.SHAPES["qwen3.6-35b-a3b-q4"]
    gpu, xf, out, ids, w = _run(shape, 2, x_dtype="f32", out_dtype="bf16")
    _check_against_oracle(shape, xf, out, ids, w)


def test_moe_decode_deterministic_and_accumulate():
    import torch
    shape = synth.SHAPES["qwen3.6-35b-a3b-q4"]
    gpu = moe.synth_layer(shape, helpers.SEED, 0)
    xb = synth.activations_bf16(5, 1, shape.hidden)
    x = helpers.bf16_bits_to_torch(xb)
    ws = gpu.new_workspace(1)
    o1, i1, w1 = gpu.decode(x, ws=ws)
    o1, i1, w1 = o1.clone(), i1.clone(), w1.clone()
    o2, i2, w2 = gpu.decode(x, ws=ws)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(i1, i2) and torch.equal(w1, w2)
    resid = torch.randn_like(o1)
    acc = resid.clone()
    gpu.decode(x, out=acc, ws=ws, accumulate=True)
    torch.cuda.synchronize()
    assert torch.allclose(acc, resid + o1, rtol=0, atol=1e-5)


@pytest.mark.parametrize("E,K,I,Is,H,bits,norm", [
    (8, 2, 32, 32, 64, 4, True),      # the tiny model's MoE shape
    (60, 4, 64, 128, 256, 8, False),  # E not a multiple of 64, norm_topk_prob false
    (128, 1, 128, 64, 512, 4, True),  # top-1
    (1024, 16, 64, 64, 128, 4, True), # widest top-k table
])
def test_moe_decode_odd_shapes(E, K, I, Is, H, bits, norm):
    shape = synth.MoEShape("odd", H, E, K, I, Is, expert_bits=bits, router_bits=8,
                           group=64 if H % 64 == 0 and I % 64 == 0 else 32, norm_topk_prob=norm)
    for batch in (1, 2, 4, 5):  # 5: the three launches
        print(f"odd shape {E},{K},{I},{Is},{H},{bits} batch {batch}", flush=True)
        gpu, xf, out, ids, w = _run(shape, batch, seed=77)
        _check_against_oracle(shape, xf, out, ids, w, seed=77)


# ---------------------------------------------------------------------------
# the single-launch path against the three-launch path: the same tiles and
# reduction orders, so equal bit for bit

def _pair(gpu, shape, x, out_dtype, ws_f, ws_s):
    import torch
    odt = torch.float32 if out_dtype == "f32" else torch.bfloat16
    of, i_f, w_f = gpu.decode(x, out_dtype=odt, ws=ws_f, path="fused")
    os_, i_s, w_s = gpu.decode(x, out_dtype=odt, ws=ws_s, path="staged")
    torch.cuda.synchronize()
    return (of, i_f, w_f), (os_, i_s, w_s)


@pytest.mark.parametrize("name", ["qwen3.6-35b-a3b-q4", "qwen3-next-80b-a3b-q4", "qwen3.6-35b-a3b-q8"])
@pytest.mark.parametrize("x_dtype,out_dtype", [("bf16", "f32"), ("f32", "bf16")])
def test_fused_equals_staged(name, x_dtype, out_dtype):
    import torch
    shape = synth.SHAPES[name]
    print(f"fused vs staged: {name} x {x_dtype} out {out_dtype}", flush=True)
    gpu = moe.synth_layer(shape, helpers.SEED, 0)
    xb = synth.activations_bf16(helpers.SEED + 11, 1, shape.hidden)
    x = helpers.bf16_bits_to_torch(xb) if x_dtype == "bf16" else torch.from_numpy(synth.bf16_to_f32(xb)).cuda()
    ws_f, ws_s = gpu.new_workspace(1), gpu.new_workspace(1)
    (of, i_f, w_f), (os_, i_s, w_s) = _pair(gpu, shape, x, out_dtype, ws_f, ws_s)
    assert gpu.workspace_error(ws_f) == 0
    assert torch.equal(i_f, i_s) and torch.equal(w_f, w_s)
    assert torch.equal(of, os_)
    _check_against_oracle(shape, synth.bf16_to_f32(xb), of, i_f.cpu().numpy(), w_f.cpu().numpy())


@pytest.mark.parametrize("name,batch", [
    ("qwen3.6-35b-a3b-q8", 4), ("qwen3.6-35b-a3b-q4", 4), ("qwen3.6-35b-a3b-q4", 2), ("qwen3-next-80b-a3b-q4", 2)])
def test_fused_batch_equals_staged(name, batch):
    """2 or 4 tokens in one launch (slot s = pick s % K of token s / K):
    the per-token tiles and sums of the single-token launch, so equal bit for
    bit to the three launches, which read each distinct expert once."""
    import torch
    shape = synth.SHAPES[name]
    print(f"fused vs staged: {name} batch {batch}", flush=True)
    gpu = moe.synth_layer(shape, helpers.SEED, 0)
    xb = synth.activations_bf16(helpers.SEED + 12, batch, shape.hidden)
    x = helpers.bf16_bits_to_torch(xb)
    ws_f, ws_s = gpu.new_workspace(batch), gpu.new_workspace(batch)
    (of, i_f, w_f), (os_, i_s, w_s) = _pair(gpu, shape, x, "f32", ws_f, ws_s)
    assert gpu.workspace_error(ws_f, batch) == 0
    assert torch.equal(i_f, i_s) and torch.equal(w_f, w_s)
    assert torch.equal(of, os_)
    _check_against_oracle(shape, synth.bf16_to_f32(xb), of, i_f.cpu().numpy(), w_f.cpu().numpy())


@pytest.mark.parametrize("bits,Is", [(4, 2048), (8, 1024)])
@pytest.mark.parametrize("batch", [1, 2, 4])
def test_fused_wide_intermediates(bits, Is, batch):
    """Routed intermediates of 1024 rows and shared ones of 2048 (4-bit: the
    compiled maximum) or 1024 (8-bit: the widest one-chunk-per-lane down
    row): a wave's share of the owned slots' and of every token's shared
    activations takes several polling rounds (one round covers 128 routed and
    256 shared pairs per wave), on the single and the batched launches; equal
    bit for bit to the three launches and within the bar of the oracle.  The
    three launches' shared down rows then need several of that matrix's
    tiles per workgroup (its rows are longer than the routed down rows)."""
    import torch
    shape = synth.MoEShape("wide-inter", 256, 64, 8, 1024, Is, expert_bits=bits, router_bits=8, group=64,
                           norm_topk_prob=True)
    print(f"wide intermediates: bits {bits} batch {batch}", flush=True)
    gpu = moe.synth_layer(shape, 91, 0)
    xb = synth.activations_bf16(92 + batch, batch, shape.hidden)
    x = helpers.bf16_bits_to_torch(xb)
    ws_f, ws_s = gpu.new_workspace(batch), gpu.new_workspace(batch)
    (of, i_f, w_f), (os_, i_s, w_s) = _pair(gpu, shape, x, "f32", ws_f, ws_s)
    from swiftlet_amd import _lib
    assert gpu.workspace_status(ws_f) == _lib.SWQ_OK
    assert torch.equal(i_f, i_s) and torch.equal(w_f, w_s)
    assert torch.equal(of, os_)
    _check_against_oracle(shape, synth.bf16_to_f32(xb), of, i_f.cpu().numpy(), w_f.cpu().numpy(), seed=91)


def test_fused_epochs_across_calls():
    """One workspace, alternating layers and fresh inputs: each call consumes
    only what it produced itself (stale words of earlier calls carry older
    epochs), and no bounded wait runs out."""
    import torch
    shape = synth.SHAPES["qwen3.6-35b-a3b-q4"]
    layers = [moe.synth_layer(shape, helpers.SEED, r) for r in range(2)]
    ws = layers[0].new_workspace(1)
    ws_s = layers[0].new_workspace(1)
    for i in range(6):
        gpu = layers[i % 2]
        print(f"epoch call {i}", flush=True)
        xb = synth.activations_bf16(helpers.SEED + 100 + i, 1, shape.hidden)
        x = helpers.bf16_bits_to_torch(xb)
        (of, i_f, w_f), (os_, i_s, w_s) = _pair(gpu, shape, x, "f32", ws, ws_s)
        assert torch.equal(i_f, i_s) and torch.equal(w_f, w_s), i
        assert torch.equal(of, os_), i
    assert layers[0].workspace_error(ws) == 0


@pytest.mark.parametrize("E,K,I,Is,H,bits,norm", [
    (8, 2, 32, 32, 64, 4, True),
    (60, 4, 64, 128, 256, 8, False),
    (1024, 16, 64, 64, 128, 4, True),
])
def test_fused_equals_staged_odd_shapes(E, K, I, Is, H, bits, norm):
    import torch
    shape = synth.MoEShape("odd", H, E, K, I, Is, expert_bits=bits, router_bits=8,
                           group=64 if H % 64 == 0 and I % 64 == 0 else 32, norm_topk_prob=norm)
    print(f"fused vs staged odd: {E},{K},{I},{Is},{H},{bits}", flush=True)
    gpu = moe.synth_layer(shape, 77, 0)
    xb = synth.activations_bf16(78, 1, shape.hidden)
    x = helpers.bf16_bits_to_torch(xb)
    ws_f, ws_s = gpu.new_workspace(1), gpu.new_workspace(1)
    (of, i_f, w_f), (os_, i_s, w_s) = _pair(gpu, shape, x, "f32", ws_f, ws_s)
    assert gpu.workspace_error(ws_f) == 0
    assert torch.equal(i_f, i_s) and torch.equal(w_f, w_s)
    assert torch.equal(of, os_)


def test_workspace_serves_every_batch():
    """One workspace, sized for batch 4, serving batch 4, batch 1 (the single
    launch) and batch 4 again: each call equals a call on a fresh workspace.
    The single launch's exchange words sit before the staged regions, so a
    staged call's raw values never land where epoch-tagged words are
    polled."""
    import torch
    shape = synth.SHAPES["qwen3.6-35b-a3b-q4"]
    gpu = moe.synth_layer(shape, helpers.SEED, 0)
    ws = gpu.new_workspace(5)
    for i, batch in enumerate((4, 1, 5, 2, 4, 1)):
        x = helpers.bf16_bits_to_torch(synth.activations_bf16(helpers.SEED + 60 + i, batch, shape.hidden))
        o, ids, w = gpu.decode(x, ws=ws)
        fo, fids, fw = gpu.decode(x, ws=gpu.new_workspace(batch))
        torch.cuda.synchronize()
        assert torch.equal(ids, fids) and torch.equal(w, fw) and torch.equal(o, fo), (i, batch)
    from swiftlet_amd import _lib
    assert gpu.workspace_status(ws) == _lib.SWQ_OK


# a layer without a shared expert (has_shared = 0: checkpoints without
# shared_expert weights load this way; QwenCPUModel.swift:559-566 runs the
# shared expert only when present; MoEGPU's shared fields are optional,
# QwenMetalModel.swift:34-39)
NO_SHARED = synth.MoEShape("no-shared", 2048, 256, 8, 512, 0, 4)


@pytest.mark.parametrize("batch,path", [(1, "fused"), (1, "staged"), (4, "auto")])
def test_no_shared_expert_matches_oracle(batch, path):
    print(f"no shared expert: batch {batch} path {path}", flush=True)
    gpu, xf, out, ids, w = _run(NO_SHARED, batch, path=path)
    assert not gpu.has_shared
    _check_against_oracle(NO_SHARED, xf, out, ids, w)


def test_no_shared_expert_fused_equals_staged():
    import torch
    gpu = moe.synth_layer(NO_SHARED, helpers.SEED, 0)
    x = helpers.bf16_bits_to_torch(synth.activations_bf16(helpers.SEED + 5, 1, NO_SHARED.hidden))
    ws_f, ws_s = gpu.new_workspace(1), gpu.new_workspace(1)
    (of, i_f, w_f), (os_, i_s, w_s) = _pair(gpu, NO_SHARED, x, "f32", ws_f, ws_s)
    assert gpu.workspace_error(ws_f) == 0
    assert torch.equal(i_f, i_s) and torch.equal(w_f, w_s) and torch.equal(of, os_)


def test_single_expert_layer():
    """One expert and a one-row router (the single-expert workload): the pick
    is expert 0 with weight 1, out = down(silu(gate x) * up x)."""
    shape = synth.SHAPES["single-expert-q4"]
    gpu, xf, out, ids, w = _run(shape, 1)
    assert ids.tolist() == [[0]] and w.tolist() == [[1.0]]
    _check_against_oracle(shape, xf, out, ids, w)


@pytest.mark.parametrize("H,I,bits,group,norm", [
    (2048, 512, 4, 64, True),    # the single-expert workload
    (2048, 512, 8, 64, False),   # 8-bit rows, softmax weight without renormalisation
    (1024, 96, 4, 32, True),     # the last gate/up tile past I, group 32
    (512, 2048, 4, 64, False),   # the widest expert, two output rows per workgroup
    (2048, 1024, 8, 64, True),   # 8-bit down rows of one pass each: every wave of a workgroup on its rows
])
def test_one_expert_launch(H, I, bits, group, norm):
    """One routed expert and no shared expert at batch 1 take the one-expert
    launch (every workgroup its own router logit and whole output rows): equal
    bit for bit to the three launches for bf16 and f32 x, f32 and bf16 out;
    within the bar of the oracle; pick 0 with weight 1; a second call on the
    same workspace (the next epoch) equal to the first, and accumulate adding
    the same output."""
    import torch
    shape = synth.MoEShape("one", H, 1, 1, I, 0, expert_bits=bits, router_bits=8, group=group,
                           norm_topk_prob=norm)
    gpu = moe.synth_layer(shape, helpers.SEED, 0)
    xb = synth.activations_bf16(helpers.SEED + 21, 1, H)
    xf = synth.bf16_to_f32(xb)
    for x_dtype, out_dtype in (("bf16", "f32"), ("f32", "bf16")):
        print(f"one expert H{H} I{I} q{bits} g{group} norm {norm} x {x_dtype} out {out_dtype}", flush=True)
        x = helpers.bf16_bits_to_torch(xb) if x_dtype == "bf16" else torch.from_numpy(xf).cuda()
        ws_f, ws_s = gpu.new_workspace(1), gpu.new_workspace(1)
        (of, i_f, w_f), (os_, i_s, w_s) = _pair(gpu, shape, x, out_dtype, ws_f, ws_s)
        assert gpu.workspace_error(ws_f) == 0
        assert i_f.tolist() == [[0]] and w_f.tolist() == [[1.0]]
        assert torch.equal(i_f, i_s) and torch.equal(w_f, w_s) and torch.equal(of, os_)
        _check_against_oracle(shape, xf, of, i_f.cpu().numpy(), w_f.cpu().numpy())
        if out_dtype == "f32":
            o2, _, _ = gpu.decode(x, ws=ws_f, path="fused")
            resid = torch.randn_like(of)
            acc = resid.clone()
            gpu.decode(x, out=acc, ws=ws_f, accumulate=True, path="fused")
            torch.cuda.synchronize()
            assert gpu.workspace_error(ws_f) == 0
            assert torch.equal(o2, of)
            assert torch.allclose(acc, resid + of, rtol=0, atol=1e-5)


def test_fused_declines_batches():
    """The single launch takes 1, 2 or 4 tokens (a divisor of its eight
    waves, up to its four-token exchange regions) and at most 32 (token,
    pick) slots; other batches go to the three launches."""
    from swiftlet_amd import _lib
    shape = synth.SHAPES["qwen3.6-35b-a3b-q4"]
    gpu = moe.synth_layer(shape, helpers.SEED, 0)
    for batch in (3, 8):
        x = helpers.bf16_bits_to_torch(synth.activations_bf16(3, batch, shape.hidden))
        with pytest.raises(_lib.SwqError) as e:
            gpu.decode(x, path="fused")
        assert e.value.code == _lib.SWQ_ERR_LIMIT
    # at most 32 (token, pick) slots: 4 tokens of top-10 go to the three launches
    s80 = synth.SHAPES["qwen3-next-80b-a3b-q4"]
    g80 = moe.synth_layer(s80, helpers.SEED, 0)
    x = helpers.bf16_bits_to_torch(synth.activations_bf16(3, 4, s80.hidden))
    with pytest.raises(_lib.SwqError) as e:
        g80.decode(x, path="fused")
    assert e.value.code == _lib.SWQ_ERR_LIMIT


# ---------------------------------------------------------------------------
# f32 scales and biases (exact widenings of the fp16 ones): the kernels
# compiled for 4-byte scale elements give the fp16 layer's results bit for
# bit (the single launch takes fp16/bf16 scales only: the three launches)

@pytest.mark.parametrize("name,batch", [
    ("qwen3.6-35b-a3b-q4", 1),
    ("qwen3.6-35b-a3b-q4", 4),
    ("qwen3.6-35b-a3b-q8", 4),
])
def test_f32_scales_equal_f16_scales(name, batch):
    import torch
    print(f"f32 scales vs f16: {name} batch {batch}", flush=True)
    shape = synth.SHAPES[name]
    a = moe.synth_layer(shape, helpers.SEED, 0)
    b = helpers.widen_layer(a)
    x = helpers.bf16_bits_to_torch(synth.activations_bf16(helpers.SEED + 91, batch, shape.hidden))
    wa, wb = a.new_workspace(batch), b.new_workspace(batch)
    oa, ia, ka = a.decode(x, ws=wa, path="staged")
    ob, ib, kb = b.decode(x, ws=wb, path="staged")
    torch.cuda.synchronize()
    assert a.workspace_error(wa, batch) == 0 and b.workspace_error(wb, batch) == 0
    assert torch.equal(ia, ib) and torch.equal(ka, kb) and torch.equal(oa, ob)
