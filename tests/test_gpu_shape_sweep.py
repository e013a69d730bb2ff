"""A seeded sweep of layer shapes through every decode path and the prefill,
against the oracle (QwenCPUModel.moeForward, QwenCPUModel.swift:500-569)
and against each other.

The benchmark shapes and a few hand-picked odd ones have their own tests;
this one draws hidden sizes, expert counts, top-k, routed and shared
intermediates (none included), code widths, group sizes, renormalisation
and batch sizes at random (fixed seed), so that plan boundaries nobody
chose by hand are crossed: tile heights that differ between the routed and
the shared matrices, polling shares of more than one round, top-k tables of
one or of sixteen picks.  Per shape and batch:
- `swq_moe_decode` (one launch where it takes the call, else three) equals
  the three launches bit for bit (ids, weights, outputs);
- both are within the decode bar of the oracle (ids exact where the k-th /
  (k+1)-th logit gap exceeds 1e-3, weights 1e-5, outputs 1e-5 relative L2);
- the prefill of the same tokens, where its matrix-core path takes the
  layer (group 64, rows of a multiple of 128 inputs, at most 2048), gives the same ids and
  weights and outputs within 1e-5 relative L2 of the oracle.
A refusal is accepted only where the documented limits say so."""

import numpy as np
import pytest

from oracle import moe_ref as R
from swiftlet_amd import _lib, moe, synth
from tests import helpers

pytestmark = pytest.mark.gpu

MARGIN = 1e-3
N_SHAPES = 24


def _shapes():
    rng = np.random.default_rng(20261202)
    out = []
    while len(out) < N_SHAPES:
        H = int(rng.choice([64, 128, 256, 512, 1024, 2048]))
        E = int(rng.choice([8, 60, 64, 128, 256, 512]))
        K = int(rng.integers(1, min(16, E) + 1))
        I = int(rng.choice([32, 64, 128, 256, 512, 1024]))
        Is = int(rng.choice([0, 32, 64, 256, 512, 1024, 2048]))
        bits = int(rng.choice([4, 8]))
        group = int(rng.choice([32, 64]))
        norm = bool(rng.integers(0, 2))
        if H % group or I % group or (Is and Is % group):
            continue
        if bits == 8 and max(I, Is) > 1024:
            continue  # 8-bit down rows of more than 1024 inputs: SWQ_ERR_LIMIT (one chunk per lane)
        out.append((H, E, K, I, Is, bits, group, norm))
    return out


SHAPES = _shapes()


def _ids_ok(ids, w, picks, ref_w, margin):
    checked = 0
    for b in range(len(picks)):
        if margin[b] > MARGIN:
            assert list(ids[b]) == [e for e, _ in picks[b]], (b, ids[b], picks[b])
            assert np.allclose(w[b], ref_w[b], rtol=1e-5, atol=1e-7), b
            checked += 1
    return checked


@pytest.mark.parametrize("H,E,K,I,Is,bits,group,norm", SHAPES)
def test_shape_sweep(H, E, K, I, Is, bits, group, norm):
    import torch
    shape = synth.MoEShape("sweep", H, E, K, I, Is, expert_bits=bits, router_bits=8, group=group,
                           norm_topk_prob=norm)
    seed = 1000 + H + E + K + I + Is
    gpu = moe.synth_layer(shape, seed, 0)
    ref_layer = helpers.ref_layer(shape, seed, 0)
    checked = 0
    for batch in (1, 2, 3, 4):
        print(f"sweep H{H} E{E} K{K} I{I} Is{Is} q{bits} g{group} norm {norm} batch {batch}", flush=True)
        xb = synth.activations_bf16(seed + batch, batch, H)
        xf = synth.bf16_to_f32(xb)
        x = helpers.bf16_bits_to_torch(xb)
        ws_a, ws_s = gpu.new_workspace(batch), gpu.new_workspace(batch)
        oa, ia, wa = gpu.decode(x, ws=ws_a)
        os_, is_, ws_ = gpu.decode(x, ws=ws_s, path="staged")
        torch.cuda.synchronize()
        assert gpu.workspace_status(ws_a) == _lib.SWQ_OK
        assert torch.equal(ia, is_) and torch.equal(wa, ws_), batch
        assert torch.equal(oa, os_), batch
        ref_out, picks, ref_w = R.moe_forward(xf, ref_layer)
        margin = R.router_margin(xf, ref_layer)
        checked += _ids_ok(ia.cpu().numpy(), wa.cpu().numpy(), picks, ref_w, margin)
        err = R.rel_l2(oa.cpu().numpy(), ref_out)
        assert err < 1e-5, (batch, err)

        # the prefill of the same tokens
        # the matrix-core path's limits: group 64, every row of a multiple of
        # 128 inputs and at most 2048
        prefill_ok = group == 64 and all(d % 128 == 0 and d <= 2048 for d in (H, I, Is or 128))
        try:
            op, ip, wp = gpu.prefill(x)
            torch.cuda.synchronize()
        except _lib.SwqError as e:
            assert not prefill_ok and e.code == _lib.SWQ_ERR_LIMIT, (e.code, batch)
            continue
        assert torch.equal(ip, ia) and torch.allclose(wp, wa, rtol=1e-6, atol=1e-7), batch
        errp = R.rel_l2(op.cpu().numpy(), ref_out)
        assert errp < 1e-5, (batch, errp)
    assert checked >= 1


def _prefill_shapes():
    rng = np.random.default_rng(777)
    out = []
    while len(out) < 8:
        H = int(rng.choice([128, 256, 512, 1024, 2048]))
        E = int(rng.choice([8, 60, 128, 256, 512]))
        K = int(rng.integers(1, min(16, E) + 1))
        I = int(rng.choice([128, 256, 512, 1024, 2048]))
        Is = int(rng.choice([0, 128, 512, 2048]))
        bits = int(rng.choice([4, 8]))
        T = int(rng.choice([1, 7, 33, 100]))
        out.append((H, E, K, I, Is, bits, bool(rng.integers(0, 2)), T))
    return out


@pytest.mark.parametrize("H,E,K,I,Is,bits,norm,T", _prefill_shapes())
def test_prefill_shape_sweep(H, E, K, I, Is, bits, norm, T):
    """Prefill shapes inside its matrix-core path (group 64, rows of a
    multiple of 128 inputs up to 2048) at 1-100 tokens: ids exact where the
    margin allows, weights 1e-5, outputs 1e-5 relative L2 of the oracle."""
    import torch
    shape = synth.MoEShape("pf-sweep", H, E, K, I, Is, expert_bits=bits, router_bits=8, group=64,
                           norm_topk_prob=norm)
    seed = 3000 + H + E + K + I + Is + T
    print(f"prefill sweep H{H} E{E} K{K} I{I} Is{Is} q{bits} norm {norm} T{T}", flush=True)
    gpu = moe.synth_layer(shape, seed, 0)
    ref_layer = helpers.ref_layer(shape, seed, 0)
    xb = synth.activations_bf16(seed, T, H)
    xf = synth.bf16_to_f32(xb)
    out, ids, w = gpu.prefill(helpers.bf16_bits_to_torch(xb))
    torch.cuda.synchronize()
    rows = np.arange(T) if T <= 16 else np.linspace(0, T - 1, 12).astype(int)
    ref_out, picks, ref_w = R.moe_forward(xf[rows], ref_layer)
    margin = R.router_margin(xf[rows], ref_layer)
    assert _ids_ok(ids.cpu().numpy()[rows], w.cpu().numpy()[rows], picks, ref_w, margin) >= max(1, len(rows) - 1)
    err = R.rel_l2(out.cpu().numpy()[rows], ref_out)
    assert err < 1e-5, err
