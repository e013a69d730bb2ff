"""Quantized GEMV and dequantisation on the device against the oracle.

Mirrors MetalKernelTests.gemvAffineMatchesCPU (MetalKernelTests.swift:21-77):
the same LCG inputs (O=48, I=128, group 32), bits 4/8, scalar and fast
kernels, f32 and bf16-truncated scales, 1e-3 absolute per row."""

import numpy as np
import pytest

from oracle import moe_ref as R
from swiftlet_amd import synth
from swiftlet_amd._lib import SWQ_BF16, SWQ_F16, SWQ_F32
from swiftlet_amd.engine import GPULinear
from tests import helpers

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("use_fast", [False, True])
def test_gemv_affine_matches_cpu(engine, bits, use_fast):
    O, I, group, packed, scales_f, biases_f, x = helpers.kat_inputs(bits)
    y = engine.gemv_quantized(x, packed, scales_f, biases_f, O, I, group, bits, SWQ_F32, use_fast)
    ref = R.gemv_kat_brute(x, packed.reshape(O, -1), scales_f, biases_f, bits, group)
    assert np.all(np.abs(y - ref) < 1e-3), np.abs(y - ref).max()

    sb = R.f32_to_bf16_bits_trunc(scales_f)
    bb = R.f32_to_bf16_bits_trunc(biases_f)
    y16 = engine.gemv_quantized(x, packed, sb, bb, O, I, group, bits, SWQ_BF16, use_fast)
    ref16 = R.gemv_kat_brute(x, packed.reshape(O, -1), R.bf16_bits_to_f32(sb), R.bf16_bits_to_f32(bb), bits, group)
    assert np.all(np.abs(y16 - ref16) < 1e-3), np.abs(y16 - ref16).max()


@pytest.mark.parametrize("rows,cols,bits,group,stype", [
    (512, 2048, 4, 64, SWQ_F16), (2048, 512, 4, 64, SWQ_F16), (256, 2048, 8, 64, SWQ_F16),
    (2048, 512, 8, 64, SWQ_BF16), (96, 256, 4, 32, SWQ_F32), (33, 128, 8, 128, SWQ_F16),
    (7, 64, 2, 32, SWQ_F32), (2048, 4096, 4, 64, SWQ_F16), (65, 3072, 4, 64, SWQ_BF16),
    (130, 2112, 4, 64, SWQ_F32),
])
def test_encode_gemv_full_shapes(engine, device, rows, cols, bits, group, stype):
    import torch
    rng = np.random.default_rng(rows * 31 + cols + bits)
    words = rng.integers(0, 2**32, size=(rows, cols * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.02, size=(rows, cols // group)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, size=(rows, cols // group)).astype(np.float32)
    if stype == SWQ_F16:
        s_raw, b_raw = s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    elif stype == SWQ_BF16:
        s_raw, b_raw = R.f32_to_bf16_bits_rne(s), R.f32_to_bf16_bits_rne(b)
    else:
        s_raw, b_raw = s, b
    lin = GPULinear.from_host(words, s_raw, b_raw, group, bits, stype, device)
    x = rng.standard_normal(cols).astype(np.float32)
    xt = torch.from_numpy(x).to(device)
    y = torch.full((rows + 5,), -7.0, dtype=torch.float32, device=device)
    engine.encode_gemv(lin, xt, y, y_off=3)
    torch.cuda.synchronize()
    yh = y.cpu().numpy()
    ref = R.gemv_affine(x, words, s_raw, b_raw, bits, group, stype)
    assert np.all(yh[:3] == -7.0) and np.all(yh[rows + 3:] == -7.0)
    err = np.abs(yh[3:rows + 3] - ref)
    assert err.max() <= 1e-5 * max(1.0, np.abs(ref).max()) + 1e-5, err.max()


def test_encode_gemv_stacked_expert_slice(engine, device):
    """wExtra/sExtra/bExtra select one expert of a stack (encodeGemv's
    expert slicing, QwenMetalModel.swift:669-673)."""
    import torch
    E, rows, cols, bits, group = 4, 64, 512, 4, 64
    w, s, b = synth.qmatrix(7, 0, "gate", E, rows, cols, bits, group)
    lin = GPULinear.from_host(w, s, b, group, bits, SWQ_F16, device)
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    xt = torch.from_numpy(x).to(device)
    for e in range(E):
        y = torch.zeros(rows, dtype=torch.float32, device=device)
        engine.encode_gemv(lin, xt, y, rows=rows, w_extra=e * lin.expert_stride_w,
                           s_extra=e * lin.expert_stride_sb, b_extra=e * lin.expert_stride_sb)
        torch.cuda.synchronize()
        ref = R.gemv_affine(x, w[e], s[e], b[e], bits, group, R.F16)
        assert np.abs(y.cpu().numpy() - ref).max() < 1e-5


def test_silu_mul(engine, device):
    import torch
    g = np.linspace(-20, 20, 1000).astype(np.float32)
    u = np.random.default_rng(3).standard_normal(1000).astype(np.float32)
    buf = torch.from_numpy(np.concatenate([g, u, np.zeros(1000, np.float32)])).to(device)
    engine.encode_silu_mul(buf, 1000, 0, 1000, 2000)
    torch.cuda.synchronize()
    h = buf.cpu().numpy()[2000:]
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(h, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("bits,group,stype", [(4, 64, SWQ_F16), (8, 64, SWQ_BF16), (4, 32, SWQ_F32), (8, 128, SWQ_F32)])
def test_dequantize_bit_exact(engine, device, bits, group, stype):
    """Dequantised values equal Checkpoint.dequantized's f32 scale*q + bias
    bit for bit (random scales and biases, so the rounding is exercised)."""
    rng = np.random.default_rng(bits * 100 + group)
    E, rows, cols = 3, 40, 256
    words = rng.integers(0, 2**32, size=(E, rows, cols * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.05, size=(E, rows, cols // group)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, size=(E, rows, cols // group)).astype(np.float32)
    if stype == SWQ_F16:
        s_raw, b_raw = s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    elif stype == SWQ_BF16:
        s_raw, b_raw = R.f32_to_bf16_bits_rne(s), R.f32_to_bf16_bits_rne(b)
    else:
        s_raw, b_raw = s, b
    lin = GPULinear.from_host(words, s_raw, b_raw, group, bits, stype, device)
    got = engine.dequantize(lin, 10, E * rows - 10)
    import torch
    torch.cuda.synchronize()
    ref = R.dequantize(words, s_raw, b_raw, bits, group, stype).reshape(E * rows, cols)[10:]
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_synth_device_matches_host(device):
    import torch
    from swiftlet_amd import moe
    shape = synth.SHAPES["qwen3.6-35b-a3b-q4"]
    for kind, ex, rows, cols, bits in (("gate", 3, 512, 2048, 4), ("router", None, 256, 2048, 8),
                                       ("down", 3, 2048, 512, 4)):
        lin = moe.synth_linear(11, 5, kind, ex, rows, cols, bits, shape.group, device)
        torch.cuda.synchronize()
        w, s, b = synth.qmatrix(11, 5, kind, ex, rows, cols, bits, shape.group)
        assert np.array_equal(lin.w.cpu().numpy().view(np.uint32), w.reshape(-1))
        assert np.array_equal(lin.scales.cpu().numpy().view(np.uint16), s.reshape(-1))
        assert np.array_equal(lin.biases.cpu().numpy().view(np.uint16), b.reshape(-1))


def _random_linear(rng, rows, cols, bits, group, stype, device):
    words = rng.integers(0, 2**32, size=(rows, cols * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.02, size=(rows, cols // group)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, size=(rows, cols // group)).astype(np.float32)
    if stype == SWQ_F16:
        s_raw, b_raw = s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    elif stype == SWQ_BF16:
        s_raw, b_raw = R.f32_to_bf16_bits_rne(s), R.f32_to_bf16_bits_rne(b)
    else:
        s_raw, b_raw = s, b
    return GPULinear.from_host(words, s_raw, b_raw, group, bits, stype, device), (words, s_raw, b_raw)


@pytest.mark.parametrize("cols,bits,stype,norm", [
    (2048, 4, SWQ_F16, None), (2048, 4, SWQ_F16, "bf16"), (4096, 4, SWQ_BF16, "f32"), (1024, 8, SWQ_F32, "f16"),
])
def test_gemv_multi_matches_separate_calls(engine, device, cols, bits, stype, norm):
    """swq_encode_gemv_multi: several matrices sharing x in one launch (the
    projections of a layer), optionally behind the fused input RMSNorm.
    Without the norm every output equals the separate swq_encode_gemv call
    bit for bit (the same tiles and sums); with it, within 1e-5 of
    swq_rmsnorm followed by the separate calls (the sum of squares is taken
    in another order) and of the oracle's rms_norm + gemv_affine."""
    import torch
    from oracle.qwen_tiny import rms_norm
    rng = np.random.default_rng(cols + bits)
    rows = [700, 320, 32, 5]
    lins, host = zip(*[_random_linear(rng, r, cols, bits, 64, stype, device) for r in rows])
    h = (rng.standard_normal(cols) * 2).astype(np.float32)
    ht = torch.from_numpy(h).to(device)
    w = None
    if norm is not None:
        wt = (1 + 0.2 * rng.standard_normal(cols)).astype(np.float32)
        w = torch.from_numpy(wt).to(device).to({"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[norm])
    ys = [torch.full((r,), -3.0, dtype=torch.float32, device=device) for r in rows]
    engine.encode_gemv_multi(list(lins), ht, ys, norm_weight=w, eps=1e-6)
    x_sep = ht if w is None else engine.rms_norm(ht.clone().unsqueeze(0), w, 1e-6)[0]
    sep = [torch.empty((r,), dtype=torch.float32, device=device) for r in rows]
    for lin, y in zip(lins, sep):
        engine.encode_gemv(lin, x_sep, y)
    torch.cuda.synchronize()
    x_ref = h if w is None else rms_norm(h, w.float().cpu().numpy(), 1e-6)
    for i, (y, ys_, (words, s_raw, b_raw)) in enumerate(zip(ys, sep, host)):
        got, want = y.cpu().numpy(), ys_.cpu().numpy()
        if w is None:
            assert np.array_equal(got, want), i
        else:
            assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max()), i
        ref = R.gemv_affine(x_ref, words, s_raw, b_raw, bits, 64, stype)
        assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max()) + 1e-5, i
