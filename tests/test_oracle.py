"""Pins of the CPU oracle (oracle/moe_ref.py, oracle/moe_ref.c) that do not
retype its formulas: the reference's own known-answer inputs, closed forms
the format fixes, brute force on small inputs, invariants, and the C
restatement against the numpy one."""

import numpy as np
import pytest

from oracle import moe_ref as R
from swiftlet_amd import synth
from tests import helpers


# ---- format -----------------------------------------------------------------

@pytest.mark.parametrize("bits", [2, 4, 8])
def test_unpack_is_lsb_first(bits):
    """Element i of a row sits at bits [bits*(i mod 32/bits), ...) of word
    i / (32/bits) (Checkpoint.swift:195-204): checked per element with
    Python integers."""
    rng = np.random.default_rng(bits)
    words = rng.integers(0, 2**32, size=(3, 5), dtype=np.uint64).astype(np.uint32)
    codes = R.unpack_codes(words, bits)
    per = 32 // bits
    for r in range(3):
        for i in range(5 * per):
            w = int(words[r, i // per])
            assert codes[r, i] == (w >> (bits * (i % per))) & ((1 << bits) - 1)
    assert np.array_equal(R.pack_codes(codes, bits), words)


def test_dequantize_closed_form_exact():
    """With bias = -8*scale (q4) and -128*scale (q8), w = scale*(q - 8) (or
    q - 128) exactly: the product of an fp16 scale and a <= 8-bit integer is
    exact in f32, so the oracle must reproduce it bit for bit."""
    for bits, kind in ((4, "gate"), (8, "router")):
        w, s, b = synth.qmatrix(3, 1, kind, None, 16, 256, bits, 64)
        d = R.dequantize(w, s, b, bits, 64, R.F16)
        q = R.unpack_codes(w, bits).astype(np.float64)
        sf = np.repeat(s.view(np.float16).astype(np.float64), 64, axis=1)
        exact = sf * (q - (8 if bits == 4 else 128))
        assert np.array_equal(d.astype(np.float64), exact)


def test_dequantize_two_roundings():
    """scale*q + bias rounds the product, then the sum (no fused multiply-add):
    compare with float64 arithmetic rounded the same two ways."""
    rng = np.random.default_rng(9)
    w = rng.integers(0, 2**32, size=(4, 8), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.05, size=(4, 2)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, size=(4, 2)).astype(np.float32)
    d = R.dequantize(w, s, b, 4, 32, R.F32)
    q = R.unpack_codes(w, 4).astype(np.float64)
    prod = (np.repeat(s, 32, 1).astype(np.float64) * q).astype(np.float32)
    two = (prod.astype(np.float64) + np.repeat(b, 32, 1)).astype(np.float32)
    fused = (np.repeat(s, 32, 1).astype(np.float64) * q + np.repeat(b, 32, 1)).astype(np.float32)
    assert np.array_equal(d, two)
    assert not np.array_equal(two, fused)  # the inputs do exercise the difference


def test_scale_dtype_decoding():
    f = np.array([0.0123, -1.5, 3.0e-5, 65504.0], dtype=np.float32)
    assert np.array_equal(R.scales_to_f32(f.astype(np.float16).view(np.uint16), R.F16),
                          f.astype(np.float16).astype(np.float32))
    bf = R.f32_to_bf16_bits_trunc(f)
    assert np.array_equal(R.scales_to_f32(bf, R.BF16), (f.view(np.uint32) & 0xFFFF0000).view(np.float32))


# ---- GEMV -------------------------------------------------------------------

@pytest.mark.parametrize("bits", [4, 8])
def test_kat_inputs_and_factored_form(bits):
    """The regenerated MetalKernelTests inputs (LCG seed 42) through the
    factored per-group sum of Kernels.metal.txt:56-75 agree with the test's
    per-element f32 brute force (MetalKernelTests.swift:33-48)."""
    O, I, group, packed, sf, bf, x = helpers.kat_inputs(bits)
    assert packed.shape == (O * I * bits // 32,) and sf.shape == (O * I // group,)
    assert -1.0 <= x.min() and x.max() <= 1.0
    brute = R.gemv_kat_brute(x, packed.reshape(O, -1), sf, bf, bits, group)
    fact = R.gemv_affine(x, packed.reshape(O, -1), sf, bf, bits, group, R.F32)
    assert np.abs(brute - fact).max() < 1e-4


def test_kat_lcg_first_values():
    """The LCG (MetalKernelTests.swift:8-16) from seed 42: independent
    big-integer evaluation of its recurrence."""
    rng = helpers.LCG(42)
    s = 42
    for _ in range(5):
        s = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        assert rng.next32() == s >> 32


def test_gemv_closed_forms():
    rng = np.random.default_rng(4)
    rows, cols, g = 6, 128, 32
    s = rng.uniform(0.01, 0.02, size=(rows, cols // g)).astype(np.float32)
    # all codes 8 with bias -8*scale: every weight is exactly zero
    w8 = R.pack_codes(np.full((rows, cols), 8, np.uint32), 4)
    assert np.all(R.gemv_affine(rng.standard_normal(cols), w8, s, -8 * s, 4, g, R.F32) == 0)
    # one-hot x picks one dequantised column
    w = rng.integers(0, 2**32, size=(rows, cols // 8), dtype=np.uint64).astype(np.uint32)
    b = rng.uniform(-0.1, 0.1, size=(rows, cols // g)).astype(np.float32)
    dense = R.dequantize(w, s, b, 4, g, R.F32)
    for i in (0, 37, 127):
        x = np.zeros(cols)
        x[i] = 1.0
        assert np.allclose(R.gemv_affine(x, w, s, b, 4, g, R.F32), dense[:, i], rtol=1e-12)
    # x = 1: y_r = sum_g (s * sum q + G * b)
    q = R.unpack_codes(w, 4).astype(np.float64).reshape(rows, -1, g).sum(-1)
    want = (s.astype(np.float64) * q + g * b.astype(np.float64)).sum(-1)
    assert np.allclose(R.gemv_affine(np.ones(cols), w, s, b, 4, g, R.F32), want, rtol=1e-12)


# ---- router -----------------------------------------------------------------

def test_softmax_row():
    rng = np.random.default_rng(5)
    l = (rng.standard_normal(256) * 3).astype(np.float32)
    p = R.softmax_row(l)
    ref = np.exp(l.astype(np.float64) - l.max())
    ref /= ref.sum()
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-6
    assert np.allclose(p, ref, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("E,K", [(256, 8), (512, 10), (8, 2), (60, 4), (5, 5)])
def test_topk_insertion_matches_bruteforce(E, K):
    rng = np.random.default_rng(E * 100 + K)
    for _ in range(20):
        l = (rng.standard_normal(E) * 2.5).astype(np.float32)
        picks = R.topk_insertion(R.softmax_row(l), K)
        assert [e for e, _ in picks] == list(R.topk_bruteforce(l, K))
        ps = [p for _, p in picks]
        assert ps == sorted(ps, reverse=True)


def test_topk_ties_go_to_lower_id():
    """Equal probabilities keep the lower expert id first and the strict
    `p > last` test keeps later equal ids out (QwenCPUModel.swift:513-518)."""
    p = np.array([0.1, 0.3, 0.3, 0.05, 0.3, 0.2], dtype=np.float32)
    assert [e for e, _ in R.topk_insertion(p, 2)] == [1, 2]
    assert [e for e, _ in R.topk_insertion(p, 4)] == [1, 2, 4, 5]
    assert list(R.topk_bruteforce(np.log(p), 4)) == [1, 2, 4, 5]


def test_renormalise():
    picks = [(3, 0.5), (1, 0.25), (7, 0.125)]
    w = R.renormalise(picks, True)
    assert abs(float(w.sum()) - 1.0) < 1e-6 and np.allclose(w, [4 / 7, 2 / 7, 1 / 7])
    assert np.array_equal(R.renormalise(picks, False), np.array([0.5, 0.25, 0.125], np.float32))


# ---- the layer ----------------------------------------------------------------

def _small_shape(bits=4):
    return synth.MoEShape("small", 256, 32, 4, 64, 64, expert_bits=bits, router_bits=8, group=64)


@pytest.mark.parametrize("bits", [4, 8])
def test_moe_forward_f32_matches_float64(bits):
    shape = _small_shape(bits)
    L = helpers.ref_layer(shape, 11, 0)
    x = synth.bf16_to_f32(synth.activations_bf16(2, 3, shape.hidden))
    o32, p32, w32 = R.moe_forward(x, L)
    o64, p64, w64 = R.moe_forward(x, L, dtype=np.float64)
    assert p32 == p64
    assert R.rel_l2(o32, o64) < 1e-5


def test_moe_forward_bruteforce_per_token():
    """The layer equals an independent float64 evaluation of Appendix-B
    semantics: full-softmax top-k, renormalised weights, SwiGLU experts,
    sigmoid-gated shared expert."""
    shape = _small_shape(4)
    L = helpers.ref_layer(shape, 12, 1)
    x = synth.bf16_to_f32(synth.activations_bf16(3, 2, shape.hidden)).astype(np.float64)
    out, _, _ = R.moe_forward(x, L)
    for s in range(2):
        logits = L.router_dense.astype(np.float64) @ x[s]
        top = R.topk_bruteforce(logits, shape.top_k)
        p = np.exp(logits - logits.max())
        p /= p.sum()
        w = p[top] / p[top].sum()
        y = np.zeros(shape.hidden)
        for e, wk in zip(top, w):
            g = L.gate.dense(e).astype(np.float64) @ x[s]
            u = L.up.dense(e).astype(np.float64) @ x[s]
            h = g / (1 + np.exp(-g)) * u
            y += wk * (L.down.dense(e).astype(np.float64) @ h)
        g = L.sg_dense.astype(np.float64) @ x[s]
        u = L.su_dense.astype(np.float64) @ x[s]
        sh = L.sd_dense.astype(np.float64) @ (g / (1 + np.exp(-g)) * u)
        y += sh / (1 + np.exp(-(L.seg_dense.astype(np.float64) @ x[s])))
        assert R.rel_l2(out[s], y) < 1e-5


def test_c_oracle_matches_numpy():
    pytest.importorskip("ctypes")
    from oracle import cref
    if not cref.LIB.exists():
        pytest.skip("oracle/liboracle.so not built")
    from swiftlet_amd import moe
    shape = _small_shape(4)
    arrays = moe.host_layer_arrays(shape, 13, 0)
    c = cref.CMoE(arrays, shape.hidden, shape.experts, shape.top_k, shape.inter, shape.shared_inter,
                  shape.group)
    x = synth.bf16_to_f32(synth.activations_bf16(4, 3, shape.hidden))
    out, ids, w = c.forward(x, 1)
    ref, picks, rw = R.moe_forward(x, helpers.ref_layer(shape, 13, 0))
    assert ids.tolist() == [[e for e, _ in p] for p in picks]
    assert np.allclose(w, rw, rtol=1e-6)
    assert R.rel_l2(out, ref) < 1e-5
    # and its dequantisation is bit-identical to the numpy one
    d = c.gate.dequantize(5)
    wa, sa, ba = arrays["gate"][0][5], arrays["gate"][1][5], arrays["gate"][2][5]
    assert np.array_equal(d.view(np.uint32), R.dequantize(wa, sa, ba, 4, 64, R.F16).view(np.uint32))


# ---- synthetic inputs -----------------------------------------------------------

def test_synth_distributions():
    w, s, b = synth.qmatrix(1, 0, "gate", 2, 64, 512, 4, 64)
    sf = s.view(np.float16).astype(np.float32)
    assert 0.0049 < sf.min() and sf.max() < 0.0201
    assert np.array_equal(b.view(np.float16).astype(np.float32), -8 * sf)
    codes = R.unpack_codes(w, 4)
    assert codes.min() == 0 and codes.max() == 15 and abs(codes.mean() - 7.5) < 0.1
    w8, s8, b8 = synth.qmatrix(1, 0, "router", None, 64, 512, 8, 64)
    s8f = s8.view(np.float16).astype(np.float32)
    assert 0.000299 < s8f.min() and s8f.max() < 0.00121
    assert np.array_equal(b8.view(np.float16).astype(np.float32), -128 * s8f)
    # a slice of a stack equals the stack's values there
    ws, ss, bs = synth.qmatrix(1, 0, "gate", 2, 64, 512, 4, 64, expert_range=(1, 2))
    assert np.array_equal(ws[0], w[1]) and np.array_equal(ss[0], s[1])
    x = synth.bf16_to_f32(synth.activations_bf16(0, 4, 2048))
    assert abs(x.mean()) < 0.05 and abs(x.std() - 1) < 0.05


def test_splitmix_reference_values():
    """splitmix64 from seed 0 (the published sequence starts
    0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F)."""
    z = np.arange(1, 4, dtype=np.uint64) * np.uint64(synth.GAMMA)
    with np.errstate(over="ignore"):
        v = synth._fin(z)
    assert [int(t) for t in v] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
