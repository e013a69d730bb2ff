"""The oracle against the reference's mlx fixtures (tests/golden/swiftlet_fixtures,
copied from Swiftlet's fixtures/).  Mirrors FixtureForwardTests
(FixtureForwardTests.swift:21-102): layer-local checks of every decoder layer
from the reference input (5e-4), end-to-end logits (0.05 for f32, 2e-3 for
the 4-bit model) and greedy ids, for the qwen3_next models and the qwen3_5
one (nested text_config, rope_parameters, split DeltaNet projections,
"language_model." names; :55-82).  Every layer contains the MoE block, so these
pin the oracle's router softmax, top-k, renormalisation, SwiGLU experts,
shared-expert gate and (through the 4-bit model) the MLX affine dequant
against mlx itself."""

import json
from pathlib import Path

import numpy as np
import pytest
from safetensors.numpy import load_file

from oracle import moe_ref as R
from oracle.qwen_tiny import TinyQwen

G = Path(__file__).resolve().parent / "golden" / "swiftlet_fixtures"


@pytest.fixture(scope="module")
def f32_model():
    return TinyQwen(G / "tiny-model"), load_file(str(G / "tiny_forward.safetensors"))


@pytest.fixture(scope="module")
def q4_model():
    return TinyQwen(G / "tiny-model-q4"), load_file(str(G / "tiny_forward_q4.safetensors"))


@pytest.fixture(scope="module")
def q35_model():
    return TinyQwen(G / "tiny-model-q35"), load_file(str(G / "tiny_forward_q35.safetensors"))


def test_tiny_model_layers_match_mlx(f32_model):
    m, fx = f32_model
    toks = fx["input_ids"][0]
    assert np.abs(m.embed[toks] - fx["embed"][0]).max() < 1e-6
    prev = fx["embed"][0]
    for i in range(m.L):
        ref = fx[f"layer_{i:02d}"][0]
        diff = np.abs(m.layer_forward(prev, i) - ref).max()
        assert diff < 5e-4, (i, diff)
        prev = ref


def test_tiny_model_logits_and_greedy_match_mlx(f32_model):
    m, fx = f32_model
    logits, _, greedy = m.forward(fx["input_ids"][0])
    assert np.abs(logits - fx["logits"][0]).max() < 0.05
    want = json.loads((G / "tiny_forward.json").read_text())["greedy_next_tokens"]
    assert greedy.tolist() == want


def test_tiny_q4_model_logits_and_greedy_match_mlx(q4_model):
    m, fx = q4_model
    logits, _, greedy = m.forward(fx["input_ids"][0])
    assert np.abs(logits - fx["logits"][0]).max() < 2e-3
    want = json.loads((G / "tiny_forward_q4.json").read_text())["greedy_next_tokens"]
    assert greedy.tolist() == want


def test_moe_block_carries_the_layer(f32_model):
    """Replacing the MoE block's output by zeros breaks the layer-local match:
    the fixture comparison above does exercise the MoE math."""
    m, fx = f32_model
    prev = fx["embed"][0]
    x2 = m.moe_input(prev, 0)
    moe_out, picks, w = R.moe_forward(x2, m.moe_layer(0))
    assert np.abs(moe_out).max() > 1e-2
    assert all(len(p) == m.c["num_experts_per_tok"] for p in picks)
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)  # norm_topk_prob is true in the fixture config


def test_planted_mistake_is_caught(q4_model):
    """A plausible oracle mistake (dequantising with the bias dropped) makes
    the q4 logits miss mlx's by far more than the 2e-3 bar."""
    m, fx = q4_model
    orig = R.dequantize

    def no_bias(words, scales, biases, bits, group, stype=R.F32):
        return orig(words, scales, np.zeros_like(np.asarray(biases)), bits, group, stype)

    R.dequantize = no_bias
    try:
        bad = TinyQwen(G / "tiny-model-q4")
        logits, _, _ = bad.forward(fx["input_ids"][0])
    finally:
        R.dequantize = orig
    assert np.abs(logits - fx["logits"][0]).max() > 2e-3


def test_tiny_q35_model_layers_match_mlx(q35_model):
    """FixtureForwardTests.tinyQwen35ModelMatchesMLX (:55-82): the split
    layout is detected, every layer (DeltaNet and attention) from mlx's input
    within 5e-4 of mlx's output."""
    m, fx = q35_model
    assert m.split and m.c["weight_prefix"] == "language_model."
    assert m.c["rope_theta"] == 1e7 and m.c["partial_rotary_factor"] == 0.25
    toks = fx["input_ids"][0]
    assert np.abs(m.embed[toks] - fx["embed"][0]).max() < 1e-6
    prev = fx["embed"][0]
    for i in range(m.L):
        ref = fx[f"layer_{i:02d}"][0]
        diff = np.abs(m.layer_forward(prev, i) - ref).max()
        assert diff < 5e-4, (i, "deltanet" if m.is_linear(i) else "attention", diff)
        prev = ref


def test_tiny_q35_model_logits_and_greedy_match_mlx(q35_model):
    m, fx = q35_model
    logits, _, greedy = m.forward(fx["input_ids"][0])
    assert np.abs(logits - fx["logits"][0]).max() < 0.05
    want = json.loads((G / "tiny_forward_q35.json").read_text())["greedy_next_tokens"]
    assert greedy.tolist() == want


def test_q35_split_projections_are_pinned(q35_model):
    """Planted mistakes in the split layout, each caught by the layer-local
    bar: b and a swapped, or the fused layout's de-interleave applied to the
    split projections' outputs."""
    from oracle import deltanet_ref as D
    m, fx = q35_model
    x = fx["embed"][0]
    ref = fx["layer_00"][0]
    assert np.abs(m.layer_forward(x, 0) - ref).max() < 5e-4
    orig = m.deltanet_inputs
    try:
        def swapped(xx, i):
            mixed, z, b, a = orig(xx, i)
            return mixed, z, a, b
        m.deltanet_inputs = swapped
        assert np.abs(m.layer_forward(x, 0) - ref).max() > 5e-4

        def fused(xx, i):
            mixed, z, b, a = orig(xx, i)
            prm = m.deltanet_params(i)
            return D.deinterleave(np.concatenate([mixed, z], -1), np.concatenate([b, a], -1),
                                  prm["nk"], prm["nv"], prm["dk"], prm["dv"])
        m.deltanet_inputs = fused
        assert np.abs(m.layer_forward(x, 0) - ref).max() > 5e-4
    finally:
        m.deltanet_inputs = orig
