"""Shared test inputs: the reference KAT's LCG, lazily generated oracle
layers for the synthetic workloads, torch/numpy conversions."""

from __future__ import annotations

import numpy as np

from oracle import moe_ref as R
from swiftlet_amd import synth

SEED = 20261201


class LCG:
    """MetalKernelTests.Rand (MetalKernelTests.swift:8-16), reproduced
    bit for bit: 64-bit LCG, next32 = state >> 32, float = next32 /
    UInt32.max * 2 - 1 evaluated in f32."""

    MUL = 6364136223846793005
    ADD = 1442695040888963407

    def __init__(self, seed: int):
        self.s = seed

    def next32(self) -> int:
        self.s = (self.s * self.MUL + self.ADD) & ((1 << 64) - 1)
        return self.s >> 32

    def float(self) -> np.float32:
        v = np.float32(self.next32()) / np.float32(4294967295)
        return np.float32(np.float32(v * np.float32(2)) - np.float32(1))


def kat_inputs(bits: int):
    """gemvAffineMatchesCPU's inputs (MetalKernelTests.swift:24-31)."""
    O, I, group = 48, 128, 32
    per = 32 // bits
    rng = LCG(42)
    packed = np.array([rng.next32() for _ in range(O * I // per)], dtype=np.uint32)
    scales = np.array([np.float32(rng.float() * np.float32(0.1)) for _ in range(O * I // group)], dtype=np.float32)
    biases = np.array([np.float32(rng.float() * np.float32(0.05)) for _ in range(O * I // group)], dtype=np.float32)
    x = np.array([rng.float() for _ in range(I)], dtype=np.float32)
    return O, I, group, packed, scales, biases, x


class LazyStack:
    """Oracle view of a synthetic expert stack: expert e is regenerated on
    the host when the oracle dequantises it."""

    def __init__(self, seed, layer, kind, experts, rows, cols, bits, group):
        self.args = (seed, layer, kind, experts, rows, cols, bits, group)
        self.out_dim, self.in_dim, self.bits, self.group = rows, cols, bits, group
        self.stype = R.F16

    def arrays(self, e: int):
        seed, layer, kind, experts, rows, cols, bits, group = self.args
        w, s, b = synth.qmatrix(seed, layer, kind, experts, rows, cols, bits, group, expert_range=(e, e + 1))
        return w[0], s[0], b[0]

    def dense(self, e=None):
        w, s, b = self.arrays(e)
        return R.dequantize(w, s, b, self.bits, self.group, R.F16)


def qlin(seed, layer, kind, rows, cols, bits, group) -> R.QLinear:
    w, s, b = synth.qmatrix(seed, layer, kind, None, rows, cols, bits, group)
    return R.QLinear(w, s, b, bits, group, R.F16)


def ref_layer(shape: synth.MoEShape, seed: int, layer: int) -> R.MoELayerRef:
    H, E, I, Is = shape.hidden, shape.experts, shape.inter, shape.shared_inter
    eb, rb, g = shape.expert_bits, shape.router_bits, shape.group
    sh = shape.has_shared
    return R.MoELayerRef(
        router=qlin(seed, layer, "router", E, H, rb, g),
        gate=LazyStack(seed, layer, "gate", E, I, H, eb, g),
        up=LazyStack(seed, layer, "up", E, I, H, eb, g),
        down=LazyStack(seed, layer, "down", E, H, I, eb, g),
        shared_gate=qlin(seed, layer, "sh_gate", Is, H, eb, g) if sh else None,
        shared_up=qlin(seed, layer, "sh_up", Is, H, eb, g) if sh else None,
        shared_down=qlin(seed, layer, "sh_down", H, Is, eb, g) if sh else None,
        shared_expert_gate=qlin(seed, layer, "seg", 1, H, rb, g) if sh else None,
        top_k=shape.top_k, norm_topk_prob=shape.norm_topk_prob)


def bf16_bits_to_torch(bits: np.ndarray, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def torch_bf16_to_bits(t) -> np.ndarray:
    import torch
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def widen_scales(lin):
    """The GPULinear with its fp16 scales and biases widened to f32 (exact)."""
    import torch
    from swiftlet_amd import _lib
    from swiftlet_amd.engine import GPULinear
    s = lin.scales.view(torch.float16).float().contiguous().view(torch.uint8)
    b = lin.biases.view(torch.float16).float().contiguous().view(torch.uint8)
    return GPULinear(lin.w, s, b, lin.out_dim, lin.in_dim, lin.group_size, lin.bits, _lib.SWQ_F32,
                     expert_stride_w=lin.expert_stride_w, expert_stride_sb=2 * lin.expert_stride_sb,
                     num_experts=lin.num_experts)


def widen_layer(layer):
    """The MoE layer with every matrix's scales and biases widened to f32."""
    from swiftlet_amd import moe
    w = lambda lin: widen_scales(lin) if lin is not None else None
    return moe.MoELayerGPU(router=w(layer.router), gate=w(layer.gate), up=w(layer.up), down=w(layer.down),
                           shared_gate=w(layer.shared_gate), shared_up=w(layer.shared_up),
                           shared_down=w(layer.shared_down), shared_expert_gate=w(layer.shared_expert_gate),
                           top_k=layer.top_k, norm_topk_prob=layer.norm_topk_prob)
