"""Seeded synthetic MoE-layer weights and activations.

Every tensor element is a pure function of (seed, stream, index): the
``index``-th output of splitmix64 seeded with a per-stream key.  The same
function runs here (numpy, for host-side checks) and on the device
(``swq_synth_*`` in csrc/synth.hip, for the multi-GB bench stacks), and
both produce identical bits, so any slice of a device-generated stack can be
regenerated on the host.

Value distributions (the benchmark's synthetic inputs):
  4-bit codes   uniform 0..15, packed 8 per uint32 LSB-first (a uniform word)
  8-bit codes   uniform 0..255, packed 4 per uint32
  4-bit scales  fp16 of m * 2^-17, m uniform in [655, 2620]   (~U(0.005, 0.02))
  8-bit scales  fp16 of m * 2^-21, m uniform in [629, 2516]   (~U(0.0003, 0.0012))
  biases        -8 * scale (4-bit) or -128 * scale (8-bit), exact in fp16
  x             N(0, 1) from numpy's PCG64 stream, rounded to bf16 (RNE)
"""

from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15
C1 = 0xBF58476D1CE4E5B9
C2 = 0x94D049BB133111EB
STREAM_MUL = 0xD1B54A32D192ED03
KEY_ADD = 0x632BE59BD9B4E019

# scale distributions: (m_lo, m_count, exponent)
SCALE_PARAMS = {4: (655, 1966, 17), 8: (629, 1888, 21)}
BIAS_FACTOR_LOG2 = {4: 3, 8: 7}  # bias = -(2^f) * scale

# tensor streams within one layer (stream = layer * 16 + kind)
KIND = {
    "router_w": 0, "router_s": 1, "gate_w": 2, "gate_s": 3, "up_w": 4, "up_s": 5,
    "down_w": 6, "down_s": 7, "sh_gate_w": 8, "sh_gate_s": 9, "sh_up_w": 10,
    "sh_up_s": 11, "sh_down_w": 12, "sh_down_s": 13, "seg_w": 14, "seg_s": 15,
}


def _fin(z: np.ndarray) -> np.ndarray:
    """splitmix64 output function (Steele, Lea, Flood 2014)."""
    z = (z ^ (z >> np.uint64(30))) * np.uint64(C1)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(C2)
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream: int) -> int:
    z = (seed * GAMMA + stream * STREAM_MUL + KEY_ADD) & M64
    with np.errstate(over="ignore"):
        return int(_fin(np.array([z], dtype=np.uint64))[0])


def u32(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    """Elements start .. start+count-1 of a stream: the high 32 bits of
    splitmix64 output (index+1) for the stream key."""
    key = np.uint64(stream_key(seed, stream))
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = key + idx * np.uint64(GAMMA)
        return (_fin(z) >> np.uint64(32)).astype(np.uint32)


def scales_f16_bits(bits: int, r: np.ndarray) -> np.ndarray:
    lo, cnt, ex = SCALE_PARAMS[bits]
    m = (lo + (r % np.uint32(cnt))).astype(np.float32)
    return (m * np.float32(2.0 ** -ex)).astype(np.float16).view(np.uint16)


def biases_from_scales(bits: int, s_bits: np.ndarray) -> np.ndarray:
    """-(2^f) * s as fp16 bits: add f to the exponent, set the sign."""
    f = BIAS_FACTOR_LOG2[bits]
    return ((s_bits.astype(np.uint32) + (f << 10)) | 0x8000).astype(np.uint16)


def qmatrix(seed: int, layer: int, kind: str, experts: int | None, rows: int,
            cols: int, bits: int, group: int, expert_range: tuple[int, int] | None = None):
    """Codes, fp16 scale bits and fp16 bias bits of one (stacked) matrix.

    Returns (words, scales, biases) shaped [E?, rows, cols*bits/32] and
    [E?, rows, cols/group]; expert_range=(e0, e1) returns a slice of the
    stack with the same values the full stack holds there."""
    wpr = cols * bits // 32
    gpr = cols // group
    wkind, skind = KIND[kind + "_w"], KIND[kind + "_s"]
    if experts is None:
        w = u32(seed, layer * 16 + wkind, 0, rows * wpr).reshape(rows, wpr)
        s = scales_f16_bits(bits, u32(seed, layer * 16 + skind, 0, rows * gpr)).reshape(rows, gpr)
        return w, s, biases_from_scales(bits, s)
    e0, e1 = expert_range if expert_range is not None else (0, experts)
    n = e1 - e0
    w = u32(seed, layer * 16 + wkind, e0 * rows * wpr, n * rows * wpr).reshape(n, rows, wpr)
    s = scales_f16_bits(bits, u32(seed, layer * 16 + skind, e0 * rows * gpr, n * rows * gpr))
    s = s.reshape(n, rows, gpr)
    return w, s, biases_from_scales(bits, s)


def activations_bf16(seed: int, n: int, hidden: int) -> np.ndarray:
    """x ~ N(0, 1) rounded to bf16 (bits), [n, hidden]."""
    rng = np.random.default_rng(seed)
    f = rng.standard_normal((n, hidden), dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    return ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# --------------------------------------------------------------------------
# workload shapes


class MoEShape:
    """Shape of one MoE layer (hidden H, experts E, top-k K, intermediate I,
    shared intermediate Is, expert/shared bits, router/shared-gate bits)."""

    def __init__(self, name, hidden, experts, top_k, inter, shared_inter,
                 expert_bits=4, router_bits=8, group=64, norm_topk_prob=True):
        self.name = name
        self.hidden, self.experts, self.top_k = hidden, experts, top_k
        self.inter, self.shared_inter = inter, shared_inter
        self.expert_bits, self.router_bits, self.group = expert_bits, router_bits, group
        self.norm_topk_prob = norm_topk_prob

    def matrix_bytes(self, rows: int, cols: int, bits: int) -> int:
        """Packed codes + fp16 scale + fp16 bias per group."""
        return rows * cols * bits // 8 + rows * (cols // self.group) * 4

    def expert_bytes(self) -> int:
        H, I, b = self.hidden, self.inter, self.expert_bits
        return 2 * self.matrix_bytes(I, H, b) + self.matrix_bytes(H, I, b)

    @property
    def has_shared(self) -> bool:
        return self.shared_inter > 0

    def shared_bytes(self) -> int:
        if not self.has_shared:
            return 0
        H, I, b = self.hidden, self.shared_inter, self.expert_bits
        return 2 * self.matrix_bytes(I, H, b) + self.matrix_bytes(H, I, b)

    def router_bytes(self) -> int:
        return self.matrix_bytes(self.experts, self.hidden, self.router_bits)

    def seg_bytes(self) -> int:
        return self.matrix_bytes(1, self.hidden, self.router_bits) if self.has_shared else 0

    def decode_bytes(self, unique_experts: int, batch: int = 1) -> int:
        """Algorithmic HBM bytes of one decode step: every matrix touched once
        plus bf16 x in and bf16 out (intermediates excluded)."""
        return (unique_experts * self.expert_bytes() + self.shared_bytes()
                + self.router_bytes() + self.seg_bytes() + batch * self.hidden * 2 * 2)


SHAPES = {
    "qwen3.6-35b-a3b-q4": MoEShape("qwen3.6-35b-a3b-q4", 2048, 256, 8, 512, 512, 4),
    "qwen3-next-80b-a3b-q4": MoEShape("qwen3-next-80b-a3b-q4", 2048, 512, 10, 512, 512, 4),
    "qwen3.6-35b-a3b-q8": MoEShape("qwen3.6-35b-a3b-q8", 2048, 256, 8, 512, 512, 8),
    # one routed SwiGLU expert at the 35B shape (x [2048], gate/up [512 x 2048],
    # down [2048 x 512], 4-bit): a one-expert router (1 x 2048, 8-bit) picks it
    # with weight 1, no shared expert
    "single-expert-q4": MoEShape("single-expert-q4", 2048, 1, 1, 512, 0, 4),
}


# --------------------------------------------------------------------------
# skewed expert load for the prefill workload

ZIPF_S = 1.1
# Calibrated at the 35B shape with 512 tokens of N(0, 1) x: the realised
# per-expert pair counts, ordered by rank, fall off as rank^-1.09 over ranks
# 4..64 (239 of 256 experts touched, 266 tiles of 64 rows).
ZIPF_TAU = 1.4


def zipf_logit_bias(seed: int, experts: int, s: float = ZIPF_S, tau: float = ZIPF_TAU) -> np.ndarray:
    """Per-expert router-logit bias b_e = -tau * s * ln(rank_e), with rank a
    seeded permutation of 1..E: added to the logits before the softmax, it
    skews the per-expert token counts towards Zipf(s)."""
    rank = np.random.default_rng(seed).permutation(experts) + 1
    return (-tau * s * np.log(rank)).astype(np.float32)
