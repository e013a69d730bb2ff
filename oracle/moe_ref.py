"""CPU oracle for the MoE-layer decode path — TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the reference's CPU path for one MoE layer:
MLX affine dequantisation, the quantized GEMV forms, softmax, insertion
top-k, renormalisation, SwiGLU experts, the sigmoid-gated shared expert and
the weighted combine.  It is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and never as the thing measured or shipped.

Reference functions restated here (paths relative to the Swiftlet repo):

  dequantize        Sources/SwiftletCore/Checkpoint.swift:168-209
  scales_to_f32     Sources/SwiftletCore/Checkpoint.swift:229-244
  gemv_affine       Sources/SwiftletCore/Kernels.metal.txt:39-77 (factored form)
  gemv_kat_brute    Tests/SwiftletCoreTests/MetalKernelTests.swift:33-48
  softmax_row       Sources/SwiftletCore/QwenCPUModel.swift:65-71
  topk_insertion    Sources/SwiftletCore/QwenCPUModel.swift:508-522
                    (same algorithm: QwenMetalModel.swift:875-892)
  silu / sigmoid    Sources/SwiftletCore/QwenCPUModel.swift:61-62
  moe_forward       Sources/SwiftletCore/QwenCPUModel.swift:500-569

Pinning (each function is checked by tests/test_oracle_*.py):
  dequantize      closed form s*(q-8) exact; mlx-quantized tiny model end to end
  gemv_affine     regenerated LCG known-answer test; float64 brute force;
                  closed forms (all codes 8 -> 0, one-hot x -> a column)
  softmax/top-k   invariants, float64 brute-force argsort on (-p, id)
  moe_forward     mlx fixtures tiny_forward*.safetensors through the tiny
                  model forward in oracle/qwen_tiny.py; float64 brute force
"""

from __future__ import annotations

import numpy as np

F32, F16, BF16 = 0, 1, 2


# --------------------------------------------------------------------------
# formats


def unpack_codes(words: np.ndarray, bits: int) -> np.ndarray:
    """Codes of packed uint32 words, LSB-first (Checkpoint.swift:195-204).

    words [..., W] uint32 -> codes [..., W * 32/bits] uint32.
    """
    per = 32 // bits
    mask = np.uint32((1 << bits) - 1)
    shifts = (np.arange(per, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    w = np.asarray(words, dtype=np.uint32)
    codes = (w[..., None] >> shifts) & mask
    return codes.reshape(*w.shape[:-1], w.shape[-1] * per)


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of unpack_codes (used to build closed-form test inputs)."""
    per = 32 // bits
    c = np.asarray(codes, dtype=np.uint32)
    c = c.reshape(*c.shape[:-1], c.shape[-1] // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    """BF16 -> f32 is `u << 16` (Checkpoint.swift:237-240)."""
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits_rne(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (finite inputs)."""
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    return ((u + r) >> 16).astype(np.uint16)


def f32_to_bf16_bits_trunc(f: np.ndarray) -> np.ndarray:
    """Truncating f32 -> bf16 (MetalKernelTests.swift:18)."""
    return (np.asarray(f, dtype=np.float32).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def scales_to_f32(raw: np.ndarray, stype: int) -> np.ndarray:
    """Decode a scale/bias tensor to f32 (Checkpoint.swift:229-244)."""
    if stype == F32:
        return np.asarray(raw).view(np.float32) if np.asarray(raw).dtype != np.float32 else np.asarray(raw)
    if stype == F16:
        return np.asarray(raw).view(np.float16).astype(np.float32)
    if stype == BF16:
        return bf16_bits_to_f32(np.asarray(raw).view(np.uint16))
    raise ValueError(f"unsupported scales type {stype}")


def dequantize(words: np.ndarray, scales: np.ndarray, biases: np.ndarray,
               bits: int, group: int, stype: int = F32) -> np.ndarray:
    """MLX affine dequantisation, Checkpoint.swift:168-209.

    w[r, i] = scale[r, i/group] * q + bias[r, i/group], computed in f32 as a
    multiply followed by an add (two roundings, no fused multiply-add).
    words [..., rows, in*bits/32]; scales/biases [..., rows, in/group].
    """
    if bits not in (4, 8):
        raise ValueError(f"unsupported bits {bits}")  # Checkpoint.swift:170
    q = unpack_codes(words, bits).astype(np.float32)
    s = np.repeat(scales_to_f32(scales, stype), group, axis=-1)
    b = np.repeat(scales_to_f32(biases, stype), group, axis=-1)
    prod = (s * q).astype(np.float32)
    return (prod + b).astype(np.float32)


# --------------------------------------------------------------------------
# GEMV forms


def gemv_affine(x: np.ndarray, words: np.ndarray, scales: np.ndarray,
                biases: np.ndarray, bits: int, group: int, stype: int = F32,
                dtype=np.float64) -> np.ndarray:
    """Factored GEMV of Kernels.metal.txt:56-75:
    y[o] = sum_g s[o,g]*sum_{i in g} q_i x_i + b[o,g]*sum_{i in g} x_i,
    evaluated in `dtype` (float64 by default: the brute-force value)."""
    q = unpack_codes(words, bits).astype(dtype)
    rows, n = q.shape
    xs = np.asarray(x, dtype=dtype)
    G = n // group
    qdot = (q * xs[None, :]).reshape(rows, G, group).sum(-1)
    xsum = xs.reshape(G, group).sum(-1)
    s = scales_to_f32(scales, stype).astype(dtype).reshape(rows, G)
    b = scales_to_f32(biases, stype).astype(dtype).reshape(rows, G)
    return (s * qdot + b * xsum[None, :]).sum(-1)


def gemv_kat_brute(x: np.ndarray, words: np.ndarray, scale_at: np.ndarray,
                   bias_at: np.ndarray, bits: int, group: int) -> np.ndarray:
    """The known-answer test's CPU reference, MetalKernelTests.swift:33-48:
    per element (scale*q + bias) * x accumulated in f32, in input order."""
    q = unpack_codes(words, bits).astype(np.float32)
    rows, n = q.shape
    s = np.repeat(np.asarray(scale_at, np.float32).reshape(rows, -1), group, axis=1)
    b = np.repeat(np.asarray(bias_at, np.float32).reshape(rows, -1), group, axis=1)
    w = ((s * q).astype(np.float32) + b).astype(np.float32)
    terms = (w * np.asarray(x, np.float32)[None, :]).astype(np.float32)
    # sequential f32 accumulation, i = 0 .. n-1
    return np.cumsum(terms, axis=1, dtype=np.float32)[:, -1]


# --------------------------------------------------------------------------
# router


def sigmoid(v):
    """QwenCPUModel.swift:61: 1 / (1 + expf(-v)) in f32."""
    v = np.asarray(v, dtype=np.float32)
    return (np.float32(1) / (np.float32(1) + np.exp(-v))).astype(np.float32)


def silu(v):
    """QwenCPUModel.swift:62: v * sigmoid(v) in f32."""
    v = np.asarray(v, dtype=np.float32)
    return (v * sigmoid(v)).astype(np.float32)


def softmax_row(logits: np.ndarray) -> np.ndarray:
    """QwenCPUModel.swift:65-71: max-subtract, expf, sequential sum, divide."""
    l = np.asarray(logits, dtype=np.float32)
    m = l.max()
    e = np.exp((l - m).astype(np.float32)).astype(np.float32)
    s = np.cumsum(e, dtype=np.float32)[-1]
    return (e / s).astype(np.float32)


def topk_insertion(p: np.ndarray, k: int) -> list[tuple[int, float]]:
    """Insertion top-k of QwenCPUModel.swift:510-520.

    Append and stable-sort by probability (descending) while fewer than k
    picks are held; afterwards replace the last pick only when p is strictly
    larger.  The result is ordered by probability, ties to the lower id.
    """
    picks: list[tuple[int, float]] = []
    for e in range(len(p)):
        pe = float(p[e])
        if len(picks) < k:
            picks.append((e, pe))
            picks.sort(key=lambda t: -t[1])  # Python sort is stable
        elif pe > picks[k - 1][1]:
            picks[k - 1] = (e, pe)
            picks.sort(key=lambda t: -t[1])
    return picks


def topk_bruteforce(logits: np.ndarray, k: int) -> np.ndarray:
    """Float64 top-k: stable argsort on (-p, id), the order insertion top-k
    produces.  Used to pin topk_insertion."""
    l = np.asarray(logits, dtype=np.float64)
    p = np.exp(l - l.max())
    p /= p.sum()
    return np.lexsort((np.arange(len(p)), -p))[:k]


def renormalise(picks: list[tuple[int, float]], norm_topk_prob: bool) -> np.ndarray:
    """QwenCPUModel.swift:546-550: w = p / sum_topk p when norm_topk_prob."""
    ps = np.array([p for _, p in picks], dtype=np.float32)
    if not norm_topk_prob:
        return ps
    total = np.cumsum(ps, dtype=np.float32)[-1]
    return (ps / total).astype(np.float32)


# --------------------------------------------------------------------------
# the layer


class QLinear:
    """A quantized (possibly expert-stacked) matrix held on the host.

    words [E?, rows, in*bits/32] uint32; scales/biases [E?, rows, in/group]
    raw (f32 array or uint16 bits for f16/bf16)."""

    def __init__(self, words, scales, biases, bits, group, stype):
        self.words = np.ascontiguousarray(words, dtype=np.uint32)
        self.scales = np.ascontiguousarray(scales)
        self.biases = np.ascontiguousarray(biases)
        self.bits, self.group, self.stype = bits, group, stype

    @property
    def stacked(self) -> bool:
        return self.words.ndim == 3

    @property
    def out_dim(self) -> int:
        return self.words.shape[-2]

    @property
    def in_dim(self) -> int:
        return self.words.shape[-1] * (32 // self.bits)

    def dense(self, expert: int | None = None) -> np.ndarray:
        """Dequantised f32 rows (of one expert when stacked)."""
        if expert is None:
            return dequantize(self.words, self.scales, self.biases, self.bits, self.group, self.stype)
        return dequantize(self.words[expert], self.scales[expert], self.biases[expert],
                          self.bits, self.group, self.stype)


class MoELayerRef:
    """Host copy of one MoE layer's weights (QwenCPUModel.MoEWeights,
    QwenCPUModel.swift:95-101).  The router, shared expert and shared gate
    are dequantised once, as the CPU model caches dense layer weights
    (QwenCPUModel.swift:129-177); routed experts stay quantized and are
    dequantised on every call (:524-535)."""

    def __init__(self, router: QLinear, gate: QLinear, up: QLinear, down: QLinear,
                 shared_gate: QLinear | None, shared_up: QLinear | None,
                 shared_down: QLinear | None, shared_expert_gate: QLinear | None,
                 top_k: int, norm_topk_prob: bool = True):
        self.router, self.gate, self.up, self.down = router, gate, up, down
        self.shared_gate, self.shared_up, self.shared_down = shared_gate, shared_up, shared_down
        self.shared_expert_gate = shared_expert_gate
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        self.router_dense = router.dense()
        self.has_shared = shared_gate is not None
        if self.has_shared:
            self.sg_dense = shared_gate.dense()
            self.su_dense = shared_up.dense()
            self.sd_dense = shared_down.dense()
            self.seg_dense = shared_expert_gate.dense().reshape(-1)

    @property
    def num_experts(self) -> int:
        return self.router.out_dim


def moe_forward(x: np.ndarray, layer: MoELayerRef, dtype=np.float32, logit_bias=None):
    """QwenCPUModel.moeForward (QwenCPUModel.swift:500-569) for S tokens.

    ``logit_bias`` ([E] f32, optional) is added to every token's router
    logits before the softmax: the synthetic skewed-load workload of the
    prefill benchmark, with no counterpart in the reference (None = the
    reference's computation).

    Returns (out [S, H], picks per token, combine weights [S, K]).
    With dtype=np.float32 this follows the reference's f32 arithmetic; with
    np.float64 every product and sum after dequantisation is float64 (the
    brute-force value).  Routing is always decided by the f32 path's
    probabilities, so both dtypes evaluate the same experts.
    """
    x = np.atleast_2d(np.asarray(x, dtype=np.float32))
    S, H = x.shape
    K = layer.top_k
    router32 = (x @ layer.router_dense.T).astype(np.float32)            # :506
    if logit_bias is not None:
        router32 = router32 + np.asarray(logit_bias, dtype=np.float32)
    picks_per_row = []
    for s in range(S):                                                   # :508-522
        p = softmax_row(router32[s])
        picks_per_row.append(topk_insertion(p, K))

    expert_w = {}                                                        # :524-535
    for picks in picks_per_row:
        for e, _ in picks:
            if e not in expert_w:
                expert_w[e] = (layer.gate.dense(e), layer.up.dense(e), layer.down.dense(e))

    out = np.zeros((S, H), dtype=dtype)
    weights = np.zeros((S, K), dtype=np.float32)
    for s in range(S):                                                   # :544-567
        picks = picks_per_row[s]
        if dtype == np.float32:
            wts = renormalise(picks, layer.norm_topk_prob)
        else:
            ps = np.array([p for _, p in picks], dtype=np.float64)
            wts = ps / ps.sum() if layer.norm_topk_prob else ps
        weights[s] = wts
        xs = x[s].astype(dtype)
        for (e, _), wk in zip(picks, wts):
            g_w, u_w, d_w = (m.astype(dtype) for m in expert_w[e])
            g = g_w @ xs
            u = u_w @ xs
            h = _silu(g, dtype) * u
            d = d_w @ h
            out[s] += dtype(wk) * d
        if layer.has_shared:
            g = layer.sg_dense.astype(dtype) @ xs
            u = layer.su_dense.astype(dtype) @ xs
            h = _silu(g, dtype) * u
            d = layer.sd_dense.astype(dtype) @ h
            sg = layer.seg_dense.astype(dtype) @ xs
            out[s] += _sigmoid(sg, dtype) * d
    return out, picks_per_row, weights


def _sigmoid(v, dtype):
    if dtype == np.float32:
        return sigmoid(v)
    return 1.0 / (1.0 + np.exp(-np.asarray(v, dtype=np.float64)))


def _silu(v, dtype):
    if dtype == np.float32:
        return silu(v)
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def router_margin(x: np.ndarray, layer: MoELayerRef, logit_bias=None) -> np.ndarray:
    """Per token: float64 gap between the k-th and (k+1)-th router logits
    (plus ``logit_bias`` as in moe_forward).

    Expert selection is compared bit for bit only where this margin exceeds
    the f32 summation-order noise of the router GEMV."""
    x = np.atleast_2d(np.asarray(x, dtype=np.float64))
    l = x @ layer.router_dense.T.astype(np.float64)
    if logit_bias is not None:
        l = l + np.asarray(logit_bias, dtype=np.float32).astype(np.float64)
    srt = -np.sort(-l, axis=1)
    K = layer.top_k
    if K >= l.shape[1]:
        return np.full(l.shape[0], np.inf)
    return srt[:, K - 1] - srt[:, K]


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
