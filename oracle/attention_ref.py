"""Gated full attention (the GQA layers) between q/k/v_proj and o_proj,
restated from QwenCPUModel.attentionForward (QwenCPUModel.swift:285-345)
and applyRope (:348-367) — TEST INFRASTRUCTURE ONLY (tests/ use it as the
checker of swq_attention_step; oracle/qwen_tiny.py runs the tiny model
through it, which pins it to mlx's fixtures).  float32 throughout.

The KV cache is carried across calls as the reference's DecodeState.kv
holds it: k and v rows appended per position, [positions, KVH, hd]."""

from __future__ import annotations

import numpy as np

from . import moe_ref as R
from .deltanet_ref import rms_norm

f32 = np.float32


def apply_rope(x, positions, rot: int, theta: float):
    """Partial NeoX RoPE on the first `rot` dims of each head (:348-367):
    invFreq = theta^(-2j/rot), angle = position * invFreq in float32.
    x [S, heads, hd]; positions [S]."""
    half = rot // 2
    j = np.arange(half)
    inv = np.power(f32(theta), (-(2 * j).astype(f32) / f32(rot)).astype(f32)).astype(f32)
    ang = (np.asarray(positions, f32)[:, None] * inv[None, :]).astype(f32)
    cs, sn = np.cos(ang).astype(f32)[:, None, :], np.sin(ang).astype(f32)[:, None, :]
    out = np.array(x, f32, copy=True)
    a, b = x[..., :half], x[..., half:rot]
    out[..., :half] = a * cs - b * sn
    out[..., half:rot] = b * cs + a * sn
    return out.astype(f32)


def attention_core(q_out, k, v, q_norm_w, k_norm_w, H: int, KVH: int, hd: int, rot: int, theta: float,
                   eps: float, cache_k=None, cache_v=None):
    """S new tokens after `past = len(cache_k)` cached positions: q_out
    [S, H*2*hd] (per head: query then output gate), k, v [S, KVH*hd].
    Returns (gated attention output [S, H*hd] — the input of o_proj,
    cache_k', cache_v')."""
    q_out = np.asarray(q_out, f32)
    S = q_out.shape[0]
    past = 0 if cache_k is None else cache_k.shape[0]
    qo = q_out.reshape(S, H, 2 * hd)
    q, gate = qo[..., :hd], qo[..., hd:].reshape(S, H * hd)
    k = np.asarray(k, f32).reshape(S, KVH, hd)
    v = np.asarray(v, f32).reshape(S, KVH, hd)
    q = rms_norm(q, np.asarray(q_norm_w, f32), eps)
    k = rms_norm(k, np.asarray(k_norm_w, f32), eps)
    pos = np.arange(past, past + S)
    q, k = apply_rope(q, pos, rot, theta), apply_rope(k, pos, rot, theta)
    ck = k if cache_k is None else np.concatenate([cache_k, k], axis=0)
    cv = v if cache_v is None else np.concatenate([cache_v, v], axis=0)
    scale = f32(1) / np.sqrt(f32(hd))
    out = np.zeros((S, H, hd), f32)
    group = H // KVH
    for h in range(H):
        kv = h // group
        for si in range(S):
            n = past + si + 1
            sc = ((ck[:n, kv, :] @ q[si, h, :]) * scale).astype(f32)
            pr = R.softmax_row(sc)
            out[si, h] = pr @ cv[:n, kv, :]
    out = (out.reshape(S, H * hd) * R.sigmoid(gate)).astype(f32)
    return out, ck, cv
