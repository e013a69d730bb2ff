"""The gated DeltaNet block between its input projections and out_proj,
restated from QwenCPUModel.deltaNetForward (QwenCPUModel.swift:371-496) —
TEST INFRASTRUCTURE ONLY (tests/ use it as the checker of swq_deltanet_step;
oracle/qwen_tiny.py runs the tiny model through it, which pins it to mlx's
fixtures).  float32 throughout, the reference's operation order where it
fixes one (separate multiply and add in the conv, the two norm scalings).

State carried across calls, as the reference's DecodeState holds it:
conv_tail [K-1, convD] (the last K-1 mixed rows, zeros on a fresh session,
:420-435) and state [nv, dv, dk] (the recurrent matrix per value head,
:452-479)."""

from __future__ import annotations

import numpy as np

from . import moe_ref as R

f32 = np.float32


def rms_norm(x, w, eps):
    """QwenCPUModel.rmsNorm (:47-59) over the last axis: x *= scale * w."""
    x = np.asarray(x, f32)
    ss = np.sum(x * x, axis=-1, keepdims=True, dtype=f32)
    scale = f32(1) / np.sqrt(ss / f32(x.shape[-1]) + f32(eps))
    return (x * (scale * w) if w is not None else x * scale).astype(f32)


def deinterleave(qkvz, ba, nk, nv, dk, dv):
    """The fused interleaved projections (qwen3_next, :386-410): per key head
    [q(dk), k(dk), v(rep*dv), z(rep*dv)] and [b(rep), a(rep)] -> mixed
    [S, q|k|v], z [S, nv*dv], b [S, nv], a [S, nv]."""
    qkvz, ba = np.asarray(qkvz, f32), np.asarray(ba, f32)
    S = qkvz.shape[0]
    rep = nv // nk
    keyD, valD = nk * dk, nv * dv
    chunk = 2 * dk + 2 * rep * dv
    mixed = np.zeros((S, 2 * keyD + valD), f32)
    z = np.zeros((S, valD), f32)
    b = np.zeros((S, nv), f32)
    a = np.zeros((S, nv), f32)
    for hk in range(nk):
        src = qkvz[:, hk * chunk:(hk + 1) * chunk]
        mixed[:, hk * dk:(hk + 1) * dk] = src[:, :dk]
        mixed[:, keyD + hk * dk:keyD + (hk + 1) * dk] = src[:, dk:2 * dk]
        for ri in range(rep):
            hv = hk * rep + ri
            mixed[:, 2 * keyD + hv * dv:2 * keyD + (hv + 1) * dv] = src[:, 2 * dk + ri * dv:2 * dk + (ri + 1) * dv]
            z[:, hv * dv:(hv + 1) * dv] = src[:, 2 * dk + rep * dv + ri * dv:2 * dk + rep * dv + (ri + 1) * dv]
        bsrc = ba[:, hk * 2 * rep:(hk + 1) * 2 * rep]
        b[:, hk * rep:(hk + 1) * rep] = bsrc[:, :rep]
        a[:, hk * rep:(hk + 1) * rep] = bsrc[:, rep:]
    return mixed, z, b, a


def deltanet_core(mixed, z, b, a, conv_w, a_log, dt_bias, norm_w, nk, nv, dk, dv, eps,
                  conv_tail=None, state=None):
    """Conv step + silu, q/k norms, the gated delta recurrence and the gated
    RMSNorm for S tokens (:412-493).  Returns (y [S, nv*dv] — the input of
    out_proj, conv_tail', state')."""
    mixed, z = np.asarray(mixed, f32), np.asarray(z, f32)
    S, convD = mixed.shape
    keyD, valD = nk * dk, nv * dv
    rep = nv // nk
    conv_w = np.asarray(conv_w, f32).reshape(convD, -1)
    K = conv_w.shape[1]
    tail = np.zeros((K - 1, convD), f32) if conv_tail is None else np.asarray(conv_tail, f32)
    padded = np.concatenate([tail, mixed], axis=0)
    conv = np.zeros((S, convD), f32)
    for s in range(S):  # acc += w[c, j] * padded[s + j, c], j = 0..K-1 (:424-431)
        acc = np.zeros(convD, f32)
        for j in range(K):
            acc = (acc + (conv_w[:, j] * padded[s + j]).astype(f32)).astype(f32)
        conv[s] = acc
    conv = R.silu(conv)
    new_tail = padded[-(K - 1):].copy() if K > 1 else np.zeros((0, convD), f32)
    qh = rms_norm(conv[:, :keyD].reshape(S, nk, dk), None, 1e-6)
    kh = rms_norm(conv[:, keyD:2 * keyD].reshape(S, nk, dk), None, 1e-6)
    vh = conv[:, 2 * keyD:].reshape(S, nv, dv)
    inv = f32(1) / np.sqrt(f32(dk))
    qh = (qh * (inv * inv)).astype(f32)
    kh = (kh * inv).astype(f32)
    a_log, dt_bias = np.asarray(a_log, f32), np.asarray(dt_bias, f32)
    st = np.zeros((nv, dv, dk), f32) if state is None else np.array(state, f32, copy=True)
    out = np.zeros((S, nv, dv), f32)
    hk_of = np.arange(nv) // rep
    b, a = np.asarray(b, f32), np.asarray(a, f32)
    for s in range(S):
        av = (a[s] + dt_bias).astype(f32)
        sp = np.where(av > 20, av, np.log1p(np.exp(np.minimum(av, 20)))).astype(f32)  # softplus (:63)
        g = np.exp(-np.exp(a_log) * sp).astype(f32)
        beta = R.sigmoid(b[s])
        kk, qq = kh[s, hk_of], qh[s, hk_of]  # [nv, dk]
        st = (st * g[:, None, None]).astype(f32)
        kv_mem = np.matmul(st, kk[:, :, None])[..., 0].astype(f32)
        delta = ((vh[s] - kv_mem) * beta[:, None]).astype(f32)
        st = (st + (kk[:, None, :] * delta[:, :, None]).astype(f32)).astype(f32)
        out[s] = np.matmul(st, qq[:, :, None])[..., 0]
    normed = rms_norm(out, np.asarray(norm_w, f32), eps).reshape(S, valD)
    y = (normed * R.silu(z)).astype(f32)
    return y, new_tail, st
