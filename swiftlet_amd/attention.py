"""Gated GQA attention (self_attn) on the device: q/k/v_proj
(swq_encode_gemv), the decode step (swq_attention_step) and o_proj — the
full-attention layer of QwenMetalModel.stepOneFast with its host-side core
(attnCoreCPU, QwenMetalModel.swift:922-951, :1086-1134) on the device,
numerics of QwenCPUModel.attentionForward (QwenCPUModel.swift:285-367).
torch supplies device memory and streams only."""

from __future__ import annotations

import ctypes

from . import _lib
from ._lib import AttentionLayer, check
from .engine import GPULinear, HipEngine, _stream_handle, _torch


class AttentionGPU:
    """One self_attn block: shapes, q/k norm weights (f32, device) and,
    optionally, its projections (q_proj, k_proj, v_proj) and o_proj."""

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int, rotary_dims: int, rope_theta: float,
                 eps: float, max_positions: int, q_norm_weight, k_norm_weight, projections=(),
                 o_proj: GPULinear | None = None, device="cuda"):
        torch = _torch()
        self.lib = _lib.load()
        self.H, self.KVH, self.hd = num_heads, num_kv_heads, head_dim
        self.rot, self.theta, self.eps, self.max_positions = rotary_dims, rope_theta, eps, max_positions
        f32 = dict(dtype=torch.float32, device=device)
        self.q_norm = torch.as_tensor(q_norm_weight, **f32).contiguous()
        self.k_norm = torch.as_tensor(k_norm_weight, **f32).contiguous()
        self.projections, self.o_proj = tuple(projections), o_proj
        self.device = device
        self._c = AttentionLayer(num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                                 rotary_dims=rotary_dims, rope_theta=rope_theta, norm_eps=eps,
                                 max_positions=max_positions, reserved=0, q_norm_weight=self.q_norm.data_ptr(),
                                 k_norm_weight=self.k_norm.data_ptr())

    def _bytes(self, fn, what):
        n = fn(ctypes.byref(self._c))
        if n == 0:
            raise _lib.SwqError(_lib.SWQ_ERR_INVALID_ARGUMENT, what)
        return n

    def new_cache(self):
        """An empty KV cache (k then v, f32 [max_positions, KVH, hd] each)."""
        torch = _torch()
        return torch.zeros(self._bytes(self.lib.swq_attention_cache_bytes, "attention_cache_bytes"),
                           dtype=torch.uint8, device=self.device)

    def cache_views(self, cache):
        torch = _torch()
        half = (self.max_positions * self.KVH * self.hd * 4 + 255) // 256 * 256
        n = self.max_positions * self.KVH * self.hd * 4
        shape = (self.max_positions, self.KVH, self.hd)
        return (cache[:n].view(torch.float32).reshape(shape), cache[half:half + n].view(torch.float32).reshape(shape))

    def new_workspace(self):
        torch = _torch()
        return torch.empty(self._bytes(self.lib.swq_attention_workspace_bytes, "attention_workspace_bytes"),
                           dtype=torch.uint8, device=self.device)

    def step(self, q_proj, k_proj, v_proj, cache, ws, position: int, out=None, stream=None):
        """One token from its projection outputs; returns the gated
        attention output [H*hd] and appends k, v to `cache`."""
        torch = _torch()
        if out is None:
            out = torch.empty(self.H * self.hd, dtype=torch.float32, device=q_proj.device)
        check(self.lib.swq_attention_step(ctypes.byref(self._c), q_proj.data_ptr(), k_proj.data_ptr(),
                                          v_proj.data_ptr(), cache.data_ptr(), cache.numel(), position,
                                          out.data_ptr(), ws.data_ptr(), ws.numel(), _stream_handle(stream)),
              "attention_step")
        return out

    def forward_token(self, engine: HipEngine, x, cache, ws, position: int, norm_weight=None, eps: float = 1e-6,
                      stream=None):
        """x [H_model] f32 -> the block's output: q/k/v_proj in one launch
        (with norm_weight, x is the un-normalised hidden state and the input
        RMSNorm runs inside that launch), the step, o_proj."""
        torch = _torch()
        pq, pk, pv = self.projections
        q = torch.empty(pq.out_dim, dtype=torch.float32, device=x.device)
        k = torch.empty(pk.out_dim, dtype=torch.float32, device=x.device)
        v = torch.empty(pv.out_dim, dtype=torch.float32, device=x.device)
        engine.encode_gemv_multi([pq, pk, pv], x, [q, k, v], norm_weight=norm_weight, eps=eps, stream=stream)
        att = self.step(q, k, v, cache, ws, position, stream=stream)
        r = torch.empty(self.o_proj.out_dim, dtype=torch.float32, device=x.device)
        engine.encode_gemv(self.o_proj, att, r, stream=stream)
        return r


def attention_from_checkpoint(ckpt, layer: int, config: dict, max_positions: int = 4096, device="cuda",
                              stream=None) -> AttentionGPU:
    """Layer `layer`'s self_attn block from a checkpoint; rope settings as
    QwenConfig reads them (QwenConfig.swift:80-88, :115)."""
    torch = _torch()
    p = f"model.layers.{layer}.self_attn."
    c = config.get("text_config", config)
    rp = c.get("rope_parameters") or {}
    theta = float(rp.get("rope_theta", c.get("rope_theta", 10_000_000)))
    factor = float(rp.get("partial_rotary_factor", c.get("partial_rotary_factor", 0.25)))
    hd = c["head_dim"]
    projs = [ckpt.gpu_linear(p + n, device=device, stream=stream) for n in ("q_proj", "k_proj", "v_proj")]

    def f32(name):
        return ckpt.load(p + name, device=device, stream=stream).to(torch.float32)

    return AttentionGPU(c["num_attention_heads"], c["num_key_value_heads"], hd, int(hd * factor), theta,
                        c.get("rms_norm_eps", 1e-6), max_positions, f32("q_norm.weight"), f32("k_norm.weight"),
                        projections=projs, o_proj=ckpt.gpu_linear(p + "o_proj", device=device, stream=stream),
                        device=device)
