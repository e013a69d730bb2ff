"""The MoE-layer operator over the C ABI.

``MoELayerGPU`` holds one layer's device-resident weights (QwenMetalModel's
MoEGPU, QwenMetalModel.swift:34-39) and runs the decode step with
``swq_moe_decode``: router, softmax, top-k, renormalisation, SwiGLU experts,
sigmoid-gated shared expert and weighted combine, in one launch for a single
token and three for batches (replacing moeForward / routerPicks /
encodePendingMoE, QwenMetalModel.swift:609-716, 798-892).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, synth
from ._lib import SWQ_BF16, SWQ_F16, SWQ_F32, MoELayer, QLinear, check
from .engine import GPULinear, _stream_handle, _torch


def _empty_linear() -> QLinear:
    return QLinear()


class MoELayerGPU:
    def __init__(self, router: GPULinear, gate: GPULinear, up: GPULinear, down: GPULinear,
                 shared_gate: GPULinear | None, shared_up: GPULinear | None,
                 shared_down: GPULinear | None, shared_expert_gate: GPULinear | None,
                 top_k: int, norm_topk_prob: bool = True):
        self.router, self.gate, self.up, self.down = router, gate, up, down
        self.shared_gate, self.shared_up, self.shared_down = shared_gate, shared_up, shared_down
        self.shared_expert_gate = shared_expert_gate
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        self.hidden = router.in_dim
        self.num_experts = router.out_dim
        self.moe_intermediate = gate.out_dim
        self.has_shared = shared_gate is not None
        self.shared_intermediate = shared_gate.out_dim if self.has_shared else 0
        self.lib = _lib.load()
        self._c = self._make_c()

    def _make_c(self) -> MoELayer:
        has = self.has_shared
        return MoELayer(
            router=self.router.c(), gate=self.gate.c(), up=self.up.c(), down=self.down.c(),
            shared_gate=self.shared_gate.c() if has else _empty_linear(),
            shared_up=self.shared_up.c() if has else _empty_linear(),
            shared_down=self.shared_down.c() if has else _empty_linear(),
            shared_expert_gate=self.shared_expert_gate.c() if has else _empty_linear(),
            hidden=self.hidden, num_experts=self.num_experts, top_k=self.top_k,
            moe_intermediate=self.moe_intermediate, shared_intermediate=self.shared_intermediate,
            norm_topk_prob=1 if self.norm_topk_prob else 0, has_shared=1 if has else 0, reserved=0)

    # -- workspace -----------------------------------------------------
    def workspace_bytes(self, batch: int) -> int:
        n = self.lib.swq_moe_decode_workspace_bytes(ctypes.byref(self._c), batch)
        if n == 0:
            raise _lib.SwqError(_lib.SWQ_ERR_INVALID_ARGUMENT, "moe_decode_workspace_bytes")
        return n

    def new_workspace(self, batch: int, stream=None):
        torch = _torch()
        n = self.workspace_bytes(batch)
        ws = torch.empty(n, dtype=torch.uint8, device=self.router.w.device)
        check(self.lib.swq_moe_workspace_init(ws.data_ptr(), n, _stream_handle(stream)), "workspace_init")
        return ws

    # -- decode --------------------------------------------------------
    def workspace_error(self, ws, batch: int = 1) -> int:
        """The word the single-launch path sets if one of its bounded waits ran
        out (0 when every call so far completed normally); leaves it as it is."""
        off = self.lib.swq_moe_workspace_error_offset(ctypes.byref(self._c), batch)
        return int(ws[off:off + 4].cpu().numpy().view(np.uint32)[0])

    def workspace_status(self, ws, clear: bool = True, stream=None) -> int:
        """swq_moe_workspace_status: SWQ_OK, or SWQ_ERR_STALLED when a call on
        this workspace since the last check ran out of one of its bounded
        waits (its outputs are then invalid).  Blocks until the stream's
        earlier work is done; clears the record unless ``clear`` is False."""
        return self.lib.swq_moe_workspace_status(ws.data_ptr(), ws.numel(), 1 if clear else 0,
                                                 _stream_handle(stream))

    def decode(self, x, out=None, out_dtype=None, ws=None, accumulate: bool = False,
               topk_ids=None, topk_weights=None, stream=None, path: str = "auto"):
        """One decode step for x [B, H] (bf16 or f32 device tensor).

        ``path``: "auto" (swq_moe_decode: one launch when the layer and batch
        allow, else three), "staged" (the three launches) or "fused" (the
        single launch; raises SwqError LIMIT when it cannot take the call).
        Without ``ws`` the call makes a workspace and reads its stall record
        afterwards (blocking; SwqError STALLED if a bounded wait ran out);
        with ``ws`` the caller reads it with workspace_status.
        Returns (out [B, H], topk_ids [B, K] int32, topk_weights [B, K] f32)."""
        torch = _torch()
        if x.dim() == 1:
            x = x.unsqueeze(0)
        B = x.shape[0]
        x_dtype = {torch.bfloat16: SWQ_BF16, torch.float32: SWQ_F32}[x.dtype]
        if out is None:
            odt = out_dtype or torch.float32
            out = torch.empty((B, self.hidden), dtype=odt, device=x.device)
        o_dtype = {torch.bfloat16: SWQ_BF16, torch.float32: SWQ_F32}[out.dtype]
        own_ws = ws is None
        if own_ws:
            ws = self.new_workspace(B, stream)
        if topk_ids is None:
            topk_ids = torch.empty((B, self.top_k), dtype=torch.int32, device=x.device)
        if topk_weights is None:
            topk_weights = torch.empty((B, self.top_k), dtype=torch.float32, device=x.device)
        args = (ctypes.byref(self._c), x.data_ptr(), x_dtype, B, out.data_ptr(), o_dtype,
                topk_ids.data_ptr(), topk_weights.data_ptr(), ws.data_ptr(), ws.numel(),
                _lib.SWQ_MOE_ACCUMULATE if accumulate else 0)
        if path == "auto":
            check(self.lib.swq_moe_decode(*args, _stream_handle(stream)), "moe_decode")
        else:
            mask = {"staged": 7, "fused": _lib.SWQ_STAGES_FUSED}[path]
            check(self.lib.swq_moe_decode_stages(*args, mask, _stream_handle(stream)), f"moe_decode ({path})")
        if own_ws:
            # a workspace made for this call: its stall record is read here
            # (blocking), as no caller can read it later
            check(self.workspace_status(ws, stream=stream), "moe_decode")
        return out, topk_ids, topk_weights

    def decode_norm(self, h, norm_weight, eps: float, residual=None, out=None, ws=None, topk_ids=None,
                    topk_weights=None, stream=None):
        """One token's MoE step with the residual add and the post-attention
        RMSNorm in the same launch (swq_moe_decode_norm): h1 = h + residual,
        out = h1 + moe(rmsnorm(h1) * norm_weight).  h, residual, out: f32
        [H] device tensors; out must be a different buffer from h and
        residual.  Returns (out, topk_ids [1, K], topk_weights [1, K])."""
        torch = _torch()
        h = h.reshape(-1)
        if out is None:
            out = torch.empty(self.hidden, dtype=torch.float32, device=h.device)
        own_ws = ws is None
        if own_ws:
            ws = self.new_workspace(1, stream)
        if topk_ids is None:
            topk_ids = torch.empty((1, self.top_k), dtype=torch.int32, device=h.device)
        if topk_weights is None:
            topk_weights = torch.empty((1, self.top_k), dtype=torch.float32, device=h.device)
        wdt = {torch.float32: SWQ_F32, torch.float16: _lib.SWQ_F16, torch.bfloat16: SWQ_BF16}[norm_weight.dtype]
        check(self.lib.swq_moe_decode_norm(ctypes.byref(self._c), h.data_ptr(),
                                           residual.data_ptr() if residual is not None else None,
                                           norm_weight.data_ptr(), wdt, eps, out.data_ptr(), topk_ids.data_ptr(),
                                           topk_weights.data_ptr(), ws.data_ptr(), ws.numel(),
                                           _stream_handle(stream)), "moe_decode_norm")
        if own_ws:
            check(self.workspace_status(ws, stream=stream), "moe_decode_norm")
        return out, topk_ids, topk_weights

    # -- prefill -------------------------------------------------------
    def prefill_workspace_bytes(self, tokens: int) -> int:
        n = self.lib.swq_moe_prefill_workspace_bytes(ctypes.byref(self._c), tokens)
        if n == 0:
            raise _lib.SwqError(_lib.SWQ_ERR_LIMIT, "moe_prefill_workspace_bytes")
        return n

    def new_prefill_workspace(self, tokens: int, stream=None):
        torch = _torch()
        n = self.prefill_workspace_bytes(tokens)
        ws = torch.empty(n, dtype=torch.uint8, device=self.router.w.device)
        check(self.lib.swq_moe_workspace_init(ws.data_ptr(), n, _stream_handle(stream)), "workspace_init")
        return ws

    def prefill(self, x, out=None, out_dtype=None, ws=None, accumulate: bool = False,
                topk_ids=None, topk_weights=None, logit_bias=None, stream=None):
        """The layer over x [T, H] (bf16 or f32 device tensor) with the pairs
        grouped by expert (swq_moe_prefill).  ``logit_bias`` (f32 [E] device
        tensor) adds a per-expert bias to the router logits before the
        softmax (swq_moe_prefill_biased, the skewed-load workload).
        Returns (out [T, H], topk_ids [T, K] int32, topk_weights [T, K] f32)."""
        torch = _torch()
        if x.dim() == 1:
            x = x.unsqueeze(0)
        T = x.shape[0]
        x_dtype = {torch.bfloat16: SWQ_BF16, torch.float32: SWQ_F32}[x.dtype]
        if out is None:
            out = torch.empty((T, self.hidden), dtype=out_dtype or torch.float32, device=x.device)
        o_dtype = {torch.bfloat16: SWQ_BF16, torch.float32: SWQ_F32}[out.dtype]
        if ws is None:
            ws = self.new_prefill_workspace(T, stream)
        if topk_ids is None:
            topk_ids = torch.empty((T, self.top_k), dtype=torch.int32, device=x.device)
        if topk_weights is None:
            topk_weights = torch.empty((T, self.top_k), dtype=torch.float32, device=x.device)
        head = (ctypes.byref(self._c), x.data_ptr(), x_dtype, T, out.data_ptr(), o_dtype,
                topk_ids.data_ptr(), topk_weights.data_ptr())
        tail = (ws.data_ptr(), ws.numel(), _lib.SWQ_MOE_ACCUMULATE if accumulate else 0,
                _stream_handle(stream))
        if logit_bias is None:
            check(self.lib.swq_moe_prefill(*head, *tail), "moe_prefill")
        else:
            assert logit_bias.dtype == torch.float32 and logit_bias.numel() == self.num_experts
            check(self.lib.swq_moe_prefill_biased(*head, logit_bias.data_ptr(), *tail), "moe_prefill_biased")
        return out, topk_ids, topk_weights

    def touched_bytes(self, unique_experts: int, batch: int = 1, x_bytes: int = 2,
                      out_bytes: int = 2) -> int:
        """Algorithmic HBM bytes of one decode step: every matrix read once,
        x in and out written once (intermediates excluded)."""
        n = unique_experts * (self.gate.matrix_bytes + self.up.matrix_bytes + self.down.matrix_bytes)
        n += self.router.matrix_bytes
        if self.has_shared:
            n += (self.shared_gate.matrix_bytes + self.shared_up.matrix_bytes
                  + self.shared_down.matrix_bytes + self.shared_expert_gate.matrix_bytes)
        return n + batch * self.hidden * (x_bytes + out_bytes)


# ---------------------------------------------------------------------------
# device-side synthetic layers


def synth_linear(seed: int, layer: int, kind: str, experts: int | None, rows: int, cols: int,
                 bits: int, group: int, device="cuda", stream=None) -> GPULinear:
    """A seeded synthetic quantized matrix generated on the device; equal,
    bit for bit, to synth.qmatrix on the host."""
    torch = _torch()
    lib = _lib.load()
    e = experts or 1
    wpr = cols * bits // 32
    gpr = cols // group
    nw = e * rows * wpr
    ns = e * rows * gpr
    w = torch.empty(nw * 4, dtype=torch.uint8, device=device)
    s = torch.empty(ns * 2, dtype=torch.uint8, device=device)
    b = torch.empty(ns * 2, dtype=torch.uint8, device=device)
    h = _stream_handle(stream)
    check(lib.swq_synth_u32(w.data_ptr(), nw, seed, layer * 16 + synth.KIND[kind + "_w"], 0, h), "synth_u32")
    check(lib.swq_synth_scales(s.data_ptr(), b.data_ptr(), ns, bits, seed,
                               layer * 16 + synth.KIND[kind + "_s"], 0, h), "synth_scales")
    stacked = experts is not None
    return GPULinear(w, s, b, rows, cols, group, bits, SWQ_F16,
                     expert_stride_w=rows * wpr * 4 if stacked else 0,
                     expert_stride_sb=rows * gpr * 2 if stacked else 0, num_experts=e)


def synth_layer(shape: synth.MoEShape, seed: int, layer: int, device="cuda", stream=None) -> MoELayerGPU:
    """One seeded synthetic MoE layer of the given shape, generated on the device."""
    H, E, I, Is = shape.hidden, shape.experts, shape.inter, shape.shared_inter
    eb, rb, g = shape.expert_bits, shape.router_bits, shape.group
    mk = lambda kind, ex, rows, cols, bits: synth_linear(seed, layer, kind, ex, rows, cols, bits, g, device, stream)
    sh = shape.has_shared
    return MoELayerGPU(
        router=mk("router", None, E, H, rb),
        gate=mk("gate", E, I, H, eb), up=mk("up", E, I, H, eb), down=mk("down", E, H, I, eb),
        shared_gate=mk("sh_gate", None, Is, H, eb) if sh else None,
        shared_up=mk("sh_up", None, Is, H, eb) if sh else None,
        shared_down=mk("sh_down", None, H, Is, eb) if sh else None,
        shared_expert_gate=mk("seg", None, 1, H, rb) if sh else None,
        top_k=shape.top_k, norm_topk_prob=shape.norm_topk_prob)


def host_layer_arrays(shape: synth.MoEShape, seed: int, layer: int, experts: list[int] | None = None):
    """Host copies (numpy) of the synthetic layer's tensors, as
    {name: (words, scale bits, bias bits, bits)}; ``experts`` restricts the
    stacked tensors to those expert ids (a dict per expert then)."""
    H, E, I, Is = shape.hidden, shape.experts, shape.inter, shape.shared_inter
    eb, rb, g = shape.expert_bits, shape.router_bits, shape.group
    out = {"router": synth.qmatrix(seed, layer, "router", None, E, H, rb, g) + (rb,)}
    if shape.has_shared:
        out.update({
            "sh_gate": synth.qmatrix(seed, layer, "sh_gate", None, Is, H, eb, g) + (eb,),
            "sh_up": synth.qmatrix(seed, layer, "sh_up", None, Is, H, eb, g) + (eb,),
            "sh_down": synth.qmatrix(seed, layer, "sh_down", None, H, Is, eb, g) + (eb,),
            "seg": synth.qmatrix(seed, layer, "seg", None, 1, H, rb, g) + (rb,),
        })
    if experts is None:
        for kind, rows, cols in (("gate", I, H), ("up", I, H), ("down", H, I)):
            out[kind] = synth.qmatrix(seed, layer, kind, E, rows, cols, eb, g) + (eb,)
    else:
        for kind, rows, cols in (("gate", I, H), ("up", I, H), ("down", H, I)):
            out[kind] = {e: tuple(a[0] for a in synth.qmatrix(seed, layer, kind, E, rows, cols, eb, g,
                                                            expert_range=(e, e + 1))) + (eb,)
                         for e in experts}
    return out
