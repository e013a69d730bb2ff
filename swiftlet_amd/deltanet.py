"""The gated DeltaNet block (linear_attn) on the device: the input
projections (swq_encode_gemv), the decode step (swq_deltanet_step) and
out_proj — QwenMetalModel.encDeltaLayer (QwenMetalModel.swift:989-1084) for
one token, numerics of QwenCPUModel.deltaNetForward (QwenCPUModel.swift:
371-496).  torch supplies device memory and streams only."""

from __future__ import annotations

import ctypes

from . import _lib
from ._lib import SWQ_DELTA_INTERLEAVED, SWQ_DELTA_SPLIT, DeltaNetLayer, check
from .engine import GPULinear, HipEngine, _stream_handle, _torch


class DeltaNetGPU:
    """One linear_attn block: shapes, small f32 parameters on the device,
    and (optionally) its projections.

    INTERLEAVED (qwen3_next): projections = (in_proj_qkvz, in_proj_ba).
    SPLIT (qwen3_5): projections = (in_proj_qkv, in_proj_z, in_proj_b,
    in_proj_a), whose outputs land as [q|k|v|z] and [b|a]."""

    def __init__(self, nk: int, nv: int, dk: int, dv: int, conv_kernel: int, layout: int, eps: float,
                 conv_weight, a_log, dt_bias, norm_weight, projections=(), out_proj: GPULinear | None = None,
                 device="cuda"):
        torch = _torch()
        self.lib = _lib.load()
        self.nk, self.nv, self.dk, self.dv, self.K = nk, nv, dk, dv, conv_kernel
        self.layout, self.eps = layout, eps
        self.key_dim, self.value_dim = nk * dk, nv * dv
        self.conv_dim = 2 * self.key_dim + self.value_dim
        f32 = dict(dtype=torch.float32, device=device)
        self.conv_weight = torch.as_tensor(conv_weight, **f32).reshape(-1).contiguous()
        self.a_log = torch.as_tensor(a_log, **f32).contiguous()
        self.dt_bias = torch.as_tensor(dt_bias, **f32).contiguous()
        self.norm_weight = torch.as_tensor(norm_weight, **f32).contiguous()
        assert self.conv_weight.numel() == self.conv_dim * conv_kernel and self.a_log.numel() == nv
        self.projections, self.out_proj = tuple(projections), out_proj
        self._c = DeltaNetLayer(
            num_key_heads=nk, num_value_heads=nv, key_head_dim=dk, value_head_dim=dv, conv_kernel=conv_kernel,
            layout=layout, norm_eps=eps, reserved=0, conv_weight=self.conv_weight.data_ptr(),
            a_log=self.a_log.data_ptr(), dt_bias=self.dt_bias.data_ptr(), norm_weight=self.norm_weight.data_ptr())

    @property
    def state_bytes(self) -> int:
        n = self.lib.swq_deltanet_state_bytes(ctypes.byref(self._c))
        if n == 0:
            raise _lib.SwqError(_lib.SWQ_ERR_INVALID_ARGUMENT, "deltanet_state_bytes")
        return n

    def new_state(self):
        """A fresh session's state (zeros), as a flat uint8 device tensor."""
        torch = _torch()
        return torch.zeros(self.state_bytes, dtype=torch.uint8, device=self.conv_weight.device)

    def state_views(self, state):
        """(conv ring [K, convD], recurrent state [nv, dv, dk]) views of a state buffer."""
        torch = _torch()
        ring_bytes = (self.K * self.conv_dim * 4 + 255) // 256 * 256
        ring = state[:self.K * self.conv_dim * 4].view(torch.float32).reshape(self.K, self.conv_dim)
        rec = state[ring_bytes:ring_bytes + self.nv * self.dv * self.dk * 4].view(torch.float32)
        return ring, rec.reshape(self.nv, self.dv, self.dk)

    def step(self, qkvz, ba, state, position: int, out=None, stream=None):
        """One token from its projection outputs; returns the gated-normed
        output [nv*dv] (f32) and updates `state`."""
        torch = _torch()
        assert qkvz.dtype == torch.float32 and ba.dtype == torch.float32
        assert qkvz.numel() >= self.conv_dim + self.value_dim and ba.numel() >= 2 * self.nv
        if out is None:
            out = torch.empty(self.value_dim, dtype=torch.float32, device=qkvz.device)
        check(self.lib.swq_deltanet_step(ctypes.byref(self._c), qkvz.data_ptr(), ba.data_ptr(), state.data_ptr(),
                                         state.numel(), position, out.data_ptr(), _stream_handle(stream)),
              "deltanet_step")
        return out

    def forward_token(self, engine: HipEngine, x, state, position: int, norm_weight=None, eps: float = 1e-6,
                      stream=None):
        """x [H] f32 -> the block's output [H]: the input projections in one
        launch (with norm_weight, x is the un-normalised hidden state and the
        input RMSNorm runs inside that launch), the step, out_proj."""
        torch = _torch()
        dev = x.device
        qkvz = torch.empty(self.conv_dim + self.value_dim, dtype=torch.float32, device=dev)
        ba = torch.empty(2 * self.nv, dtype=torch.float32, device=dev)
        if self.layout == SWQ_DELTA_INTERLEAVED:
            ys = [qkvz, ba]
        else:
            ys = [qkvz.data_ptr(), qkvz.data_ptr() + 4 * self.conv_dim, ba.data_ptr(), ba.data_ptr() + 4 * self.nv]
        engine.encode_gemv_multi(list(self.projections), x, ys, norm_weight=norm_weight, eps=eps, stream=stream)
        y = self.step(qkvz, ba, state, position, stream=stream)
        r = torch.empty(self.out_proj.out_dim, dtype=torch.float32, device=dev)
        engine.encode_gemv(self.out_proj, y, r, stream=stream)
        return r


def deltanet_from_checkpoint(ckpt, layer: int, config: dict, device="cuda", stream=None) -> DeltaNetGPU:
    """Layer `layer`'s linear_attn block from a checkpoint (swiftlet_amd.
    checkpoint.Checkpoint): the projections resident, the small parameters
    as f32.  The layout follows QwenConfig (QwenConfig.swift:103): split when
    the checkpoint holds in_proj_qkv, interleaved otherwise."""
    torch = _torch()
    p = f"model.layers.{layer}.linear_attn."
    split = ckpt.contains(p + "in_proj_qkv.weight")
    names = ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a") if split else ("in_proj_qkvz", "in_proj_ba")
    projs = [ckpt.gpu_linear(p + n, device=device, stream=stream) for n in names]

    def f32(name):
        return ckpt.load(p + name, device=device, stream=stream).to(torch.float32)

    c = config
    return DeltaNetGPU(c["linear_num_key_heads"], c["linear_num_value_heads"], c["linear_key_head_dim"],
                       c["linear_value_head_dim"], c["linear_conv_kernel_dim"],
                       SWQ_DELTA_SPLIT if split else SWQ_DELTA_INTERLEAVED, c.get("rms_norm_eps", 1e-6),
                       f32("conv1d.weight"), f32("A_log"), f32("dt_bias"), f32("norm.weight"),
                       projections=projs, out_proj=ckpt.gpu_linear(p + "out_proj", device=device, stream=stream),
                       device=device)
