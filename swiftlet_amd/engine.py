"""Host-side mirror of SwiftletCore's quantized-matmul operator API over the
C ABI: ``GPULinear`` (MetalShardStore.swift:48-62 plus ExpertStack strides,
QwenMetalModel.swift:16-21) and ``HipEngine`` with the ``gemvQuantized`` /
``encodeGemv`` / ``encodeSiluMul`` entry points (MetalEngine.swift:95-232)
and ``Checkpoint``'s dequantisation (Checkpoint.swift:148-209).

torch provides device memory and streams; all arithmetic runs in libswq.so.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import SWQ_BF16, SWQ_F16, SWQ_F32, QLinear, SwqError, check


class NoDevice(SwqError):
    """MetalEngine.Error.noDevice (MetalEngine.swift:8-11)."""


def _torch():
    import torch
    return torch


def _stream_handle(stream) -> ctypes.c_void_p:
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def to_device_bytes(arr: np.ndarray, device="cuda"):
    """A contiguous host array as a flat uint8 device tensor."""
    torch = _torch()
    a = np.ascontiguousarray(arr)
    return torch.from_numpy(a.reshape(-1).view(np.uint8).copy()).to(device)


def scales_type_of(dtype_name: str) -> int:
    """ScalesType(dtype:) of MetalEngine.swift:72-79."""
    return {"F32": SWQ_F32, "F16": SWQ_F16, "BF16": SWQ_BF16}[dtype_name]


class GPULinear:
    """One device-resident quantized linear module, optionally an expert
    stack.  Non-owning in the C ABI; this object keeps the tensors alive."""

    def __init__(self, w, scales, biases, out_dim: int, in_dim: int, group_size: int, bits: int,
                 scales_type: int, w_off: int = 0, s_off: int = 0, b_off: int = 0,
                 expert_stride_w: int = 0, expert_stride_sb: int = 0, num_experts: int = 1):
        self.w, self.scales, self.biases = w, scales, biases
        self.out_dim, self.in_dim = out_dim, in_dim
        self.group_size, self.bits, self.scales_type = group_size, bits, scales_type
        self.w_off, self.s_off, self.b_off = w_off, s_off, b_off
        self.expert_stride_w, self.expert_stride_sb = expert_stride_w, expert_stride_sb
        self.num_experts = num_experts

    @property
    def matrix_bytes(self) -> int:
        """Packed codes + scales + biases of one matrix (one expert)."""
        sb = 4 if self.scales_type == SWQ_F32 else 2
        return (self.out_dim * self.in_dim * self.bits // 8
                + 2 * self.out_dim * (self.in_dim // self.group_size) * sb)

    def c(self) -> QLinear:
        return QLinear(
            w=self.w.data_ptr(), scales=self.scales.data_ptr(), biases=self.biases.data_ptr(),
            w_off=self.w_off, s_off=self.s_off, b_off=self.b_off,
            out_dim=self.out_dim, in_dim=self.in_dim, group_size=self.group_size, bits=self.bits,
            scales_type=self.scales_type, reserved=0,
            expert_stride_w=self.expert_stride_w, expert_stride_sb=self.expert_stride_sb)

    @classmethod
    def from_host(cls, words: np.ndarray, scales: np.ndarray, biases: np.ndarray, group_size: int,
                  bits: int, scales_type: int, device="cuda") -> "GPULinear":
        """Upload MLX-layout arrays: words [E?, rows, in*bits/32] uint32,
        scales/biases [E?, rows, in/group] (f32 array or 16-bit bit patterns)."""
        words = np.ascontiguousarray(words, dtype=np.uint32)
        stacked = words.ndim == 3
        e = words.shape[0] if stacked else 1
        rows = words.shape[-2]
        in_dim = words.shape[-1] * (32 // bits)
        sdt = np.float32 if scales_type == SWQ_F32 else np.uint16
        s_np = np.ascontiguousarray(scales).view(sdt)
        b_np = np.ascontiguousarray(biases).view(sdt)
        sbytes = 4 if scales_type == SWQ_F32 else 2
        assert s_np.size == e * rows * (in_dim // group_size) == b_np.size
        return cls(to_device_bytes(words, device), to_device_bytes(s_np, device),
                   to_device_bytes(b_np, device), rows, in_dim, group_size, bits, scales_type,
                   expert_stride_w=rows * in_dim * bits // 8 if stacked else 0,
                   expert_stride_sb=rows * (in_dim // group_size) * sbytes if stacked else 0,
                   num_experts=e)


class HipEngine:
    """Device owner with MetalEngine's operator entry points."""

    def __init__(self):
        self.lib = _lib.load()
        n = ctypes.c_int(0)
        st = self.lib.swq_device_count(ctypes.byref(n))
        if st != _lib.SWQ_OK:
            raise NoDevice(st, "HipEngine()")
        self.device_count = n.value

    # MetalEngine.gemvQuantized (MetalEngine.swift:190-232): blocking, host memory.
    def gemv_quantized(self, x, packed, scales, biases, out_dim: int, in_dim: int, group_size: int,
                       bits: int, scales_type: int, use_fast: bool = False) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        packed = np.ascontiguousarray(packed)
        scales = np.ascontiguousarray(scales)
        biases = np.ascontiguousarray(biases)
        y = np.zeros(out_dim, dtype=np.float32)
        check(self.lib.swq_gemv_quantized(
            x.ctypes.data, packed.ctypes.data, packed.nbytes, scales.ctypes.data, scales.nbytes,
            biases.ctypes.data, biases.nbytes, out_dim, in_dim, group_size, bits, scales_type,
            1 if use_fast else 0, y.ctypes.data), "gemv_quantized")
        return y

    # MetalEngine.encodeGemv (MetalEngine.swift:95-170): stream-ordered, fp32 x/y.
    def encode_gemv(self, lin: GPULinear, x, y, rows: int | None = None, w_extra: int = 0,
                    s_extra: int = 0, b_extra: int = 0, x_off: int = 0, y_off: int = 0, stream=None):
        torch = _torch()
        assert x.dtype == torch.float32 and y.dtype == torch.float32
        c = lin.c()
        check(self.lib.swq_encode_gemv(ctypes.byref(c), rows or 0, w_extra, s_extra, b_extra,
                                       x.data_ptr(), x_off, y.data_ptr(), y_off,
                                       _stream_handle(stream)), "encode_gemv")

    # encNormCopy + the projections' encodeGemv calls of one layer, one launch.
    def encode_gemv_multi(self, lins, x, ys, norm_weight=None, eps: float = 1e-6, stream=None):
        """ys[i] = W_i x (x: f32 device vector; ys: f32 device tensors or raw
        device addresses); with norm_weight, x is replaced by rmsnorm(x) *
        norm_weight inside the kernel."""
        torch = _torch()
        n = len(lins)
        arr = (QLinear * n)(*[l.c() for l in lins])
        ptrs = (ctypes.c_void_p * n)(*[y if isinstance(y, int) else y.data_ptr() for y in ys])
        wdt, wptr = SWQ_F32, None
        if norm_weight is not None:
            wdt = {torch.float32: SWQ_F32, torch.float16: SWQ_F16, torch.bfloat16: SWQ_BF16}[norm_weight.dtype]
            wptr = norm_weight.data_ptr()
        check(self.lib.swq_encode_gemv_multi(arr, n, ptrs, x.data_ptr(), wptr, wdt, eps, _stream_handle(stream)),
              "encode_gemv_multi")

    # MetalEngine.encodeSiluMul (MetalEngine.swift:172-187).
    def encode_silu_mul(self, buf, count: int, g_off: int, u_off: int, dst_off: int, stream=None):
        check(self.lib.swq_encode_silu_mul(buf.data_ptr(), count, g_off, u_off, dst_off,
                                           _stream_handle(stream)), "encode_silu_mul")

    # add_inplace + norm_copy (Kernels.metal.txt:425-452) around the MoE block
    # (QwenMetalModel.swift:938-951), numerics of QwenCPUModel.rmsNorm (:47-59).
    def rms_norm(self, h, weight, eps: float, residual=None, out=None, out_dtype=None, stream=None):
        """h [rows, dim] f32 device tensor: h += residual (in place, when
        given), then returns rmsnorm(h) * weight as out_dtype (f32 / bf16)."""
        torch = _torch()
        assert h.dtype == torch.float32 and h.is_contiguous()
        if h.dim() == 1:
            h = h.unsqueeze(0)
        rows, dim = h.shape
        if out is None:
            out = torch.empty((rows, dim), dtype=out_dtype or torch.float32, device=h.device)
        odt = {torch.float32: SWQ_F32, torch.bfloat16: SWQ_BF16}[out.dtype]
        wdt, wptr = SWQ_F32, None
        if weight is not None:
            wdt = {torch.float32: SWQ_F32, torch.float16: SWQ_F16, torch.bfloat16: SWQ_BF16}[weight.dtype]
            assert weight.numel() == dim
            wptr = weight.data_ptr()
        if residual is not None:
            assert residual.dtype == torch.float32 and residual.numel() == h.numel()
        check(self.lib.swq_rmsnorm(h.data_ptr(), residual.data_ptr() if residual is not None else None, wptr,
                                   wdt, eps, rows, dim, out.data_ptr(), odt, _stream_handle(stream)), "rmsnorm")
        return out

    # SwiftletSession.sample (SwiftletSession.swift:226-273) on the device.
    def new_sample_workspace(self, vocab: int, device="cuda"):
        torch = _torch()
        n = self.lib.swq_sample_workspace_bytes(vocab)
        if n == 0:
            raise SwqError(_lib.SWQ_ERR_LIMIT, "sample_workspace_bytes")
        return torch.zeros(n, dtype=torch.uint8, device=device)

    def sample(self, logits, temperature: float, top_k: int, top_p: float, presence: float = 0.0,
               frequency: float = 0.0, seen: dict | None = None, banned=(), u: float = 0.0, ws=None,
               stream=None) -> int:
        """The next token from f32 device logits [vocab]; u in [0, 1) is the
        draw's uniform number.  Blocking (reads the token back)."""
        torch = _torch()
        dev = logits.device
        vocab = logits.numel()
        if ws is None:
            ws = self.new_sample_workspace(vocab, dev)
        seen = seen or {}
        ids = torch.tensor(list(seen.keys()) or [0], dtype=torch.int32, device=dev)
        cnt = torch.tensor(list(seen.values()) or [0], dtype=torch.int32, device=dev)
        ban = torch.tensor(list(banned) or [0], dtype=torch.int32, device=dev)
        out = torch.empty(1, dtype=torch.int32, device=dev)
        opt = _lib.SampleOptions(temperature, top_k, top_p, presence, frequency)
        check(self.lib.swq_sample(logits.data_ptr(), vocab, ctypes.byref(opt), ids.data_ptr(), cnt.data_ptr(),
                                  len(seen), ban.data_ptr(), len(banned), u, out.data_ptr(), ws.data_ptr(),
                                  ws.numel(), _stream_handle(stream)), "sample")
        return int(out.item())

    # Checkpoint.moduleWeightSlice (Checkpoint.swift:148-155): rows of the
    # flattened [experts*out, in] weight as fp32.
    def dequantize(self, lin: GPULinear, row0: int, rows: int, stream=None):
        torch = _torch()
        out = torch.empty((rows, lin.in_dim), dtype=torch.float32, device=lin.w.device)
        c = lin.c()
        check(self.lib.swq_dequantize(ctypes.byref(c), row0, rows, out.data_ptr(),
                                      _stream_handle(stream)), "dequantize")
        return out
