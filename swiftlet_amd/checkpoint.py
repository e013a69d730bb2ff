"""Checkpoint and .qpack loading into HBM, over the library's native reader
(swq_checkpoint_* / swq_qpack_* in include/swq.h).

Checkpoint        Checkpoint (Checkpoint.swift:7-160): tensor names, infos,
                  quant specs, raw bytes; resident modules via
                  MetalShardStore.residentLinear (MetalShardStore.swift:67-118).
QpackExpertReader QpackExpertReader (Qpack.swift:168-203): the layout, one
                  blob on the host (readExpert), and whole layers in HBM
                  addressed in place as expert stacks.
moe_layer_from_checkpoint
                  the MoE block of one decoder layer as QwenMetalModel
                  assembles MoEGPU (QwenMetalModel.swift:167-200), experts
                  from the stacked switch_mlp tensors or a qpack container.

torch supplies device memory only; every byte is read and copied by the
library."""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

from . import _lib
from .engine import GPULinear, _stream_handle, _torch
from .moe import MoELayerGPU

# stored dtype -> torch dtype of the same width (unsigned 16/32/64-bit words as
# the signed type's bit patterns)
_TORCH_DTYPES = {"F32": "float32", "F16": "float16", "BF16": "bfloat16", "I32": "int32", "U32": "int32",
                 "I64": "int64", "U64": "int64", "I16": "int16", "U16": "int16", "U8": "uint8", "I8": "int8",
                 "F64": "float64", "BOOL": "bool", "F8_E5M2": "uint8", "F8_E4M3": "uint8"}


@dataclass(frozen=True)
class TensorInfo:
    """SafetensorsFile.TensorInfo: dtype name, shape, stored bytes."""
    dtype: str
    shape: tuple
    nbytes: int


def _info(ti: _lib.TensorInfo) -> TensorInfo:
    return TensorInfo(ti.dtype.decode(), tuple(ti.shape[i] for i in range(ti.ndim)), ti.nbytes)


def _device_bytes(n: int, device):
    torch = _torch()
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


class Checkpoint:
    """An mlx-lm checkpoint directory (single file or index + shards)."""

    def __init__(self, directory):
        self.lib = _lib.load()
        self.dir = Path(directory)
        h = ctypes.c_void_p()
        _lib.check(self.lib.swq_checkpoint_open(str(self.dir).encode(), ctypes.byref(h)), f"open {self.dir}")
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            self.lib.swq_checkpoint_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def tensor_names(self) -> list[str]:
        n = self.lib.swq_checkpoint_tensor_count(self._h)
        return [self.lib.swq_checkpoint_tensor_name(self._h, i).decode() for i in range(n)]

    def contains(self, name: str) -> bool:
        ti = _lib.TensorInfo()
        return self.lib.swq_checkpoint_tensor(self._h, name.encode(), ctypes.byref(ti)) == _lib.SWQ_OK

    def info(self, name: str) -> TensorInfo:
        ti = _lib.TensorInfo()
        _lib.check(self.lib.swq_checkpoint_tensor(self._h, name.encode(), ctypes.byref(ti)), name)
        return _info(ti)

    def is_quantized(self, path: str) -> bool:
        """Checkpoint.isQuantized (Checkpoint.swift:106-109)."""
        return self.contains(path + ".scales")

    def quant_spec(self, path: str):
        """(group_size, bits), or None for a module stored unquantized."""
        g, b = ctypes.c_int(), ctypes.c_int()
        st = self.lib.swq_checkpoint_quant(self._h, path.encode(), ctypes.byref(g), ctypes.byref(b))
        if st == _lib.SWQ_ERR_MISSING_TENSOR:
            return None
        _lib.check(st, path)
        return g.value, b.value

    def raw_tensor(self, name: str) -> bytes:
        """Checkpoint.rawTensor (Checkpoint.swift:86-90): the stored bytes."""
        n = self.info(name).nbytes
        buf = ctypes.create_string_buffer(max(n, 1))
        _lib.check(self.lib.swq_checkpoint_read(self._h, name.encode(), buf, n), name)
        return buf.raw[:n]

    def load(self, name: str, device="cuda", stream=None):
        """The stored bytes in HBM as a typed device tensor of the stored shape
        (U32 as int32 bit patterns)."""
        torch = _torch()
        ti = self.info(name)
        buf = _device_bytes(ti.nbytes, device)
        _lib.check(self.lib.swq_checkpoint_load(self._h, name.encode(), ctypes.c_void_p(buf.data_ptr()),
                                                ti.nbytes, _stream_handle(stream)), name)
        dt = getattr(torch, _TORCH_DTYPES[ti.dtype])
        return buf[:ti.nbytes].view(dt).reshape(ti.shape)

    def gpu_linear(self, path: str, rows_per_expert: int = 0, device="cuda", stream=None) -> GPULinear:
        """A quantized module resident in one device buffer; rows_per_expert
        > 0: a stacked expert tensor."""
        n = self.lib.swq_checkpoint_linear_bytes(self._h, path.encode())
        if n < 0:
            raise _lib.SwqError(n, path)
        buf = _device_bytes(n, device)
        q = _lib.QLinear()
        _lib.check(self.lib.swq_checkpoint_linear(self._h, path.encode(), rows_per_expert,
                                                  ctypes.c_void_p(buf.data_ptr()), n, ctypes.byref(q),
                                                  _stream_handle(stream)), path)
        rows_all = 1
        for d in self.info(path + ".weight").shape[:-1]:
            rows_all *= d
        return _linear_from_c(q, buf, rows_all // q.out_dim)


def _linear_from_c(q: _lib.QLinear, buf, experts: int) -> GPULinear:
    return GPULinear(buf, buf, buf, q.out_dim, q.in_dim, q.group_size, q.bits, q.scales_type,
                     w_off=q.w_off, s_off=q.s_off, b_off=q.b_off, expert_stride_w=q.expert_stride_w,
                     expert_stride_sb=q.expert_stride_sb, num_experts=experts)


@dataclass(frozen=True)
class Section:
    """Qpack.Section (Qpack.swift:22-28)."""
    name: str
    dtype: str
    shape: tuple
    offset: int
    size: int


class QpackExpertReader:
    """A .qpack container's expert blobs."""

    def __init__(self, container_dir):
        self.lib = _lib.load()
        self.dir = Path(container_dir)
        h = ctypes.c_void_p()
        _lib.check(self.lib.swq_qpack_open(str(self.dir).encode(), ctypes.byref(h)), f"open {self.dir}")
        self._h = h
        li = _lib.QpackLayoutInfo()
        _lib.check(self.lib.swq_qpack_layout(self._h, ctypes.byref(li)), "qpack layout")
        self.expert_count, self.layer_count = li.expert_count, li.layer_count
        self.expert_stride = li.expert_stride
        self.quant_bits, self.quant_group_size = li.quant_bits, li.quant_group_size
        self.sections = []
        for i in range(li.section_count):
            name, off, ti = ctypes.c_char_p(), ctypes.c_int64(), _lib.TensorInfo()
            _lib.check(self.lib.swq_qpack_section(self._h, i, ctypes.byref(name), ctypes.byref(off),
                                                  ctypes.byref(ti)), "qpack section")
            t = _info(ti)
            self.sections.append(Section(name.value.decode(), t.dtype, t.shape, off.value, t.nbytes))

    def close(self):
        if getattr(self, "_h", None):
            self.lib.swq_qpack_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def section(self, name: str):
        i = self.lib.swq_qpack_find_section(self._h, name.encode())
        return self.sections[i] if i >= 0 else None

    def is_linear_layer(self, layer: int) -> bool:
        v = self.lib.swq_qpack_is_linear_layer(self._h, layer)
        if v < 0:
            raise _lib.SwqError(v, f"layer {layer}")
        return bool(v)

    def read_expert(self, layer: int, expert: int) -> bytes:
        """readExpert (Qpack.swift:185-197): one blob of expert_stride bytes."""
        buf = ctypes.create_string_buffer(self.expert_stride)
        _lib.check(self.lib.swq_qpack_read_expert(self._h, layer, expert, buf, self.expert_stride),
                   f"layer {layer} expert {expert}")
        return buf.raw

    def load_experts(self, layer: int, first: int = 0, count: int | None = None, device="cuda", stream=None):
        """Blobs [first, first + count) of a layer in HBM, byte for byte."""
        count = self.expert_count - first if count is None else count
        n = count * self.expert_stride
        buf = _device_bytes(n, device)
        _lib.check(self.lib.swq_qpack_load_experts(self._h, layer, first, count, ctypes.c_void_p(buf.data_ptr()),
                                                   n, _stream_handle(stream)), f"layer {layer}")
        return buf

    def expert_linear(self, blobs, proj: str) -> GPULinear:
        """The expert stack of `proj` addressed inside resident blobs."""
        q = _lib.QLinear()
        _lib.check(self.lib.swq_qpack_expert_linear(self._h, ctypes.c_void_p(blobs.data_ptr()), proj.encode(),
                                                    ctypes.byref(q)), proj)
        return _linear_from_c(q, blobs, blobs.numel() // self.expert_stride)


def moe_layer_from_checkpoint(ckpt: Checkpoint, layer: int, config: dict, qpack: QpackExpertReader | None = None,
                              device="cuda", stream=None) -> MoELayerGPU:
    """Layer `layer`'s MoE block: router, shared expert and its gate from the
    checkpoint (resident), the routed experts from the stacked switch_mlp
    tensors or, with `qpack`, from the container's layer file in HBM."""
    p = f"model.layers.{layer}.mlp."

    def dense(path):
        return ckpt.gpu_linear(path, device=device, stream=stream)

    I, H = config["moe_intermediate_size"], config["hidden_size"]
    if qpack is not None:
        blobs = qpack.load_experts(layer, device=device, stream=stream)
        gate, up, down = (qpack.expert_linear(blobs, n) for n in ("gate_proj", "up_proj", "down_proj"))
    else:
        gate = ckpt.gpu_linear(p + "switch_mlp.gate_proj", I, device, stream)
        up = ckpt.gpu_linear(p + "switch_mlp.up_proj", I, device, stream)
        down = ckpt.gpu_linear(p + "switch_mlp.down_proj", H, device, stream)
    has_shared = ckpt.contains(p + "shared_expert.gate_proj.weight")
    return MoELayerGPU(dense(p + "gate"), gate, up, down,
                       dense(p + "shared_expert.gate_proj") if has_shared else None,
                       dense(p + "shared_expert.up_proj") if has_shared else None,
                       dense(p + "shared_expert.down_proj") if has_shared else None,
                       dense(p + "shared_expert_gate") if has_shared else None,
                       top_k=config["num_experts_per_tok"],
                       norm_topk_prob=bool(config.get("norm_topk_prob", False)))
