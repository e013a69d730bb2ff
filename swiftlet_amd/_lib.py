"""ctypes binding of libswq.so (the C ABI declared in include/swq.h and
include/swq_bench.h).  Loading fails loudly when the library is not built:
there is no fallback path."""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("SWQ_LIBRARY", Path(__file__).resolve().parent / "libswq.so"))

SWQ_OK = 0
SWQ_ERR_INVALID_ARGUMENT = -1
SWQ_ERR_BAD_SHAPE = -2
SWQ_ERR_UNSUPPORTED_BITS = -3
SWQ_ERR_UNSUPPORTED_DTYPE = -4
SWQ_ERR_MISALIGNED = -5
SWQ_ERR_WORKSPACE = -6
SWQ_ERR_EXPERT_RANGE = -7
SWQ_ERR_HIP = -8
SWQ_ERR_NO_DEVICE = -9
SWQ_ERR_LIMIT = -10
SWQ_ERR_MISSING_TENSOR = -11
SWQ_ERR_IO = -12
SWQ_ERR_FORMAT = -13
SWQ_ERR_STALLED = -14

SWQ_F32, SWQ_F16, SWQ_BF16 = 0, 1, 2
SWQ_MAX_BATCH, SWQ_MAX_TOPK = 16, 16
SWQ_MOE_ACCUMULATE = 1
SWQ_STAGES_FUSED = 8  # swq_bench.h: the single-launch path
SWQ_PREFILL_ALL = 63  # swq_bench.h: every launch of swq_moe_prefill_stages


class SwqError(RuntimeError):
    """A negative status from the C ABI."""

    def __init__(self, code: int, what: str = ""):
        self.code = code
        msg = strerror(code)
        super().__init__(f"{what}: {msg} ({code})" if what else f"{msg} ({code})")


class QLinear(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p),
        ("w_off", ctypes.c_int64), ("s_off", ctypes.c_int64), ("b_off", ctypes.c_int64),
        ("out_dim", ctypes.c_int32), ("in_dim", ctypes.c_int32),
        ("group_size", ctypes.c_int32), ("bits", ctypes.c_int32),
        ("scales_type", ctypes.c_int32), ("reserved", ctypes.c_int32),
        ("expert_stride_w", ctypes.c_int64), ("expert_stride_sb", ctypes.c_int64),
    ]


class SampleOptions(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32), ("top_p", ctypes.c_float),
                ("presence_penalty", ctypes.c_float), ("frequency_penalty", ctypes.c_float)]


SWQ_MAX_DIMS = 8


class TensorInfo(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_char * 8), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * SWQ_MAX_DIMS), ("nbytes", ctypes.c_int64)]


class QpackLayoutInfo(ctypes.Structure):
    _fields_ = [("expert_count", ctypes.c_int32), ("layer_count", ctypes.c_int32),
                ("expert_stride", ctypes.c_int64), ("quant_bits", ctypes.c_int32),
                ("quant_group_size", ctypes.c_int32), ("section_count", ctypes.c_int32)]


SWQ_DELTA_INTERLEAVED, SWQ_DELTA_SPLIT = 0, 1


class DeltaNetLayer(ctypes.Structure):
    _fields_ = [
        ("num_key_heads", ctypes.c_int32), ("num_value_heads", ctypes.c_int32),
        ("key_head_dim", ctypes.c_int32), ("value_head_dim", ctypes.c_int32),
        ("conv_kernel", ctypes.c_int32), ("layout", ctypes.c_int32), ("norm_eps", ctypes.c_float),
        ("reserved", ctypes.c_int32), ("conv_weight", ctypes.c_void_p), ("a_log", ctypes.c_void_p),
        ("dt_bias", ctypes.c_void_p), ("norm_weight", ctypes.c_void_p),
    ]


class AttentionLayer(ctypes.Structure):
    _fields_ = [
        ("num_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("rotary_dims", ctypes.c_int32), ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float),
        ("max_positions", ctypes.c_int32), ("reserved", ctypes.c_int32),
        ("q_norm_weight", ctypes.c_void_p), ("k_norm_weight", ctypes.c_void_p),
    ]


class MoELayer(ctypes.Structure):
    _fields_ = [
        ("router", QLinear), ("gate", QLinear), ("up", QLinear), ("down", QLinear),
        ("shared_gate", QLinear), ("shared_up", QLinear), ("shared_down", QLinear),
        ("shared_expert_gate", QLinear),
        ("hidden", ctypes.c_int32), ("num_experts", ctypes.c_int32), ("top_k", ctypes.c_int32),
        ("moe_intermediate", ctypes.c_int32), ("shared_intermediate", ctypes.c_int32),
        ("norm_topk_prob", ctypes.c_int32), ("has_shared", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_c = ctypes
_P = _c.c_void_p
_I = _c.c_int
_I64 = _c.c_int64
_U64 = _c.c_uint64
_SZ = _c.c_size_t

# name -> (restype, argtypes); the complete exported surface of the headers.
SIGNATURES = {
    "swq_strerror": (_c.c_char_p, [_I]),
    "swq_version": (_I, []),
    "swq_device_count": (_I, [_c.POINTER(_I)]),
    "swq_gemv_quantized": (_I, [_P, _P, _SZ, _P, _SZ, _P, _SZ, _I, _I, _I, _I, _I, _I, _P]),
    "swq_encode_gemv": (_I, [_c.POINTER(QLinear), _I, _I64, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "swq_encode_silu_mul": (_I, [_P, _I, _I64, _I64, _I64, _P]),
    "swq_encode_gemv_multi": (_I, [_c.POINTER(QLinear), _I, _c.POINTER(_P), _P, _P, _I, _c.c_float, _P]),
    "swq_dequantize": (_I, [_c.POINTER(QLinear), _I64, _I64, _P, _P]),
    "swq_rmsnorm": (_I, [_P, _P, _P, _I, _c.c_float, _I, _I, _P, _I, _P]),
    "swq_sample_workspace_bytes": (_SZ, [_I]),
    "swq_sample": (_I, [_P, _I, _c.POINTER(SampleOptions), _P, _P, _I, _P, _I, _c.c_float, _P, _P, _SZ, _P]),
    "swq_deltanet_state_bytes": (_SZ, [_c.POINTER(DeltaNetLayer)]),
    "swq_deltanet_step": (_I, [_c.POINTER(DeltaNetLayer), _P, _P, _P, _SZ, _I64, _P, _P]),
    "swq_attention_cache_bytes": (_SZ, [_c.POINTER(AttentionLayer)]),
    "swq_attention_workspace_bytes": (_SZ, [_c.POINTER(AttentionLayer)]),
    "swq_attention_step": (_I, [_c.POINTER(AttentionLayer), _P, _P, _P, _P, _SZ, _I64, _P, _P, _SZ, _P]),
    "swq_checkpoint_open": (_I, [_c.c_char_p, _c.POINTER(_P)]),
    "swq_checkpoint_close": (None, [_P]),
    "swq_checkpoint_tensor_count": (_I, [_P]),
    "swq_checkpoint_tensor_name": (_c.c_char_p, [_P, _I]),
    "swq_checkpoint_tensor": (_I, [_P, _c.c_char_p, _c.POINTER(TensorInfo)]),
    "swq_checkpoint_quant": (_I, [_P, _c.c_char_p, _c.POINTER(_I), _c.POINTER(_I)]),
    "swq_checkpoint_read": (_I, [_P, _c.c_char_p, _P, _I64]),
    "swq_checkpoint_load": (_I, [_P, _c.c_char_p, _P, _I64, _P]),
    "swq_checkpoint_linear_bytes": (_I64, [_P, _c.c_char_p]),
    "swq_checkpoint_linear": (_I, [_P, _c.c_char_p, _I, _P, _I64, _c.POINTER(QLinear), _P]),
    "swq_qpack_open": (_I, [_c.c_char_p, _c.POINTER(_P)]),
    "swq_qpack_close": (None, [_P]),
    "swq_qpack_layout": (_I, [_P, _c.POINTER(QpackLayoutInfo)]),
    "swq_qpack_is_linear_layer": (_I, [_P, _I]),
    "swq_qpack_section": (_I, [_P, _I, _c.POINTER(_c.c_char_p), _c.POINTER(_I64), _c.POINTER(TensorInfo)]),
    "swq_qpack_find_section": (_I, [_P, _c.c_char_p]),
    "swq_qpack_read_expert": (_I, [_P, _I, _I, _P, _I64]),
    "swq_qpack_load_experts": (_I, [_P, _I, _I, _I, _P, _I64, _P]),
    "swq_qpack_expert_linear": (_I, [_P, _P, _c.c_char_p, _c.POINTER(QLinear)]),
    "swq_moe_decode_workspace_bytes": (_SZ, [_c.POINTER(MoELayer), _I]),
    "swq_moe_workspace_init": (_I, [_P, _SZ, _P]),
    "swq_moe_workspace_status": (_I, [_P, _SZ, _I, _P]),
    "swq_moe_decode_noalloc": (_I, [_c.POINTER(MoELayer), _P, _I, _I, _P, _I, _P, _P, _I, _P]),
    "swq_moe_decode": (_I, [_c.POINTER(MoELayer), _P, _I, _I, _P, _I, _P, _P, _P, _SZ, _I, _P]),
    "swq_moe_decode_norm": (_I, [_c.POINTER(MoELayer), _P, _P, _P, _I, _c.c_float, _P, _P, _P, _P, _SZ, _P]),
    "swq_synth_u32": (_I, [_P, _I64, _U64, _U64, _I64, _P]),
    "swq_synth_scales": (_I, [_P, _P, _I64, _I, _U64, _U64, _I64, _P]),
    "swq_moe_decode_stages": (_I, [_c.POINTER(MoELayer), _P, _I, _I, _P, _I, _P, _P, _P, _SZ, _I, _I, _P]),
    "swq_bench_stall": (_I, [_I, _P]),
    "swq_moe_workspace_error_offset": (_SZ, [_c.POINTER(MoELayer), _I]),
    "swq_moe_prefill_workspace_bytes": (_SZ, [_c.POINTER(MoELayer), _I]),
    "swq_moe_prefill": (_I, [_c.POINTER(MoELayer), _P, _I, _I, _P, _I, _P, _P, _P, _SZ, _I, _P]),
    "swq_moe_prefill_biased": (_I, [_c.POINTER(MoELayer), _P, _I, _I, _P, _I, _P, _P, _P, _P, _SZ, _I, _P]),
    "swq_moe_prefill_stages": (_I, [_c.POINTER(MoELayer), _P, _I, _I, _P, _I, _P, _P, _P, _P, _SZ, _I, _I, _P]),
}

_lib = None


def load() -> ctypes.CDLL:
    """The loaded library; raises if libswq.so has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m swiftlet_amd.build` "
            "(the HIP library is required; there is no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def strerror(code: int) -> str:
    try:
        return load().swq_strerror(code).decode()
    except ImportError:
        return f"status {code}"


def check(code: int, what: str = "") -> int:
    if code != SWQ_OK:
        raise SwqError(code, what)
    return code
