"""ctypes wrapper of oracle/liboracle.so, the C restatement of
QwenCPUModel.moeForward (see moe_ref.c) — TEST INFRASTRUCTURE ONLY.

Used as the CPU baseline of bench.py and as a cross-check of the numpy
oracle.  Build: ``make -C oracle``."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import moe_ref as R

LIB = Path(__file__).resolve().parent / "liboracle.so"


class OqMat(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("b", ctypes.c_void_p),
                ("rows", ctypes.c_int32), ("in_", ctypes.c_int32), ("group", ctypes.c_int32),
                ("bits", ctypes.c_int32), ("estride_w", ctypes.c_int64), ("estride_sb", ctypes.c_int64)]


_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise ImportError(f"{LIB} missing: run `make -C oracle`")
        _lib = ctypes.CDLL(str(LIB))
        _lib.oracle_moe_forward.restype = ctypes.c_int
        _lib.oracle_max_threads.restype = ctypes.c_int
        _lib.oracle_dequantize.restype = None
    return _lib


class CStack:
    """Host stack of fp16-scaled quantized matrices for the C oracle."""

    def __init__(self, words: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int, group: int):
        self.words = np.ascontiguousarray(words, dtype=np.uint32)
        self.scales = np.ascontiguousarray(scales).view(np.uint16)
        self.biases = np.ascontiguousarray(biases).view(np.uint16)
        e = self.words.shape[0] if self.words.ndim == 3 else 1
        rows = self.words.shape[-2]
        self.mat = OqMat(self.words.ctypes.data, self.scales.ctypes.data, self.biases.ctypes.data,
                         rows, self.words.shape[-1] * (32 // bits), group, bits,
                         self.words.size // e, self.scales.size // e)

    def dequantize(self, expert: int) -> np.ndarray:
        out = np.empty((self.mat.rows, self.mat.in_), dtype=np.float32)
        load().oracle_dequantize(ctypes.byref(self.mat), expert, out.ctypes.data_as(ctypes.c_void_p))
        return out


class CMoE:
    """One MoE layer for the C oracle: dense router / shared weights
    (dequantised once, as QwenCPUModel caches dense layer weights) and
    quantized expert stacks (dequantised per call)."""

    def __init__(self, arrays: dict, hidden: int, experts: int, top_k: int, inter: int, shared_inter: int,
                 group: int, norm_topk_prob: bool = True):
        self.H, self.E, self.K, self.I, self.Is = hidden, experts, top_k, inter, shared_inter
        self.norm = norm_topk_prob
        dense = lambda k: np.ascontiguousarray(R.dequantize(arrays[k][0], arrays[k][1], arrays[k][2],
                                                            arrays[k][3], group, R.F16))
        self.router = dense("router")
        self.has_shared = shared_inter > 0
        if self.has_shared:
            self.sh_gate, self.sh_up, self.sh_down = dense("sh_gate"), dense("sh_up"), dense("sh_down")
            self.seg = dense("seg").reshape(-1)
        else:  # never read: the C oracle skips the shared expert
            self.sh_gate = self.sh_up = self.sh_down = self.seg = np.zeros(1, dtype=np.float32)
        self.gate = CStack(*arrays["gate"][:3], arrays["gate"][3], group)
        self.up = CStack(*arrays["up"][:3], arrays["up"][3], group)
        self.down = CStack(*arrays["down"][:3], arrays["down"][3], group)
        mx = max(inter, shared_inter)
        self.scratch = np.empty(3 * inter * hidden + 3 * mx + 2 * hidden + experts + 64, dtype=np.float32)

    def forward(self, x: np.ndarray, threads: int = 1):
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        S = x.shape[0]
        out = np.empty((S, self.H), dtype=np.float32)
        ids = np.empty((S, self.K), dtype=np.int32)
        w = np.empty((S, self.K), dtype=np.float32)
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        st = load().oracle_moe_forward(
            p(x), S, self.H, self.E, self.K, self.I, self.Is, int(self.norm), int(self.has_shared),
            p(self.router), ctypes.byref(self.gate.mat), ctypes.byref(self.up.mat), ctypes.byref(self.down.mat),
            p(self.sh_gate), p(self.sh_up), p(self.sh_down), p(self.seg), p(out), p(ids), p(w),
            p(self.scratch), threads)
        if st != 0:
            raise RuntimeError("oracle_moe_forward rejected its arguments")
        return out, ids, w


def max_threads() -> int:
    return load().oracle_max_threads()
