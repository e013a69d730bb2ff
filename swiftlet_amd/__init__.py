"""MI355X-native MoE-layer decode hot path of Swiftlet, behind a C ABI.

libswq.so (csrc/*.hip, built by ``python -m swiftlet_amd.build``) holds the
gfx950 kernels; this package binds it with ctypes and mirrors SwiftletCore's
operator API (engine.HipEngine, engine.GPULinear, moe.MoELayerGPU)."""

__all__ = ["build", "engine", "moe", "synth"]
