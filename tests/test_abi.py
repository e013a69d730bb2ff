"""The C ABI without a GPU: libswq.so loads, exports every symbol the headers
declare, and its host-side validation returns the documented status codes
before touching a device (the boundary's failure modes: in % group, bits
outside {2,4,8}, top_k > E, misaligned pointers, short workspace)."""

import ctypes
import re
from pathlib import Path

import pytest

from swiftlet_amd import _lib
from swiftlet_amd._lib import MoELayer, QLinear

ROOT = Path(__file__).resolve().parent.parent
FAKE = 0x7F0000000000  # a well-aligned address; validation fails before any use


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(swq_\w+)\s*\(", text))
    return sorted(names)


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert "swq_moe_decode" in names and "swq_encode_gemv" in names
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_strerror_and_version(lib):
    assert lib.swq_version() >= 100
    for code in range(0, -15, -1):
        s = lib.swq_strerror(code).decode()
        assert s and s != "unknown status", code
    assert lib.swq_strerror(-99).decode() == "unknown status"


def lin(out_dim, in_dim, bits=4, group=64, stype=_lib.SWQ_F16, stride_w=0, stride_sb=0, base=FAKE):
    return QLinear(w=base, scales=base + (1 << 30), biases=base + (2 << 30), w_off=0, s_off=0, b_off=0,
                   out_dim=out_dim, in_dim=in_dim, group_size=group, bits=bits, scales_type=stype,
                   reserved=0, expert_stride_w=stride_w, expert_stride_sb=stride_sb)


def layer(H=2048, E=256, K=8, I=512, Is=512, bits=4, rbits=8, **kw):
    ew = I * H * bits // 8
    es = I * (H // 64) * 2
    d = dict(router=lin(E, H, rbits), gate=lin(I, H, bits, stride_w=ew, stride_sb=es),
             up=lin(I, H, bits, stride_w=ew, stride_sb=es), down=lin(H, I, bits, stride_w=ew, stride_sb=es),
             shared_gate=lin(Is, H, bits), shared_up=lin(Is, H, bits), shared_down=lin(H, Is, bits),
             shared_expert_gate=lin(1, H, rbits), hidden=H, num_experts=E, top_k=K, moe_intermediate=I,
             shared_intermediate=Is, norm_topk_prob=1, has_shared=1, reserved=0)
    d.update(kw)
    return MoELayer(**d)


def test_workspace_status_validation(lib):
    """The stall record of the single-launch path sits in the workspace
    header at a fixed offset; the query rejects a missing or short
    workspace before touching a device."""
    assert lib.swq_moe_workspace_status(None, 1 << 20, 1, None) == _lib.SWQ_ERR_WORKSPACE
    assert lib.swq_moe_workspace_status(FAKE, 255, 1, None) == _lib.SWQ_ERR_WORKSPACE
    L = layer()
    assert lib.swq_moe_workspace_error_offset(ctypes.byref(L), 1) == 64
    assert lib.swq_strerror(_lib.SWQ_ERR_STALLED).decode().startswith("a single-launch MoE call")


def test_workspace_query(lib):
    L = layer()
    n1 = lib.swq_moe_decode_workspace_bytes(ctypes.byref(L), 1)
    n4 = lib.swq_moe_decode_workspace_bytes(ctypes.byref(L), 4)
    assert n1 > 8 * 512 * 4 and n4 > n1 and n1 % 256 == 0
    assert lib.swq_moe_decode_workspace_bytes(ctypes.byref(L), 0) == 0
    assert lib.swq_moe_decode_workspace_bytes(ctypes.byref(L), 17) == 0  # above SWQ_MAX_BATCH


def decode(lib, L, batch=1, ws_bytes=None, x=FAKE, x_dtype=_lib.SWQ_BF16, out_dtype=_lib.SWQ_F32, flags=0, ws=FAKE):
    if ws_bytes is None:
        ws_bytes = max(lib.swq_moe_decode_workspace_bytes(ctypes.byref(L), batch), 1 << 20)
    return lib.swq_moe_decode(ctypes.byref(L), x, x_dtype, batch, FAKE, out_dtype, None, None, ws, ws_bytes,
                              flags, None)


@pytest.mark.parametrize("mutate,code", [
    (dict(top_k=0), _lib.SWQ_ERR_EXPERT_RANGE),
    (dict(top_k=300), _lib.SWQ_ERR_EXPERT_RANGE),
    (dict(top_k=17, num_experts=64, router=lin(64, 2048, 8)), _lib.SWQ_ERR_LIMIT),
    (dict(reserved=1), _lib.SWQ_ERR_INVALID_ARGUMENT),
    (dict(router=lin(256, 2048, 3)), _lib.SWQ_ERR_UNSUPPORTED_BITS),
    (dict(router=lin(256, 2048, 8, group=96)), _lib.SWQ_ERR_BAD_SHAPE),      # in % group != 0
    (dict(router=lin(256, 2048, 8, stype=7)), _lib.SWQ_ERR_UNSUPPORTED_DTYPE),
    (dict(router=lin(128, 2048, 8)), _lib.SWQ_ERR_BAD_SHAPE),                # out_dim != E
    (dict(router=lin(256, 2048, 8, base=FAKE + 4)), _lib.SWQ_ERR_MISALIGNED),
    (dict(gate=lin(512, 2048, 4, stride_w=0, stride_sb=0)), _lib.SWQ_ERR_INVALID_ARGUMENT),
    (dict(hidden=4096), _lib.SWQ_ERR_BAD_SHAPE),                             # router in_dim != hidden
    (dict(hidden=4096, router=lin(256, 4096, 8)), _lib.SWQ_ERR_LIMIT),       # 8-bit rows above 2048
])
def test_layer_validation(lib, mutate, code):
    assert decode(lib, layer(**mutate)) == code


def test_call_validation(lib):
    L = layer()
    assert decode(lib, L, batch=0) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert decode(lib, L, batch=17) == _lib.SWQ_ERR_LIMIT
    assert decode(lib, L, ws_bytes=64) == _lib.SWQ_ERR_WORKSPACE
    assert decode(lib, L, ws=0) == _lib.SWQ_ERR_WORKSPACE
    assert decode(lib, L, x=0) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert decode(lib, L, x=FAKE + 2) == _lib.SWQ_ERR_MISALIGNED
    assert decode(lib, L, x_dtype=_lib.SWQ_F16) == _lib.SWQ_ERR_UNSUPPORTED_DTYPE
    assert decode(lib, L, flags=4) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert decode(lib, L, flags=_lib.SWQ_MOE_ACCUMULATE, out_dtype=_lib.SWQ_BF16) == _lib.SWQ_ERR_UNSUPPORTED_DTYPE


def test_gemv_validation(lib):
    bad = lin(16, 100, 4, group=64)  # in % group != 0
    assert lib.swq_encode_gemv(ctypes.byref(bad), 0, 0, 0, 0, FAKE, 0, FAKE, 0, None) == _lib.SWQ_ERR_BAD_SHAPE
    bad = lin(16, 128, 5, group=64)
    assert lib.swq_encode_gemv(ctypes.byref(bad), 0, 0, 0, 0, FAKE, 0, FAKE, 0, None) == _lib.SWQ_ERR_UNSUPPORTED_BITS
    ok = lin(16, 128, 4, group=64)
    assert lib.swq_encode_gemv(ctypes.byref(ok), 0, 0, 0, 0, 0, 0, FAKE, 0, None) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert lib.swq_dequantize(ctypes.byref(ok), 10, 10, FAKE, None) == _lib.SWQ_ERR_BAD_SHAPE  # past out_dim
    assert lib.swq_encode_silu_mul(FAKE, 0, 0, 0, 0, None) == _lib.SWQ_ERR_INVALID_ARGUMENT


def test_gemv_multi_validation(lib):
    """swq_encode_gemv_multi rejects bad calls before any launch (every call
    here fails validation: no kernel ever sees the fake addresses)."""
    F = _lib.SWQ_F32
    two = (QLinear * 2)(lin(64, 2048), lin(32, 2048))
    ys = (ctypes.c_void_p * 2)(FAKE, FAKE)
    call = lib.swq_encode_gemv_multi
    assert call(two, 0, ys, FAKE, None, F, 1e-6, None) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert call(two, 5, ys, FAKE, None, F, 1e-6, None) == _lib.SWQ_ERR_LIMIT  # more than four matrices
    assert call(two, 2, ys, FAKE + 4, None, F, 1e-6, None) == _lib.SWQ_ERR_MISALIGNED  # x
    assert call(two, 2, ys, FAKE, FAKE + 8, _lib.SWQ_BF16, 1e-6, None) == _lib.SWQ_ERR_MISALIGNED  # norm weight
    assert call(two, 2, ys, FAKE, FAKE, 7, 1e-6, None) == _lib.SWQ_ERR_UNSUPPORTED_DTYPE
    assert call(two, 2, ys, FAKE, FAKE, F, -1.0, None) == _lib.SWQ_ERR_INVALID_ARGUMENT
    mixed = (QLinear * 2)(lin(64, 2048), lin(32, 1024))
    assert call(mixed, 2, ys, FAKE, None, F, 1e-6, None) == _lib.SWQ_ERR_BAD_SHAPE  # in_dim differs
    wide = (QLinear * 1)(lin(64, 8192))
    assert call(wide, 1, ys, FAKE, None, F, 1e-6, None) == _lib.SWQ_ERR_LIMIT  # in_dim above 4096


def test_rmsnorm_validation(lib):
    F = _lib.SWQ_F32
    assert lib.swq_rmsnorm(0, None, None, F, 1e-6, 1, 64, FAKE, F, None) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert lib.swq_rmsnorm(FAKE, None, None, F, 1e-6, 0, 64, FAKE, F, None) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert lib.swq_rmsnorm(FAKE, None, None, F, -1.0, 1, 64, FAKE, F, None) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert lib.swq_rmsnorm(FAKE, None, FAKE, 7, 1e-6, 1, 64, FAKE, F, None) == _lib.SWQ_ERR_UNSUPPORTED_DTYPE
    assert lib.swq_rmsnorm(FAKE, None, None, F, 1e-6, 1, 64, FAKE, _lib.SWQ_F16, None) == _lib.SWQ_ERR_UNSUPPORTED_DTYPE
    assert lib.swq_rmsnorm(FAKE + 2, None, None, F, 1e-6, 1, 64, FAKE, F, None) == _lib.SWQ_ERR_MISALIGNED
    assert lib.swq_rmsnorm(FAKE, None, FAKE + 1, _lib.SWQ_BF16, 1e-6, 1, 64, FAKE, F, None) == _lib.SWQ_ERR_MISALIGNED


def test_no_device_reported(lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is visible")
    n = ctypes.c_int(5)
    assert lib.swq_device_count(ctypes.byref(n)) == _lib.SWQ_ERR_NO_DEVICE and n.value == 0
    from swiftlet_amd.engine import HipEngine, NoDevice
    with pytest.raises(NoDevice):
        HipEngine()


def prefill(lib, L, T=64, ws_bytes=None, x=FAKE, x_dtype=_lib.SWQ_BF16, out_dtype=_lib.SWQ_F32, flags=0):
    if ws_bytes is None:
        ws_bytes = max(lib.swq_moe_prefill_workspace_bytes(ctypes.byref(L), T), 1 << 20)
    return lib.swq_moe_prefill(ctypes.byref(L), x, x_dtype, T, FAKE, out_dtype, None, None, FAKE, ws_bytes,
                               flags, None)


def test_prefill_workspace_query(lib):
    L = layer()
    n = lib.swq_moe_prefill_workspace_bytes(ctypes.byref(L), 512)
    rows = 512 * 8 + 512
    assert n > rows * 2048 * 4 + rows * 512 * 4 and n % 256 == 0  # y rows, h hi/lo planes
    assert lib.swq_moe_prefill_workspace_bytes(ctypes.byref(L), 1024) > n
    assert lib.swq_moe_prefill_workspace_bytes(ctypes.byref(L), 0) == 0
    assert lib.swq_moe_prefill_workspace_bytes(ctypes.byref(layer(router=lin(256, 2048, 8, group=32))), 8) == 0


@pytest.mark.parametrize("mutate,code", [
    (dict(router=lin(256, 2048, 8, group=32)), _lib.SWQ_ERR_LIMIT),        # group 64 only
    (dict(I=64, Is=64), _lib.SWQ_ERR_LIMIT),                                # down rows of 64 inputs
    (dict(router=lin(256, 2048, 2)), _lib.SWQ_ERR_UNSUPPORTED_BITS),
    (dict(shared_down=lin(2048, 512, 8)), _lib.SWQ_ERR_LIMIT),              # shared bits != routed
    (dict(hidden=4096, router=lin(256, 4096, 8)), _lib.SWQ_ERR_BAD_SHAPE),  # gate in_dim != hidden
    (dict(hidden=8192, router=lin(256, 8192, 8)), _lib.SWQ_ERR_LIMIT),      # rows above 4096 inputs
    (dict(top_k=0), _lib.SWQ_ERR_EXPERT_RANGE),
    (dict(reserved=2), _lib.SWQ_ERR_INVALID_ARGUMENT),
    (dict(router=lin(256, 2048, 8, base=FAKE + 4)), _lib.SWQ_ERR_MISALIGNED),
])
def test_prefill_layer_validation(lib, mutate, code):
    assert prefill(lib, layer(**mutate)) == code


def test_prefill_call_validation(lib):
    L = layer()
    assert prefill(lib, L, T=0) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert prefill(lib, L, ws_bytes=64) == _lib.SWQ_ERR_WORKSPACE
    assert prefill(lib, L, x=0) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert prefill(lib, L, x=FAKE + 2) == _lib.SWQ_ERR_MISALIGNED
    assert prefill(lib, L, x_dtype=_lib.SWQ_F16) == _lib.SWQ_ERR_UNSUPPORTED_DTYPE
    assert prefill(lib, L, flags=2) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert prefill(lib, L, flags=_lib.SWQ_MOE_ACCUMULATE, out_dtype=_lib.SWQ_BF16) == _lib.SWQ_ERR_UNSUPPORTED_DTYPE
    n = lib.swq_moe_prefill_workspace_bytes(ctypes.byref(L), 64)
    assert lib.swq_moe_prefill_biased(ctypes.byref(L), FAKE, _lib.SWQ_BF16, 64, FAKE, _lib.SWQ_F32, None, None,
                                      None, FAKE, n, 0, None) == _lib.SWQ_ERR_INVALID_ARGUMENT


def test_deltanet_validation(lib):
    """swq_deltanet_step's failure modes, returned before any launch."""
    from swiftlet_amd._lib import DeltaNetLayer
    ok = dict(num_key_heads=16, num_value_heads=32, key_head_dim=128, value_head_dim=128, conv_kernel=4,
              layout=_lib.SWQ_DELTA_SPLIT, norm_eps=1e-6, reserved=0, conv_weight=FAKE, a_log=FAKE, dt_bias=FAKE,
              norm_weight=FAKE)
    L = DeltaNetLayer(**ok)
    n = lib.swq_deltanet_state_bytes(ctypes.byref(L))
    assert n == 4 * (2 * 16 * 128 + 32 * 128) * 4 + 32 * 128 * 128 * 4  # ring [K][convD] + state [nv][dv][dk]

    def step(layer, state_bytes=n, position=0, state=FAKE, qkvz=FAKE):
        return lib.swq_deltanet_step(ctypes.byref(layer), qkvz, FAKE, state, state_bytes, position, FAKE, None)

    for field, value, code in [("num_value_heads", 31, _lib.SWQ_ERR_BAD_SHAPE),
                               ("key_head_dim", 96, _lib.SWQ_ERR_LIMIT),
                               ("value_head_dim", 2048, _lib.SWQ_ERR_LIMIT),
                               ("conv_kernel", 9, _lib.SWQ_ERR_LIMIT),
                               ("layout", 2, _lib.SWQ_ERR_INVALID_ARGUMENT),
                               ("reserved", 1, _lib.SWQ_ERR_INVALID_ARGUMENT),
                               ("a_log", None, _lib.SWQ_ERR_INVALID_ARGUMENT)]:
        bad = DeltaNetLayer(**dict(ok, **{field: value}))
        assert step(bad) == code, field
        assert lib.swq_deltanet_state_bytes(ctypes.byref(bad)) == 0, field
    assert step(L, state_bytes=n - 1) == _lib.SWQ_ERR_WORKSPACE
    assert step(L, position=-1) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert step(L, state=FAKE + 16) == _lib.SWQ_ERR_MISALIGNED
    assert step(L, qkvz=None) == _lib.SWQ_ERR_INVALID_ARGUMENT


def test_attention_validation(lib):
    """swq_attention_step's failure modes, returned before any launch."""
    from swiftlet_amd._lib import AttentionLayer
    ok = dict(num_heads=16, num_kv_heads=2, head_dim=256, rotary_dims=64, rope_theta=1e7, norm_eps=1e-6,
              max_positions=100, reserved=0, q_norm_weight=FAKE, k_norm_weight=FAKE)
    L = AttentionLayer(**ok)
    n = lib.swq_attention_cache_bytes(ctypes.byref(L))
    assert n == 2 * 100 * 2 * 256 * 4
    w = lib.swq_attention_workspace_bytes(ctypes.byref(L))
    assert w >= 16 * (256 + 2) * 4

    def step(layer, position=0, cache_bytes=n, ws_bytes=w, cache=FAKE):
        return lib.swq_attention_step(ctypes.byref(layer), FAKE, FAKE, FAKE, cache, cache_bytes, position, FAKE,
                                      FAKE, ws_bytes, None)

    for field, value, code in [("num_kv_heads", 3, _lib.SWQ_ERR_BAD_SHAPE),
                               ("num_heads", 64, _lib.SWQ_ERR_LIMIT),
                               ("head_dim", 96, _lib.SWQ_ERR_LIMIT),
                               ("rotary_dims", 63, _lib.SWQ_ERR_BAD_SHAPE),
                               ("rotary_dims", 512, _lib.SWQ_ERR_BAD_SHAPE),
                               ("max_positions", 0, _lib.SWQ_ERR_INVALID_ARGUMENT),
                               ("reserved", 1, _lib.SWQ_ERR_INVALID_ARGUMENT),
                               ("k_norm_weight", None, _lib.SWQ_ERR_INVALID_ARGUMENT)]:
        bad = AttentionLayer(**dict(ok, **{field: value}))
        assert step(bad) == code, field
        assert lib.swq_attention_cache_bytes(ctypes.byref(bad)) == 0, field
    assert step(L, position=100) == _lib.SWQ_ERR_LIMIT
    assert step(L, position=-1) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert step(L, cache_bytes=n - 1) == _lib.SWQ_ERR_WORKSPACE
    assert step(L, ws_bytes=w - 1) == _lib.SWQ_ERR_WORKSPACE
    assert step(L, cache=FAKE + 64) == _lib.SWQ_ERR_MISALIGNED


def test_moe_decode_norm_validation(lib):
    """swq_moe_decode_norm's argument checks (before any launch)."""
    L = layer()
    ws_bytes = lib.swq_moe_decode_workspace_bytes(ctypes.byref(L), 1)
    H = L.hidden

    def call(h=FAKE, res=None, w=FAKE, wdt=_lib.SWQ_BF16, eps=1e-6, out=FAKE + (1 << 20), ws=FAKE, wsb=ws_bytes):
        return lib.swq_moe_decode_norm(ctypes.byref(L), h, res, w, wdt, eps, out, None, None, ws, wsb, None)

    assert call(h=None) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert call(w=None) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert call(wdt=7) == _lib.SWQ_ERR_UNSUPPORTED_DTYPE
    assert call(eps=-1.0) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert call(out=FAKE + 4 * (H - 1)) == _lib.SWQ_ERR_INVALID_ARGUMENT  # out overlaps h
    assert call(res=FAKE + (2 << 20), out=FAKE + (2 << 20) + 8) == _lib.SWQ_ERR_INVALID_ARGUMENT  # out overlaps r
    assert call(wsb=ws_bytes - 1) == _lib.SWQ_ERR_WORKSPACE
    assert call(h=FAKE + 2) == _lib.SWQ_ERR_MISALIGNED
