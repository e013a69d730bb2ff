"""swq_moe_decode_noalloc, the variant of swq_moe_decode whose workspace is a
static device array inside the library, against swq_moe_decode itself (a
workspace of its own per layer): equal bit for bit on two calls in a row, the
second with a smaller input (batch 4 on the three launches, then batch 1 on
the single launch), then a different, smaller layer sharing the same array,
a layer of one routed expert (its own single launch on the same array), then
the first layer again; f32 activations, bf16 outputs and the
accumulate flag; calls between swq_moe_decode_norm calls; the entry point
captured in a HIP graph and replayed; in a fresh process, a first call made
under capture is refused and the next one outside capture recovers.  Every
test ends with the array's stall record clear.  A layer whose workspace exceeds the array is refused before
any launch."""

import ctypes

import pytest

from swiftlet_amd import _lib, moe, synth
from tests import helpers

pytestmark = pytest.mark.gpu


def _noalloc(lib, layer, x, out, ids, w, flags=0, stream=None):
    import torch
    xdt = _lib.SWQ_BF16 if x.dtype == torch.bfloat16 else _lib.SWQ_F32
    odt = _lib.SWQ_BF16 if out.dtype == torch.bfloat16 else _lib.SWQ_F32
    return lib.swq_moe_decode_noalloc(ctypes.byref(layer._c), x.data_ptr(), xdt, x.shape[0], out.data_ptr(), odt,
                                      ids.data_ptr(), w.data_ptr(), flags, stream)


def _status(lib):
    """The stall record of this device's array (a NULL workspace of 0 bytes
    names it), cleared by the read."""
    return lib.swq_moe_workspace_status(None, 0, 1, None)


def _compare(lib, layer, batch, seed):
    import torch
    print(f"noalloc vs decode: E {layer.num_experts} batch {batch}", flush=True)
    x = helpers.bf16_bits_to_torch(synth.activations_bf16(seed, batch, layer.hidden))
    ref_out, ref_ids, ref_w = layer.decode(x)
    out = torch.full_like(ref_out, float("nan"))
    ids = torch.full_like(ref_ids, -1)
    w = torch.full_like(ref_w, float("nan"))
    _lib.check(_noalloc(lib, layer, x, out, ids, w), "moe_decode_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(ids, ref_ids)
    assert torch.equal(w, ref_w)
    assert torch.equal(out, ref_out)


def test_noalloc_matches_decode():
    lib = _lib.load()
    big = moe.synth_layer(synth.SHAPES["qwen3.6-35b-a3b-q4"], helpers.SEED, 0)
    _compare(lib, big, 4, helpers.SEED + 41)
    _compare(lib, big, 1, helpers.SEED + 42)  # smaller input, the single launch
    small = moe.synth_layer(synth.MoEShape("odd", 256, 60, 4, 64, 128, expert_bits=8, router_bits=8, group=64,
                                           norm_topk_prob=False), 77, 0)
    _compare(lib, small, 1, 78)
    _compare(lib, small, 3, 79)
    one = moe.synth_layer(synth.SHAPES["single-expert-q4"], helpers.SEED, 0)
    _compare(lib, one, 1, 80)  # the one-expert launch
    _compare(lib, big, 1, helpers.SEED + 43)
    _compare(lib, one, 1, 81)
    assert _status(lib) == _lib.SWQ_OK


def test_noalloc_refuses_layers_beyond_its_array():
    import torch
    lib = _lib.load()
    # top-16 over 1024 experts with 4096-row experts at batch 16: the staged
    # activations alone are 4 MiB
    shape = synth.MoEShape("wide", 128, 1024, 16, 4096, 64, expert_bits=4, router_bits=8, group=64)
    layer = moe.synth_layer(shape, 5, 0)
    x = torch.zeros((16, 128), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((16, 128), dtype=torch.float32, device="cuda")
    ids = torch.empty((16, 16), dtype=torch.int32, device="cuda")
    w = torch.empty((16, 16), dtype=torch.float32, device="cuda")
    assert _noalloc(lib, layer, x, out, ids, w) == _lib.SWQ_ERR_LIMIT


def test_noalloc_dtypes_and_accumulate():
    """f32 activations, bf16 outputs and the accumulate flag, on the single
    launch and the three launches, against swq_moe_decode with the same
    arguments."""
    import torch
    lib = _lib.load()
    layer = moe.synth_layer(synth.SHAPES["qwen3.6-35b-a3b-q4"], helpers.SEED, 0)
    for batch in (1, 3):
        print(f"noalloc dtypes/accumulate: batch {batch}", flush=True)
        xb = helpers.bf16_bits_to_torch(synth.activations_bf16(helpers.SEED + 50 + batch, batch, layer.hidden))
        x32 = xb.float() * 1.25
        ids = torch.empty((batch, layer.top_k), dtype=torch.int32, device="cuda")
        w = torch.empty((batch, layer.top_k), dtype=torch.float32, device="cuda")
        # f32 x -> bf16 out
        ref, ref_ids, ref_w = layer.decode(x32, out_dtype=torch.bfloat16)
        out = torch.full_like(ref, float("nan"))
        _lib.check(_noalloc(lib, layer, x32, out, ids, w), "moe_decode_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(ids, ref_ids) and torch.equal(w, ref_w)
        # bf16 x, accumulate into f32 out that already holds values
        base = torch.linspace(-1.0, 1.0, batch * layer.hidden, device="cuda").reshape(batch, layer.hidden)
        ref_acc = base.clone()
        layer.decode(xb, out=ref_acc, accumulate=True)
        out_acc = base.clone()
        _lib.check(_noalloc(lib, layer, xb, out_acc, ids, w, flags=_lib.SWQ_MOE_ACCUMULATE), "moe_decode_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out_acc, ref_acc)
    assert _status(lib) == _lib.SWQ_OK


def test_noalloc_interleaved_with_norm_step():
    """No-alloc calls between swq_moe_decode_norm calls (their own workspace)
    leave both results as they are alone."""
    import torch
    lib = _lib.load()
    layer = moe.synth_layer(synth.SHAPES["qwen3.6-35b-a3b-q4"], helpers.SEED, 0)
    H = layer.hidden
    g = torch.Generator(device="cpu").manual_seed(7)
    h = (torch.randn(H, generator=g) * 0.5).cuda()
    r = (torch.randn(H, generator=g) * 0.5).cuda()
    nw = (1.0 + 0.1 * torch.randn(H, generator=g)).cuda()
    ws = layer.new_workspace(1)
    ref_norm = layer.decode_norm(h, nw, 1e-6, residual=r, ws=ws)[0].clone()
    xb = helpers.bf16_bits_to_torch(synth.activations_bf16(helpers.SEED + 60, 1, H))
    ref, ref_ids, ref_w = layer.decode(xb)
    out = torch.empty_like(ref)
    ids = torch.empty_like(ref_ids)
    w = torch.empty_like(ref_w)
    for i in range(3):
        print(f"noalloc / decode_norm interleave {i}", flush=True)
        _lib.check(_noalloc(lib, layer, xb, out, ids, w), "moe_decode_noalloc")
        got_norm = layer.decode_norm(h, nw, 1e-6, residual=r, ws=ws)[0]
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(ids, ref_ids)
        assert torch.equal(got_norm, ref_norm)
    assert layer.workspace_status(ws) == _lib.SWQ_OK
    assert _status(lib) == _lib.SWQ_OK


def test_noalloc_replays_under_graph_capture():
    """The entry point captured in a HIP graph (after a first call outside
    capture has set the array up): every replay, with new activations copied
    into the captured input between replays and eager work in between,
    equals swq_moe_decode on the same input."""
    import torch
    lib = _lib.load()
    layer = moe.synth_layer(synth.SHAPES["qwen3.6-35b-a3b-q4"], helpers.SEED, 0)
    H, K = layer.hidden, layer.top_k
    x = torch.zeros((1, H), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((1, H), dtype=torch.float32, device="cuda")
    ids = torch.empty((1, K), dtype=torch.int32, device="cuda")
    w = torch.empty((1, K), dtype=torch.float32, device="cuda")
    _lib.check(_noalloc(lib, layer, x, out, ids, w), "moe_decode_noalloc")  # set-up, outside capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            st = _noalloc(lib, layer, x, out, ids, w, stream=ctypes.c_void_p(side.cuda_stream))
    _lib.check(st, "moe_decode_noalloc under capture")
    for i in range(4):
        print(f"graph replay {i}", flush=True)
        xi = helpers.bf16_bits_to_torch(synth.activations_bf16(helpers.SEED + 70 + i, 1, H))
        x.copy_(xi)
        graph.replay()
        torch.cuda.synchronize()
        ref, ref_ids, ref_w = layer.decode(xi)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(ids, ref_ids)
        assert torch.equal(w, ref_w)
        assert torch.equal(out, ref)
    assert _status(lib) == _lib.SWQ_OK


_FIRST_UNDER_CAPTURE = r"""
import ctypes, sys
import torch
from swiftlet_amd import _lib, moe, synth
from tests import helpers
lib = _lib.load()
layer = moe.synth_layer(synth.SHAPES["qwen3.6-35b-a3b-q4"], helpers.SEED, 0)
H, K = layer.hidden, layer.top_k
x = helpers.bf16_bits_to_torch(synth.activations_bf16(helpers.SEED + 80, 1, H))
out = torch.empty((1, H), dtype=torch.float32, device="cuda")
ids = torch.empty((1, K), dtype=torch.int32, device="cuda")
w = torch.empty((1, K), dtype=torch.float32, device="cuda")
def call(stream=None):
    return lib.swq_moe_decode_noalloc(ctypes.byref(layer._c), x.data_ptr(), _lib.SWQ_BF16, 1, out.data_ptr(),
                                      _lib.SWQ_F32, ids.data_ptr(), w.data_ptr(), 0, stream)
torch.cuda.synchronize()
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        out.add_(0.0)
        st = call(ctypes.c_void_p(side.cuda_stream))
assert st == _lib.SWQ_ERR_INVALID_ARGUMENT, st   # the first call, under capture: refused, nothing latched
_lib.check(call(), "noalloc after capture")       # the set-up runs now
torch.cuda.synchronize()
ref, ref_ids, ref_w = layer.decode(x)
torch.cuda.synchronize()
assert torch.equal(out, ref) and torch.equal(ids, ref_ids) and torch.equal(w, ref_w)
layer.decode(x, path="fused")                     # the device still takes the single launch
assert lib.swq_moe_workspace_status(None, 0, 1, None) == _lib.SWQ_OK
print("first-under-capture: ok", flush=True)
"""


def test_noalloc_first_call_under_capture_recovers():
    """In a fresh process, the very first no-alloc call made under stream
    capture is refused without latching anything: the next call outside
    capture sets the array up and equals swq_moe_decode, and the device
    still takes the single launch (the set-up's probe ran then)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
    print("fresh process: first no-alloc call under capture", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_UNDER_CAPTURE], cwd=root, env=env, capture_output=True,
                       text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "first-under-capture: ok" in r.stdout
