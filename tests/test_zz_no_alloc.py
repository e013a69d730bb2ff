"""swq_moe_decode_noalloc, the variant of swq_moe_decode whose workspace is a
static device array inside the library, against swq_moe_decode itself (a
workspace of its own per layer): equal bit for bit on two calls in a row, the
second with a smaller input (batch 4 on the three launches, then batch 1 on
the single launch), then a different, smaller layer sharing the same array,
then the first layer again.  A layer whose workspace exceeds the array is
refused before any launch."""

import ctypes

import pytest

from swiftlet_amd import _lib, moe, synth
from tests import helpers

pytestmark = pytest.mark.gpu


def _noalloc(lib, layer, x, out, ids, w):
    return lib.swq_moe_decode_noalloc(ctypes.byref(layer._c), x.data_ptr(), _lib.SWQ_BF16, x.shape[0],
                                      out.data_ptr(), _lib.SWQ_F32, ids.data_ptr(), w.data_ptr(), 0, None)


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
    _compare(lib, big, 1, helpers.SEED + 43)


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
