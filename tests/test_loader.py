"""Checkpoint and .qpack reading without a GPU (swq_checkpoint_* /
swq_qpack_* host functions).

The reference's own round trip (QpackTests.repackRoundTrip,
QpackTests.swift:15-63): the tiny 4-bit checkpoint repacked into a
container (the oracle's restatement of QpackRepacker), every expert blob
byte-identical to the checkpoint's slices, the dense file readable with the
same bytes and without the expert tensors, the stride a 16 KiB multiple,
gate_proj.weight's per-expert shape [I, H/8].  Beyond it: every tensor's
dtype/shape/bytes against an independent Python parse of the files, a
sharded checkpoint with an index and "language_model." names
(Checkpoint.swift:50-80), the quantization overrides (:31-47, :111-120), and
the failure modes (missing files and tensors, truncated or inconsistent
headers, a stride off the page size, a layer file of the wrong size, a
foreign manifest)."""

import json
import shutil
import struct
from pathlib import Path

import pytest

from oracle import qpack_ref as Q
from swiftlet_amd import _lib
from swiftlet_amd.checkpoint import Checkpoint, QpackExpertReader

FIXTURES = Path(__file__).resolve().parent / "golden" / "swiftlet_fixtures"
Q4 = FIXTURES / "tiny-model-q4"
F32 = FIXTURES / "tiny-model"


@pytest.fixture(scope="module")
def container(tmp_path_factory):
    out = tmp_path_factory.mktemp("qpack") / "tiny-q4.qpack"
    Q.repack(Q4, out)
    return out


@pytest.mark.parametrize("ckpt_dir", [Q4, F32], ids=["q4", "f32"])
def test_tensor_infos_and_bytes_match_the_files(ckpt_dir):
    want = Q.read_checkpoint(ckpt_dir)
    c = Checkpoint(ckpt_dir)
    assert sorted(c.tensor_names) == sorted(want)
    for name, (dtype, shape, raw) in want.items():
        ti = c.info(name)
        assert (ti.dtype, list(ti.shape), ti.nbytes) == (dtype, shape, len(raw)), name
        assert c.raw_tensor(name) == raw, name


@pytest.mark.parametrize("name", ["tiny-model-q4/model.safetensors", "tiny-model/model.safetensors",
                                  "tiny_forward_q4.safetensors"])
def test_oracle_reader_matches_the_safetensors_package(name):
    """The test-side parse itself, against the safetensors package's loader."""
    import numpy as np
    from safetensors.numpy import load_file
    want = load_file(str(FIXTURES / name))
    got = Q.read_safetensors(FIXTURES / name)
    assert sorted(got) == sorted(want)
    for k, arr in want.items():
        dtype, shape, raw = got[k]
        assert list(arr.shape) == shape and arr.dtype.itemsize == Q.ELEM[dtype], k
        assert np.ascontiguousarray(arr).tobytes() == raw, k


def test_quant_specs_follow_config():
    c = Checkpoint(Q4)
    cfg = json.loads((Q4 / "config.json").read_text())["quantization"]
    spec = (cfg["group_size"], cfg["bits"])
    assert c.quant_spec("model.layers.0.mlp.gate") == spec
    assert c.quant_spec("model.layers.3.self_attn.q_proj") == spec
    assert c.quant_spec("model.layers.0.mlp.switch_mlp.down_proj") == spec
    assert c.quant_spec("model.layers.0.input_layernorm") is None  # stored plain
    assert c.quant_spec("model.layers.0.no_such_module") is None
    assert Checkpoint(F32).quant_spec("model.layers.0.mlp.gate") is None


def test_quant_overrides_most_specific_key_wins(tmp_path):
    shutil.copyfile(Q4 / "model.safetensors", tmp_path / "model.safetensors")
    cfg = json.loads((Q4 / "config.json").read_text())
    cfg["quantization"] = {"group_size": 32, "bits": 4, "mlp.gate": {"group_size": 64, "bits": 8},
                           "model.layers.0.mlp.gate": {"group_size": 128, "bits": 2}}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    c = Checkpoint(tmp_path)
    assert c.quant_spec("model.layers.0.mlp.gate") == (128, 2)
    assert c.quant_spec("model.layers.1.mlp.gate") == (64, 8)
    assert c.quant_spec("model.layers.1.mlp.shared_expert.up_proj") == (32, 4)


def test_sharded_checkpoint_with_prefixed_names(tmp_path):
    tensors = Q.read_checkpoint(Q4)
    names = sorted(tensors)
    shards = {"model-00001-of-00002.safetensors": names[::2], "model-00002-of-00002.safetensors": names[1::2]}
    weight_map = {}
    for fname, part in shards.items():
        rows = []
        for n in part:
            stored = "language_model." + n if n.startswith("model.layers.1.") else n
            rows.append((stored, *tensors[n]))
            weight_map[stored] = fname
        Q.write_safetensors(tmp_path / fname, rows)
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    shutil.copyfile(Q4 / "config.json", tmp_path / "config.json")
    c = Checkpoint(tmp_path)
    assert len(c.tensor_names) == len(names)
    for n in names:
        assert c.raw_tensor(n) == tensors[n][2], n  # unprefixed name resolves
    assert c.contains("language_model.model.layers.1.mlp.gate.weight")
    assert c.quant_spec("model.layers.1.mlp.gate") == (32, 4)


def test_qwen35_checkpoint_resolves_unprefixed_names():
    """The tiny qwen3_5 fixture stores every weight as language_model.*: each
    resolves by its unprefixed name with the stored bytes, and it holds the
    split DeltaNet projections the loader's layout choice looks for."""
    from safetensors.numpy import load_file
    d = FIXTURES / "tiny-model-q35"
    raw = load_file(str(d / "model.safetensors"))
    c = Checkpoint(d)
    assert len(c.tensor_names) == len(raw)
    for stored, arr in raw.items():
        assert stored.startswith("language_model.")
        n = stored[len("language_model."):]
        assert c.raw_tensor(n) == arr.tobytes(), n
    assert c.contains("model.layers.0.linear_attn.in_proj_qkv.weight")
    assert not c.contains("model.layers.0.linear_attn.in_proj_qkvz.weight")
    assert c.quant_spec("model.layers.0.mlp.gate") is None  # stored unquantized


def test_repack_round_trip(container):
    """QpackTests.repackRoundTrip (QpackTests.swift:15-63)."""
    cfg = json.loads((Q4 / "config.json").read_text())
    ck = Checkpoint(Q4)
    r = QpackExpertReader(container)
    assert r.expert_count == cfg["num_experts"]
    assert r.layer_count == cfg["num_hidden_layers"]
    assert r.expert_stride % 16384 == 0
    assert (r.quant_bits, r.quant_group_size) == (cfg["quantization"]["bits"], cfg["quantization"]["group_size"])
    assert [s.name for s in r.sections] == [f"{p}.{k}" for p in ("gate_proj", "up_proj", "down_proj")
                                          for k in ("weight", "scales", "biases")]
    for layer in range(r.layer_count):  # every blob (the reference samples 2 layers x 3 experts)
        for e in range(r.expert_count):
            blob = r.read_expert(layer, e)
            assert len(blob) == r.expert_stride
            for s in r.sections:
                full = ck.raw_tensor(f"model.layers.{layer}.mlp.switch_mlp.{s.name}")
                assert blob[s.offset:s.offset + s.size] == full[e * s.size:(e + 1) * s.size], (layer, e, s.name)
            end = r.sections[-1].offset + r.sections[-1].size
            assert blob[end:] == bytes(r.expert_stride - end)  # padding is zero
    packed = Checkpoint(container)
    for name in ("model.embed_tokens.weight", "model.layers.0.input_layernorm.weight",
                 "model.layers.0.mlp.gate.scales", "model.layers.3.self_attn.q_norm.weight"):
        a, b = ck.info(name), packed.info(name)
        assert ck.raw_tensor(name) == packed.raw_tensor(name) and a.dtype == b.dtype, name
    assert not packed.contains("model.layers.0.mlp.switch_mlp.gate_proj.weight")
    assert r.section("gate_proj.weight").shape == (cfg["moe_intermediate_size"], cfg["hidden_size"] // 8)
    assert r.section("no_such.weight") is None
    assert [r.is_linear_layer(i) for i in range(r.layer_count)] == \
        [(i + 1) % cfg["full_attention_interval"] != 0 for i in range(r.layer_count)]


def test_json_strings_numbers_and_escapes(tmp_path):
    """Header names with escapes and non-ASCII text; numbers in exponent form."""
    name = "café.\U0001F600.w\"q\\x"
    Q.write_safetensors(tmp_path / "model.safetensors", [(name, "F32", [2], struct.pack("<2f", 1.0, 2.0))])
    raw = (tmp_path / "model.safetensors").read_bytes()
    (n,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + n])
    text = json.dumps(header, ensure_ascii=True).encode()  # \u escapes, a surrogate pair
    assert b"\\ud83d\\ude00" in text
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", len(text)) + text + raw[8 + n:])
    (tmp_path / "config.json").write_text('{"rms_norm_eps": 1e-06, "rope_theta": 1.0E+7, "x": [true, false, null]}')
    c = Checkpoint(tmp_path)
    assert c.tensor_names == [name]
    assert c.raw_tensor(name) == struct.pack("<2f", 1.0, 2.0)


def _status(fn):
    with pytest.raises(_lib.SwqError) as e:
        fn()
    return e.value.code


def test_checkpoint_failure_modes(tmp_path):
    assert _status(lambda: Checkpoint(tmp_path / "absent")) == _lib.SWQ_ERR_IO
    c = Checkpoint(Q4)
    assert _status(lambda: c.info("no.such.tensor")) == _lib.SWQ_ERR_MISSING_TENSOR
    assert _status(lambda: c.raw_tensor("no.such.tensor")) == _lib.SWQ_ERR_MISSING_TENSOR
    lib = _lib.load()
    assert lib.swq_checkpoint_linear_bytes(c._h, b"model.layers.0.input_layernorm") == _lib.SWQ_ERR_UNSUPPORTED_BITS
    assert lib.swq_checkpoint_linear_bytes(c._h, b"model.layers.0.no_such") == _lib.SWQ_ERR_MISSING_TENSOR
    assert lib.swq_checkpoint_linear_bytes(c._h, b"model.layers.0.mlp.gate") > 0

    good = (Q4 / "model.safetensors").read_bytes()
    (n,) = struct.unpack("<Q", good[:8])
    header = json.loads(good[8:8 + n])

    def write(dirname, data, cfg=True):
        d = tmp_path / dirname
        d.mkdir()
        (d / "model.safetensors").write_bytes(data)
        if cfg:
            shutil.copyfile(Q4 / "config.json", d / "config.json")
        return d

    assert _status(lambda: Checkpoint(write("short", good[:5]))) == _lib.SWQ_ERR_FORMAT
    assert _status(lambda: Checkpoint(write("trunc", good[:8 + n // 2]))) == _lib.SWQ_ERR_FORMAT
    assert _status(lambda: Checkpoint(write("len", struct.pack("<Q", 1 << 40) + good[8:]))) == _lib.SWQ_ERR_FORMAT
    bad = dict(header)
    k = "model.layers.0.mlp.gate.weight"
    bad[k] = dict(bad[k], shape=[8, 9])  # bytes no longer match the shape
    hb = json.dumps(bad).encode()
    assert _status(lambda: Checkpoint(write("shape", struct.pack("<Q", len(hb)) + hb + good[8 + n:]))) == \
        _lib.SWQ_ERR_FORMAT
    assert _status(lambda: Checkpoint(write("data", good[:-16]))) == _lib.SWQ_ERR_FORMAT  # data past the end
    d = write("cfg", good, cfg=False)
    (d / "config.json").write_text("{\"quantization\": {\"bits\": 4,}}")
    assert _status(lambda: Checkpoint(d)) == _lib.SWQ_ERR_FORMAT
    d = tmp_path / "index"
    d.mkdir()
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"a": "missing.safetensors"}}))
    assert _status(lambda: Checkpoint(d)) == _lib.SWQ_ERR_IO


def test_qpack_failure_modes(container, tmp_path):
    assert _status(lambda: QpackExpertReader(tmp_path / "absent")) == _lib.SWQ_ERR_IO

    def variant(name, edit_layout=None, edit_manifest=None):
        d = tmp_path / name
        shutil.copytree(container, d)
        if edit_layout:
            p = d / "packed_experts" / "layout.json"
            lay = json.loads(p.read_text())
            edit_layout(lay)
            p.write_text(json.dumps(lay))
        if edit_manifest:
            p = d / "manifest.json"
            m = json.loads(p.read_text())
            edit_manifest(m)
            p.write_text(json.dumps(m))
        return d

    assert _status(lambda: QpackExpertReader(variant("stride", lambda l: l.update(expertStride=16000)))) == \
        _lib.SWQ_ERR_FORMAT

    def past_blob(lay):
        lay["sections"][-1]["offset"] = lay["expertStride"] - 8
    assert _status(lambda: QpackExpertReader(variant("past", past_blob))) == _lib.SWQ_ERR_FORMAT
    assert _status(lambda: QpackExpertReader(variant("magic", edit_manifest=lambda m: m.update(magic="GTURBO")))) == \
        _lib.SWQ_ERR_FORMAT
    d = variant("short")
    f = d / "packed_experts" / "layer_02.bin"
    f.write_bytes(f.read_bytes()[:-1])
    r = QpackExpertReader(d)
    assert _status(lambda: r.read_expert(2, 0)) == _lib.SWQ_ERR_FORMAT
    assert r.read_expert(1, 0) == QpackExpertReader(container).read_expert(1, 0)
    assert _status(lambda: r.read_expert(r.layer_count, 0)) == _lib.SWQ_ERR_INVALID_ARGUMENT
    assert _status(lambda: r.read_expert(0, r.expert_count)) == _lib.SWQ_ERR_INVALID_ARGUMENT
    (d / "packed_experts" / "layer_03.bin").unlink()
    assert _status(lambda: r.read_expert(3, 0)) == _lib.SWQ_ERR_IO
