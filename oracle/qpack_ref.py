"""The .qpack container writer, restated from QpackRepacker.repack
(Qpack.swift:64-165) — TEST INFRASTRUCTURE ONLY: tests/ use it to turn the
reference's tiny checkpoints into containers that the library's loader then
reads; the product path never imports it.

Also a raw safetensors reader and writer (SafetensorsFile, Safetensors.swift:
the 8-byte little-endian header length, the JSON header of name -> dtype,
shape, data_offsets relative to the data start, then the bytes; the writer
of :97-115 packs tensors back to back with no padding)."""

from __future__ import annotations

import json
import shutil
import struct
from pathlib import Path

PAGE_ALIGNMENT = 16384  # Qpack.pageAlignment (Qpack.swift:19)
EXPERT_SUFFIXES = ("gate_proj", "up_proj", "down_proj")  # Qpack.swift:62
ELEM = {"BOOL": 1, "U8": 1, "I8": 1, "F8_E5M2": 1, "F8_E4M3": 1, "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
        "I32": 4, "U32": 4, "F32": 4, "I64": 8, "U64": 8, "F64": 8}


def read_safetensors(path: Path) -> dict[str, tuple[str, list[int], bytes]]:
    """name -> (dtype, shape, raw bytes) of one safetensors file."""
    data = Path(path).read_bytes()
    (n,) = struct.unpack("<Q", data[:8])
    header = json.loads(data[8:8 + n])
    out = {}
    for name, t in header.items():
        if name == "__metadata__":
            continue
        b, e = t["data_offsets"]
        out[name] = (t["dtype"], list(t["shape"]), data[8 + n + b:8 + n + e])
    return out


def write_safetensors(path: Path, tensors: list[tuple[str, str, list[int], bytes]]) -> None:
    """SafetensorsFile.write (Safetensors.swift:97-115): tensors back to back."""
    header, off = {}, 0
    for name, dtype, shape, raw in tensors:
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    h = json.dumps(header, sort_keys=True, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for _, _, _, raw in tensors:
            f.write(raw)


def read_checkpoint(ckpt_dir: Path) -> dict[str, tuple[str, list[int], bytes]]:
    """Every tensor of model.safetensors or of the shards an index maps."""
    ckpt_dir = Path(ckpt_dir)
    index = ckpt_dir / "model.safetensors.index.json"
    if index.exists():
        out = {}
        for shard in sorted(set(json.loads(index.read_text())["weight_map"].values())):
            out.update(read_safetensors(ckpt_dir / shard))
        return out
    return read_safetensors(ckpt_dir / "model.safetensors")


def repack(ckpt_dir: Path, out_dir: Path) -> dict:
    """QpackRepacker.repack: the expert section table from layer 0's stacked
    switch_mlp tensors (gate/up/down x weight/scales/biases, absent ones
    skipped, :72-93), stride = the payload rounded up to 16 KiB (:94), one
    layer_NN.bin of E blobs per layer (:106-123), layout.json (:125-127),
    the dense model.safetensors without experts, MTP or vision tensors
    (:129-140), the config and tokenizer files (:142-150), manifest.json
    (:152-161).  Returns the layout."""
    ckpt_dir, out_dir = Path(ckpt_dir), Path(out_dir)
    cfg = json.loads((ckpt_dir / "config.json").read_text())
    E, L = cfg["num_experts"], cfg["num_hidden_layers"]
    interval = cfg.get("full_attention_interval", 4)
    tensors = read_checkpoint(ckpt_dir)
    experts_dir = out_dir / "packed_experts"
    experts_dir.mkdir(parents=True, exist_ok=True)

    l0 = "model.layers.0.mlp.switch_mlp."
    sections, offset = [], 0
    for proj in EXPERT_SUFFIXES:
        for part in ("weight", "scales", "biases"):
            name = l0 + proj + "." + part
            if name not in tensors:
                continue
            dtype, shape, _ = tensors[name]
            assert shape[0] == E, name
            per_shape = shape[1:]
            size = ELEM[dtype]
            for d in per_shape:
                size *= d
            sections.append({"name": proj + "." + part, "dtype": dtype, "shape": per_shape,
                             "offset": offset, "size": size})
            offset += size
    stride = (offset + PAGE_ALIGNMENT - 1) // PAGE_ALIGNMENT * PAGE_ALIGNMENT
    layout = {"expertCount": E, "layerCount": L, "expertStride": stride, "sections": sections,
              "linearLayers": [(i + 1) % interval != 0 for i in range(L)]}

    files = {}
    for layer in range(L):
        prefix = f"model.layers.{layer}.mlp.switch_mlp."
        blob = bytearray(stride * E)
        for s in sections:
            dtype, shape, raw = tensors[prefix + s["name"]]
            assert shape[0] == E
            n = s["size"]
            for e in range(E):
                blob[e * stride + s["offset"]:e * stride + s["offset"] + n] = raw[e * n:(e + 1) * n]
        name = f"layer_{layer:02d}.bin"
        (experts_dir / name).write_bytes(bytes(blob))
        files["packed_experts/" + name] = len(blob)
    layout_bytes = json.dumps(layout, sort_keys=True, indent=2).encode()
    (experts_dir / "layout.json").write_bytes(layout_bytes)
    files["packed_experts/layout.json"] = len(layout_bytes)

    dense = []
    for name in sorted(tensors):
        if ".mlp.switch_mlp." in name or name.startswith("mtp.") or ".mtp." in name:
            continue
        if name.startswith("vision_tower.") or "model.visual" in name:
            continue
        dtype, shape, raw = tensors[name]
        dense.append((name, dtype, shape, raw))
    write_safetensors(out_dir / "model.safetensors", dense)
    files["model.safetensors"] = (out_dir / "model.safetensors").stat().st_size

    for aux in ("config.json", "tokenizer.json", "tokenizer_config.json", "vocab.json", "merges.txt",
                "added_tokens.json", "special_tokens_map.json", "chat_template.jinja"):
        src = ckpt_dir / aux
        if src.exists():
            shutil.copyfile(src, out_dir / aux)
            files[aux] = (out_dir / aux).stat().st_size

    q = cfg.get("quantization") or {}
    manifest = {"magic": "QPACK", "version": 1, "modelName": cfg.get("model_type", ""),
                "sourceCheckpoint": ckpt_dir.name, "files": files}
    if "bits" in q:
        manifest["quantBits"] = q["bits"]
    if "group_size" in q:
        manifest["quantGroupSize"] = q["group_size"]
    (out_dir / "manifest.json").write_text(json.dumps(manifest, sort_keys=True, indent=2))
    return layout
