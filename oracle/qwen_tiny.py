"""Whole-model f32 forward of the tiny qwen3_next fixtures — TEST
INFRASTRUCTURE ONLY.

The reference's only vectors that exercise the MoE math (router softmax,
top-k, renormalisation, SwiGLU experts, shared expert gate) and the MLX
affine dequantisation together are mlx's captures of a tiny whole model
(fixtures/tiny_forward*.safetensors).  Reaching the MoE block requires the
rest of each decoder layer, so this module restates QwenCPUModel's
non-MoE ops for that model and delegates the MoE block to
oracle.moe_ref.moe_forward.  Both checkpoint families the reference reads:
qwen3_next (flat config, fused-interleaved DeltaNet projections) and qwen3_5
(config nested under text_config, rope under rope_parameters, split DeltaNet
projections, weights named "language_model.*"):

  config (both families)           QwenConfig.swift:50-105
  "language_model." names          Checkpoint.swift:74-80
  Checkpoint quant spec / dequant  Checkpoint.swift:31-49, 126-133, 168-209
  rms_norm                         QwenCPUModel.swift:47-59
  layer_forward                    QwenCPUModel.swift:259-281
  attention_forward                QwenCPUModel.swift:285-345
  apply_rope                       QwenCPUModel.swift:348-367
  deltanet_forward                 QwenCPUModel.swift:371-496 (split
                                   projections: :415-420)
  forward / greedy                 QwenCPUModel.swift:208-236
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
from safetensors.numpy import load_file

from . import attention_ref as A
from . import deltanet_ref as D
from . import moe_ref as R

f32 = np.float32


def text_config(cfg: dict) -> dict:
    """QwenConfig(url:) (QwenConfig.swift:50-105): the text model's fields
    (nested under text_config in multimodal checkpoints), rope_theta and
    partial_rotary_factor from rope_parameters when present, plus
    "split_layout" (the qwen3_5 family: model_type qwen3_5* / qwen3_6* or a
    nested config) and "weight_prefix" ("language_model." when nested)."""
    text = cfg.get("text_config", cfg)
    nested = "text_config" in cfg
    c = dict(text)
    c["model_type"] = text.get("model_type", cfg.get("model_type", "qwen3_next"))
    c["tie_word_embeddings"] = text.get("tie_word_embeddings", cfg.get("tie_word_embeddings", False))
    rp = text.get("rope_parameters")
    if isinstance(rp, dict):
        c["rope_theta"] = float(rp.get("rope_theta", 10_000_000))
        c["partial_rotary_factor"] = float(rp.get("partial_rotary_factor", 0.25))
    else:
        c["rope_theta"] = float(text["rope_theta"])
        c["partial_rotary_factor"] = float(text.get("partial_rotary_factor", 0.25))
    mt = c["model_type"]
    c["split_layout"] = mt.startswith("qwen3_5") or mt.startswith("qwen3_6") or nested
    c["weight_prefix"] = "language_model." if nested else ""
    return c


class TinyCheckpoint:
    """Checkpoint(dir:) for a single-file mlx checkpoint.  Names resolve as
    given, else with the "language_model." prefix (Checkpoint.swift:74-80)."""

    def __init__(self, directory: Path):
        directory = Path(directory)
        self.cfg = json.loads((directory / "config.json").read_text())
        raw = load_file(str(directory / "model.safetensors"))
        pre = "language_model."
        self.t = dict(raw)
        for k, v in raw.items():
            if k.startswith(pre) and k[len(pre):] not in raw:
                self.t[k[len(pre):]] = v
        q = self.cfg.get("quantization") or {}
        self.default = (q["group_size"], q["bits"]) if "group_size" in q and "bits" in q else None
        self.overrides = {k: (v["group_size"], v["bits"]) for k, v in q.items()
                          if isinstance(v, dict) and "group_size" in v and "bits" in v}

    def is_quantized(self, path: str) -> bool:
        return path + ".scales" in self.t

    def spec(self, path: str):
        for key, s in self.overrides.items():
            if path.endswith(key) or key.endswith(path):
                return s
        return self.default

    def quantized(self, path: str):
        """(words, scales, biases, bits, group) of a quantized module."""
        group, bits = self.spec(path)
        return (self.t[path + ".weight"], self.t[path + ".scales"], self.t[path + ".biases"], bits, group)

    def module_weight(self, path: str) -> np.ndarray:
        if self.is_quantized(path):
            w, s, b, bits, group = self.quantized(path)
            return R.dequantize(w, s.astype(f32), b.astype(f32), bits, group, R.F32)
        return self.t[path + ".weight"].astype(f32)

    def tensor(self, name: str) -> np.ndarray:
        return self.t[name].astype(f32)


class _Dense:
    """Plain f32 matrix (or expert stack) in the QLinear interface the MoE
    oracle consumes."""

    def __init__(self, w: np.ndarray):
        self.w = np.asarray(w, f32)
        self.out_dim, self.in_dim = self.w.shape[-2], self.w.shape[-1]

    def dense(self, expert=None):
        return self.w if expert is None else self.w[expert]


def rms_norm(x: np.ndarray, w, eps: float) -> np.ndarray:
    """QwenCPUModel.rmsNorm (:47-59), rows over the last axis."""
    x = np.asarray(x, f32)
    ss = np.sum(x * x, axis=-1, keepdims=True, dtype=f32)
    scale = f32(1) / np.sqrt(ss / f32(x.shape[-1]) + f32(eps))
    return (x * (scale * w) if w is not None else x * scale).astype(f32)


class TinyQwen:
    def __init__(self, directory: Path):
        self.ck = TinyCheckpoint(directory)
        c = text_config(self.ck.cfg)
        self.c = c
        self.split = c["split_layout"]
        self.D = c["hidden_size"]
        self.eps = c.get("rms_norm_eps", 1e-6)
        self.L = c["num_hidden_layers"]
        self.interval = c.get("full_attention_interval", 4)
        self.embed = self.ck.module_weight("model.embed_tokens")
        self.lm_head = self.embed if c.get("tie_word_embeddings", False) else self.ck.module_weight("lm_head")
        self.final_norm = self.ck.tensor("model.norm.weight")

    def is_linear(self, i: int) -> bool:
        return (i + 1) % self.interval != 0

    # -- MoE ------------------------------------------------------------
    def moe_layer(self, i: int) -> R.MoELayerRef:
        """The layer's MoE weights as the oracle's layer object; quantized
        modules keep their packed form (the experts are dequantised per call)."""
        p = f"model.layers.{i}.mlp."
        ck = self.ck

        def lin(path):
            if ck.is_quantized(path):
                w, s, b, bits, group = ck.quantized(path)
                return R.QLinear(w, s.astype(f32), b.astype(f32), bits, group, R.F32)
            return _Dense(ck.t[path + ".weight"])

        return R.MoELayerRef(
            router=lin(p + "gate"),
            gate=lin(p + "switch_mlp.gate_proj"), up=lin(p + "switch_mlp.up_proj"),
            down=lin(p + "switch_mlp.down_proj"),
            shared_gate=lin(p + "shared_expert.gate_proj"), shared_up=lin(p + "shared_expert.up_proj"),
            shared_down=lin(p + "shared_expert.down_proj"), shared_expert_gate=lin(p + "shared_expert_gate"),
            top_k=self.c["num_experts_per_tok"], norm_topk_prob=bool(self.c.get("norm_topk_prob", False)))

    # -- attention (QwenCPUModel.swift:285-345) ---------------------------
    def attention_params(self, i: int):
        """Layer i's attention shapes and norm weights for attention_core."""
        c, ck = self.c, self.ck
        p = f"model.layers.{i}.self_attn."
        hd = c["head_dim"]
        return dict(q_norm_w=ck.tensor(p + "q_norm.weight"), k_norm_w=ck.tensor(p + "k_norm.weight"),
                    H=c["num_attention_heads"], KVH=c["num_key_value_heads"], hd=hd,
                    rot=int(hd * c["partial_rotary_factor"]), theta=c["rope_theta"], eps=self.eps)

    def attention_projections(self, x: np.ndarray, i: int):
        """q_proj (query | gate per head), k_proj and v_proj outputs."""
        p = f"model.layers.{i}.self_attn."
        ck = self.ck
        return tuple((x @ ck.module_weight(p + n).T).astype(f32) for n in ("q_proj", "k_proj", "v_proj"))

    def attention_forward(self, x: np.ndarray, i: int) -> np.ndarray:
        q_out, k, v = self.attention_projections(x, i)
        out, _, _ = A.attention_core(q_out, k, v, **self.attention_params(i))
        return (out @ self.ck.module_weight(f"model.layers.{i}.self_attn.o_proj").T).astype(f32)

    # -- gated DeltaNet, either projection layout (QwenCPUModel.swift:371-496)
    def deltanet_params(self, i: int):
        """Layer i's DeltaNet shapes and small parameters for deltanet_core."""
        c, ck = self.c, self.ck
        p = f"model.layers.{i}.linear_attn."
        return dict(conv_w=ck.tensor(p + "conv1d.weight"), a_log=ck.tensor(p + "A_log"),
                    dt_bias=ck.tensor(p + "dt_bias"), norm_w=ck.tensor(p + "norm.weight"),
                    nk=c["linear_num_key_heads"], nv=c["linear_num_value_heads"],
                    dk=c["linear_key_head_dim"], dv=c["linear_value_head_dim"], eps=self.eps)

    def deltanet_projections(self, x: np.ndarray, i: int):
        """The projections' outputs: (in_proj_qkvz, in_proj_ba) in the fused
        layout, (in_proj_qkv, in_proj_z, in_proj_b, in_proj_a) in the split."""
        p = f"model.layers.{i}.linear_attn."
        names = ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a") if self.split else ("in_proj_qkvz", "in_proj_ba")
        return tuple((x @ self.ck.module_weight(p + n).T).astype(f32) for n in names)

    def deltanet_inputs(self, x: np.ndarray, i: int):
        """(mixed [q|k|v], z, b, a) of the core: the split layout's
        projections are these already (QwenCPUModel.swift:415-420); the fused
        ones are de-interleaved per key head."""
        prm = self.deltanet_params(i)
        pr = self.deltanet_projections(x, i)
        if self.split:
            return pr
        return D.deinterleave(pr[0], pr[1], prm["nk"], prm["nv"], prm["dk"], prm["dv"])

    def deltanet_forward(self, x: np.ndarray, i: int) -> np.ndarray:
        prm = self.deltanet_params(i)
        mixed, z, b, a = self.deltanet_inputs(x, i)
        y, _, _ = D.deltanet_core(mixed, z, b, a, **prm)
        return (y @ self.ck.module_weight(f"model.layers.{i}.linear_attn.out_proj").T).astype(f32)

    # -- layer / model ------------------------------------------------------
    def layer_forward(self, h: np.ndarray, i: int) -> np.ndarray:
        """norm -> (DeltaNet | attention) -> residual -> norm -> MoE -> residual."""
        ck = self.ck
        p = f"model.layers.{i}."
        x = rms_norm(h, ck.tensor(p + "input_layernorm.weight"), self.eps)
        r = self.deltanet_forward(x, i) if self.is_linear(i) else self.attention_forward(x, i)
        h = (h + r).astype(f32)
        x2 = rms_norm(h, ck.tensor(p + "post_attention_layernorm.weight"), self.eps)
        m, _, _ = R.moe_forward(x2, self.moe_layer(i))
        return (h + m).astype(f32)

    def moe_input(self, h: np.ndarray, i: int) -> np.ndarray:
        """The MoE block's input inside layer i for layer input h."""
        ck = self.ck
        p = f"model.layers.{i}."
        x = rms_norm(h, ck.tensor(p + "input_layernorm.weight"), self.eps)
        r = self.deltanet_forward(x, i) if self.is_linear(i) else self.attention_forward(x, i)
        h = (h + r).astype(f32)
        return rms_norm(h, ck.tensor(p + "post_attention_layernorm.weight"), self.eps)

    def forward(self, tokens):
        h = self.embed[np.asarray(tokens)].astype(f32)
        layers = []
        for i in range(self.L):
            h = self.layer_forward(h, i)
            layers.append(h)
        hn = rms_norm(h, self.final_norm, self.eps)
        logits = (hn @ self.lm_head.T).astype(f32)
        return logits, layers, np.argmax(logits, axis=-1)
