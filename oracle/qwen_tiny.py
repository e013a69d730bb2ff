"""Whole-model f32 forward of the tiny qwen3_next fixtures — TEST
INFRASTRUCTURE ONLY.

The reference's only vectors that exercise the MoE math (router softmax,
top-k, renormalisation, SwiGLU experts, shared expert gate) and the MLX
affine dequantisation together are mlx's captures of a tiny whole model
(fixtures/tiny_forward*.safetensors).  Reaching the MoE block requires the
rest of each decoder layer, so this module restates QwenCPUModel's
non-MoE ops for that model (qwen3_next, fused-interleaved DeltaNet layout)
and delegates the MoE block to oracle.moe_ref.moe_forward:

  Checkpoint quant spec / dequant  Checkpoint.swift:31-49, 126-133, 168-209
  rms_norm                         QwenCPUModel.swift:47-59
  layer_forward                    QwenCPUModel.swift:259-281
  attention_forward                QwenCPUModel.swift:285-345
  apply_rope                       QwenCPUModel.swift:348-367
  deltanet_forward                 QwenCPUModel.swift:371-496
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


class TinyCheckpoint:
    """Checkpoint(dir:) for a single-file mlx checkpoint."""

    def __init__(self, directory: Path):
        directory = Path(directory)
        self.cfg = json.loads((directory / "config.json").read_text())
        self.t = load_file(str(directory / "model.safetensors"))
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
        c = self.ck.cfg
        self.c = c
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
                    rot=int(hd * c.get("partial_rotary_factor", 0.25)), theta=float(c["rope_theta"]), eps=self.eps)

    def attention_projections(self, x: np.ndarray, i: int):
        """q_proj (query | gate per head), k_proj and v_proj outputs."""
        p = f"model.layers.{i}.self_attn."
        ck = self.ck
        return tuple((x @ ck.module_weight(p + n).T).astype(f32) for n in ("q_proj", "k_proj", "v_proj"))

    def attention_forward(self, x: np.ndarray, i: int) -> np.ndarray:
        q_out, k, v = self.attention_projections(x, i)
        out, _, _ = A.attention_core(q_out, k, v, **self.attention_params(i))
        return (out @ self.ck.module_weight(f"model.layers.{i}.self_attn.o_proj").T).astype(f32)

    # -- gated DeltaNet, fused interleaved layout (QwenCPUModel.swift:371-496)
    def deltanet_params(self, i: int):
        """Layer i's DeltaNet shapes and small parameters for deltanet_core."""
        c, ck = self.c, self.ck
        p = f"model.layers.{i}.linear_attn."
        return dict(conv_w=ck.tensor(p + "conv1d.weight"), a_log=ck.tensor(p + "A_log"),
                    dt_bias=ck.tensor(p + "dt_bias"), norm_w=ck.tensor(p + "norm.weight"),
                    nk=c["linear_num_key_heads"], nv=c["linear_num_value_heads"],
                    dk=c["linear_key_head_dim"], dv=c["linear_value_head_dim"], eps=self.eps)

    def deltanet_projections(self, x: np.ndarray, i: int):
        """The fused projections' outputs (in_proj_qkvz, in_proj_ba)."""
        p = f"model.layers.{i}.linear_attn."
        return (x @ self.ck.module_weight(p + "in_proj_qkvz").T).astype(f32), \
            (x @ self.ck.module_weight(p + "in_proj_ba").T).astype(f32)

    def deltanet_forward(self, x: np.ndarray, i: int) -> np.ndarray:
        prm = self.deltanet_params(i)
        qkvz, ba = self.deltanet_projections(x, i)
        mixed, z, b, a = D.deinterleave(qkvz, ba, prm["nk"], prm["nv"], prm["dk"], prm["dv"])
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
