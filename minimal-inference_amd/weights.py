"""HuggingFace safetensors checkpoints into ``model.Model``.

The reference loads Qwen2 / Mistral checkpoints by HF parameter name
(model.py:443-474; it globs every shard and warns on missing names,
this loader raises).  ``Model`` keeps q/k/v and gate/up fused, so each HF
tensor is copied into its rows of the fused weight:

  model.embed_tokens.weight                  -> embed
  model.layers.N.input_layernorm.weight      -> layers[N].in_norm
  model.layers.N.self_attn.{q,k,v}_proj.*    -> layers[N].w_qkv / b_qkv rows
                                                [0, Hq*D) / [Hq*D, (Hq+Hkv)*D) / [(Hq+Hkv)*D, ...)
  model.layers.N.self_attn.o_proj.weight     -> layers[N].w_o
  model.layers.N.post_attention_layernorm.*  -> layers[N].post_norm
  model.layers.N.mlp.{gate,up}_proj.weight   -> layers[N].w_gate_up rows [0, I) / [I, 2I)
  model.layers.N.mlp.down_proj.weight        -> layers[N].w_down
  model.norm.weight                          -> norm
  lm_head.weight                             -> lm_head (absent when tied)

Only safetensors files are read (no pickle).  Every tensor the model needs
must be present once; unknown names (rotary caches and the like) are
ignored.
"""

from __future__ import annotations

import json
import os
import re

import torch

_LAYER = re.compile(r"^model\.layers\.(\d+)\.(.+)$")


def checkpoint_files(model_path: str) -> list[str]:
    """The safetensors shards of a checkpoint directory (index file order)."""
    index = os.path.join(model_path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            shards = sorted(set(json.load(f)["weight_map"].values()))
        return [os.path.join(model_path, s) for s in shards]
    single = os.path.join(model_path, "model.safetensors")
    if os.path.exists(single):
        return [single]
    found = sorted(x for x in os.listdir(model_path) if x.endswith(".safetensors"))
    if not found:
        raise FileNotFoundError(f"no .safetensors files in {model_path}")
    return [os.path.join(model_path, x) for x in found]


def _targets(model) -> dict[str, tuple[torch.Tensor, int, int]]:
    """HF name -> (destination tensor, first row, row count)."""
    cfg = model.cfg
    nq, nkv, d, inter = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size
    out = {"model.embed_tokens.weight": (model.embed, 0, cfg.vocab_size),
           "model.norm.weight": (model.norm, 0, cfg.hidden_size)}
    if model.lm_head is not model.embed:
        out["lm_head.weight"] = (model.lm_head, 0, cfg.vocab_size)
    spans = {"q": (0, nq * d), "k": (nq * d, nkv * d), "v": ((nq + nkv) * d, nkv * d)}
    for i, L in enumerate(model.layers):
        p = f"model.layers.{i}."
        out[p + "input_layernorm.weight"] = (L.in_norm, 0, cfg.hidden_size)
        out[p + "post_attention_layernorm.weight"] = (L.post_norm, 0, cfg.hidden_size)
        for name, (r0, n) in spans.items():
            out[p + f"self_attn.{name}_proj.weight"] = (L.w_qkv, r0, n)
            if L.b_qkv is not None:
                out[p + f"self_attn.{name}_proj.bias"] = (L.b_qkv, r0, n)
        out[p + "self_attn.o_proj.weight"] = (L.w_o, 0, cfg.hidden_size)
        out[p + "mlp.gate_proj.weight"] = (L.w_gate_up, 0, inter)
        out[p + "mlp.up_proj.weight"] = (L.w_gate_up, inter, inter)
        out[p + "mlp.down_proj.weight"] = (L.w_down, 0, cfg.hidden_size)
    return out


def load_weights(model, model_path: str) -> None:
    """Copy a checkpoint's tensors into ``model`` (cast to the model dtype)."""
    from safetensors import safe_open

    targets = _targets(model)
    seen: set[str] = set()
    for path in checkpoint_files(model_path):
        with safe_open(path, framework="pt", device="cpu") as f:
            for name in f.keys():
                if name not in targets:
                    m = _LAYER.match(name)
                    if m and int(m.group(1)) >= len(model.layers):
                        raise ValueError(f"{name}: checkpoint has more layers than the config")
                    continue
                if name in seen:
                    raise ValueError(f"{name} appears in more than one shard")
                dst, r0, n = targets[name]
                src = f.get_tensor(name)
                want = (n,) + tuple(dst.shape[1:])
                if tuple(src.shape) != want:
                    raise ValueError(f"{name}: shape {tuple(src.shape)}, expected {want}")
                dst[r0: r0 + n].copy_(src.to(dst.dtype))
                seen.add(name)
    missing = sorted(set(targets) - seen)
    if missing:
        raise ValueError(f"checkpoint lacks {len(missing)} tensors, e.g. {missing[:3]}")
