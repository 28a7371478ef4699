"""Safetensors loading into a decoder (nanovllm/utils/loader.py:8-34).

``load_model`` walks every ``*.safetensors`` of a local model directory
and copies each tensor into the parameter of the same name, through the
parameter's ``weight_loader`` when it has one; q/k/v and gate/up tensors are
routed to the fused parameter with their shard id by
``model.packed_modules_mapping``, as in the reference.  GPTQ checkpoints
(``qweight``/``qzeros``/``scales`` per projection, ``g_idx`` skipped) load the
same way into ``W4A16Qwen3ForCausalLM``, whose mapping is empty;
``load_w4a16_model`` then concatenates q/k/v and gate/up along N
(``fuse_projections_``).  ``write_gptq_checkpoint`` writes a synthetic
checkpoint in that format (random codes, zeros and scales) for tests and
benchmarks.
"""
from __future__ import annotations

import os
from glob import glob

import torch
from safetensors import safe_open
from torch import nn


def default_weight_loader(param: nn.Parameter, loaded_weight: torch.Tensor):
    param.data.copy_(loaded_weight)


def resolve_model_path(path: str) -> str:
    """A local directory as given, else the local Hugging Face cache entry
    for a repository id (never a download)."""
    if os.path.isdir(path):
        return path
    from huggingface_hub import snapshot_download
    return snapshot_download(repo_id=path, local_files_only=True)


def _destination(weight_name: str, mapping: dict):
    """(parameter name, shard id) a checkpoint tensor is loaded into: the
    first ``packed_modules_mapping`` key contained in the name routes it to
    the fused parameter with that key's shard id; any other tensor goes to
    the parameter of its own name (shard id None)."""
    key = next((k for k in mapping if k in weight_name), None)
    if key is None:
        return weight_name, None
    fused, shard_id = mapping[key]
    return weight_name.replace(key, fused), shard_id


def checkpoint_tensors(root: str):
    """(name, CPU tensor) for every tensor of every ``*.safetensors`` file
    under ``root``, file by file in name order; GPTQ ``g_idx`` tensors
    (static groups: always k // 128) are not yielded."""
    for path in sorted(glob(os.path.join(root, "*.safetensors"))):
        with safe_open(path, "pt", "cpu") as f:
            for name in f.keys():
                if not name.endswith(".g_idx"):
                    yield name, f.get_tensor(name)


def load_model(model: nn.Module, path: str) -> None:
    """Copy every checkpoint tensor into ``model``: fused q/k/v and gate/up
    parameters through their ``weight_loader`` with the shard id, the rest
    through theirs (or a plain copy)."""
    mapping = getattr(model, "packed_modules_mapping", {})
    for name, tensor in checkpoint_tensors(resolve_model_path(path)):
        target, shard_id = _destination(name, mapping)
        param = model.get_parameter(target)
        if shard_id is None:
            getattr(param, "weight_loader", default_weight_loader)(param, tensor)
        else:
            param.weight_loader(param, tensor, shard_id)


def load_w4a16_model(model: nn.Module, path: str) -> nn.Module:
    """GPTQ checkpoint into a W4A16Qwen3ForCausalLM, then the N-concatenated
    q/k/v and gate/up projections (the reference's use_w4a16 path,
    nanovllm/engine/model_runner.py:35-37 with nanovllm/utils/loader.py:12-34)."""
    load_model(model, path)
    return model.fuse_projections_()


def gptq_tensors(in_features: int, out_features: int, gen: torch.Generator) -> dict:
    """Random GPTQ tensors of one projection: qweight int32 [in/8, out] and
    qzeros int32 [in/128, out/8] with uniform nibbles, fp16 scales
    [in/128, out] uniform in [0.005, 0.02], g_idx int32 [in] (= k // 128)."""
    return {
        "qweight": torch.randint(-2**31, 2**31, (in_features // 8, out_features), generator=gen, dtype=torch.int64).to(
            torch.int32),
        "qzeros": torch.randint(-2**31, 2**31, (in_features // 128, out_features // 8), generator=gen,
                                dtype=torch.int64).to(torch.int32),
        "scales": (0.005 + 0.015 * torch.rand(in_features // 128, out_features, generator=gen)).to(torch.float16),
        "g_idx": torch.arange(in_features, dtype=torch.int32) // 128,
    }


def write_gptq_checkpoint(root, cfg, seed: int = 0) -> str:
    """A GPTQ (group 128) Qwen3 checkpoint in the layout the reference's
    W4A16 model loads: bf16 embeddings, norms and LM head, GPTQ tensors for
    q/k/v/o/gate/up/down of every layer, and config.json."""
    import json
    from pathlib import Path

    from safetensors.torch import save_file
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    g = torch.Generator().manual_seed(seed)
    h, inter = cfg.hidden_size, cfg.intermediate_size
    hd = getattr(cfg, "head_dim", None) or h // cfg.num_attention_heads
    q, kv = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
    t = {"model.embed_tokens.weight": (torch.randn(cfg.vocab_size, h, generator=g) * 0.02).to(torch.bfloat16),
         "model.norm.weight": torch.ones(h, dtype=torch.bfloat16),
         "lm_head.weight": (torch.randn(cfg.vocab_size, h, generator=g) * 0.02).to(torch.bfloat16)}
    for i in range(cfg.num_hidden_layers):
        pre = f"model.layers.{i}."
        for name, (fi, fo) in {"self_attn.q_proj": (h, q), "self_attn.k_proj": (h, kv), "self_attn.v_proj": (h, kv),
                               "self_attn.o_proj": (q, h), "mlp.gate_proj": (h, inter), "mlp.up_proj": (h, inter),
                               "mlp.down_proj": (inter, h)}.items():
            for k, v in gptq_tensors(fi, fo, g).items():
                t[f"{pre}{name}.{k}"] = v
        for name, n in (("input_layernorm", h), ("post_attention_layernorm", h), ("self_attn.q_norm", hd),
                        ("self_attn.k_norm", hd)):
            t[f"{pre}{name}.weight"] = (1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
    save_file(t, str(root / "model.safetensors"))
    (root / "config.json").write_text(json.dumps(cfg.to_dict()))
    return str(root)
