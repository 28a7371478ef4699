"""BF16 safetensors loading into a decoder (nanovllm/utils/loader.py:8-34).

``load_model`` walks every ``*.safetensors`` of a local model directory
and copies each tensor into the parameter of the same name, through the
parameter's ``weight_loader`` when it has one; q/k/v and gate/up tensors are
routed to the fused parameter with their shard id by
``model.packed_modules_mapping``, as in the reference.
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


def load_model(model: nn.Module, path: str):
    path = resolve_model_path(path)
    packed_modules_mapping = getattr(model, "packed_modules_mapping", {})
    for file in sorted(glob(os.path.join(path, "*.safetensors"))):
        with safe_open(file, "pt", "cpu") as f:
            for weight_name in f.keys():
                if weight_name.endswith(".g_idx"):
                    continue
                for k, (v, shard_id) in packed_modules_mapping.items():
                    if k in weight_name:
                        param = model.get_parameter(weight_name.replace(k, v))
                        param.weight_loader(param, f.get_tensor(weight_name), shard_id)
                        break
                else:
                    param = model.get_parameter(weight_name)
                    getattr(param, "weight_loader", default_weight_loader)(param, f.get_tensor(weight_name))
