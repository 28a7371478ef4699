"""The calibrated RHT/G128 W4A4 checkpoint: loading, and writing one.

``load_w4a4_model`` keeps the reference's contract
(nanovllm/utils/loader_w4a4.py:14-96): the manifest must name the format
``rht_gptq_static_group128_bf16_scale_i4_v1``, be complete, and carry the
quantization settings the kernels implement (group 128, static groups, no
run-time column permutation, activation group 128 with clipping 0.9, layout
``row_DH_paley12_kron_sylvester_v1``); the base model's ``config.json`` must
hash to the manifest's ``model_config_sha256``; every layer shard must hash
to its manifest entry and lie inside the checkpoint directory.  The BF16
embeddings, norms and LM head come from the base directory's safetensors
(parameters only: the quantized projections are buffers); each layer's
q/k/v and gate/up tensors are concatenated along N into the fused
``W4A4Linear`` modules, o and down copied as they are.  Every check raises
the reference's ValueError/TypeError.

``save_w4a4_checkpoint`` writes the same on-disk format
(benchmarks/calibrate_rht_gptq_grouped.py:63-87,131-136,189-204,231-237:
``manifest.json`` plus ``weights/layer_{i:02d}.safetensors`` with
``signs.{qkv,o,gate_up,down}``, ``{self_attn|mlp}.<proj>.packed`` and
``.scale`` and the ``format``/``layer`` metadata) from per-layer tensors;
``synthetic_w4a4_checkpoint`` fills it with seeded random codes and scales
(the random-init end-to-end workload), and ``synthetic_base_model`` writes a
matching BF16 base directory (``config.json`` and the non-projection
parameters).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from ..layers.linear_w4a4 import W4A4Linear
from .loader import default_weight_loader, resolve_model_path

FORMAT = "rht_gptq_static_group128_bf16_scale_i4_v1"
LAYOUT_VERSION = "row_DH_paley12_kron_sylvester_v1"
# (parent module, fused module, source projections in concatenation order, signs key)
GROUPS = (
    ("self_attn", "qkv_proj", ("q_proj", "k_proj", "v_proj"), "qkv"),
    ("self_attn", "o_proj", ("o_proj",), "o"),
    ("mlp", "gate_up_proj", ("gate_proj", "up_proj"), "gate_up"),
    ("mlp", "down_proj", ("down_proj",), "down"),
)


def sha256(path) -> str:
    digest = hashlib.sha256()
    with Path(path).open("rb") as handle:
        for chunk in iter(lambda: handle.read(8 * 1024**2), b""):
            digest.update(chunk)
    return digest.hexdigest()


def _check_contract(manifest: dict) -> dict:
    cfg = manifest.get("config", {})
    if manifest.get("format") != FORMAT or not manifest.get("complete"):
        raise ValueError("Incomplete or unsupported W4A4 checkpoint")
    if (cfg.get("group_size") != 128 or not cfg.get("static_groups")
            or cfg.get("runtime_column_permutation") is not False
            or cfg.get("evaluation_activation_group_size") != 128
            or cfg.get("evaluation_activation_clipping") != 0.9
            or cfg.get("layout_version") != LAYOUT_VERSION):
        raise ValueError("Checkpoint quantization contract differs from the native kernel")
    return cfg


@torch.no_grad()
def load_w4a4_model(model, model_path, checkpoint_path):
    base = Path(resolve_model_path(str(model_path)))
    checkpoint = Path(checkpoint_path).resolve()
    manifest = json.loads((checkpoint / "manifest.json").read_text())
    cfg = _check_contract(manifest)
    if sha256(base / "config.json") != cfg.get("model_config_sha256"):
        raise ValueError("Base model config does not match the calibrated checkpoint")
    layers = model.model.layers
    if set(manifest.get("layers", {})) != {str(i) for i in range(len(layers))}:
        raise ValueError("Checkpoint layer set does not match the model")

    # Only embeddings, head and norms are parameters of the quantized model;
    # the base files' projection weights are skipped unread.
    remaining = dict(model.named_parameters())
    for shard in sorted(base.glob("*.safetensors")):
        with safe_open(str(shard), framework="pt", device="cpu") as handle:
            for name in handle.keys():
                if name in remaining:
                    param = remaining.pop(name)
                    value = handle.get_tensor(name)
                    if value.dtype != torch.bfloat16 or param.dtype != torch.bfloat16:
                        raise ValueError(f"Expected BF16 base parameter: {name}")
                    getattr(param, "weight_loader", default_weight_loader)(param, value)
    if remaining:
        raise ValueError(f"Missing base parameters: {sorted(remaining)}")

    count = 0
    for index, layer in enumerate(layers):
        entry = manifest["layers"][str(index)]
        shard = (checkpoint / entry["file"]).resolve()
        if not shard.is_relative_to(checkpoint) or sha256(shard) != entry["sha256"]:
            raise ValueError(f"Invalid checkpoint shard: layer {index}")
        with safe_open(str(shard), framework="pt", device="cpu") as handle:
            for parent, target, sources, sign_name in GROUPS:
                module = getattr(getattr(layer, parent), target)
                if not isinstance(module, W4A4Linear):
                    raise TypeError(f"Expected W4A4Linear at layer {index}/{target}")
                signs = handle.get_tensor(f"signs.{sign_name}")
                if (signs.dtype != torch.int8 or signs.shape != module.signs.shape
                        or not torch.all((signs == 1) | (signs == -1))):
                    raise ValueError(f"Invalid RHT signs at layer {index}/{target}")
                packed = torch.cat([handle.get_tensor(f"{parent}.{name}.packed") for name in sources])
                scale = torch.cat([handle.get_tensor(f"{parent}.{name}.scale") for name in sources])
                if (packed.dtype != torch.int8 or packed.shape != module.packed_weight.shape
                        or scale.dtype != torch.bfloat16 or scale.shape != module.weight_scale.shape
                        or not torch.isfinite(scale).all() or not torch.all(scale > 0)):
                    raise ValueError(f"Invalid weight/scale at layer {index}/{target}")
                module.packed_weight.copy_(packed)
                module.weight_scale.copy_(scale)
                module.signs.copy_(signs)
                module.weights_tiled = False  # the buffer now holds the reference layout
                count += len(sources)
    for module in model.modules():  # decode-kernel weight order (GPU modules; bit-identical results)
        if isinstance(module, W4A4Linear):
            module.tile_weights_()
    return {"format": FORMAT, "projections": count, "native_linear_modules": len(layers) * 4,
            "checkpoint_manifest_sha256": sha256(checkpoint / "manifest.json"),
            "weight_group_size": 128, "activation_group_size": 128, "activation_clipping": 0.9,
            "scale_dtype": "bfloat16", "split_k": False}


def _write_json(path: Path, value) -> None:
    temporary = path.with_suffix(path.suffix + ".tmp")
    temporary.write_text(json.dumps(value, indent=2) + "\n")
    temporary.replace(path)


def save_w4a4_checkpoint(checkpoint_dir, layers, model_config_path, seed: int = 0) -> dict:
    """Write a complete checkpoint.  ``layers[i]`` maps shard tensor names
    (``signs.qkv``, ``self_attn.q_proj.packed``, ``self_attn.q_proj.scale``,
    ...) to tensors.  Returns the manifest."""
    root = Path(checkpoint_dir)
    (root / "weights").mkdir(parents=True, exist_ok=True)
    config = {"group_size": 128, "static_groups": True, "runtime_column_permutation": False,
              "evaluation_activation_group_size": 128, "evaluation_activation_clipping": 0.9,
              "layout_version": LAYOUT_VERSION, "model_config_sha256": sha256(model_config_path),
              "seed": seed, "code_range": [-8, 7], "weight_scales": "synthetic"}
    manifest = {"format": FORMAT, "complete": False, "config": config, "layers": {}}
    for index, tensors in enumerate(layers):
        path = root / "weights" / f"layer_{index:02d}.safetensors"
        temporary = path.with_suffix(".tmp")
        save_file({k: v.contiguous() for k, v in tensors.items()}, str(temporary),
                  metadata={"format": FORMAT, "layer": str(index)})
        temporary.replace(path)
        manifest["layers"][str(index)] = {"file": str(path.relative_to(root)), "bytes": path.stat().st_size,
                                          "sha256": sha256(path)}
    manifest["complete"] = True
    manifest["projections"] = 7 * len(layers)
    _write_json(root / "manifest.json", manifest)
    return manifest


def _projection_shapes(hf_config) -> dict:
    """(parent, projection) -> (N, K) of the unfused projections."""
    head_dim = getattr(hf_config, "head_dim", None) or hf_config.hidden_size // hf_config.num_attention_heads
    h, i = hf_config.hidden_size, hf_config.intermediate_size
    q, kv = hf_config.num_attention_heads * head_dim, hf_config.num_key_value_heads * head_dim
    return {("self_attn", "q_proj"): (q, h), ("self_attn", "k_proj"): (kv, h), ("self_attn", "v_proj"): (kv, h),
            ("self_attn", "o_proj"): (h, q), ("mlp", "gate_proj"): (i, h), ("mlp", "up_proj"): (i, h),
            ("mlp", "down_proj"): (h, i)}


def synthetic_layer(hf_config, layer_index: int, seed: int, generator: torch.Generator | None = None) -> dict:
    """Seeded random shard tensors of one layer: codes uniform in [-8, 7]
    packed two per byte (even k in the low nibble), group-128 BF16 scales
    uniform in [0.005, 0.02], and RHT signs seeded as the reference's
    calibration seeds them (seed + 17 * layer + group index, in the group
    order qkv, o, gate_up, down)."""
    from ..workloads import pack_int4, signs as make_signs
    gen = generator or torch.Generator("cpu").manual_seed(seed * 1000003 + layer_index)
    shapes = _projection_shapes(hf_config)
    out = {}
    for group_index, (parent, _, sources, sign_name) in enumerate(GROUPS):
        K = shapes[(parent, sources[0])][1]
        out[f"signs.{sign_name}"] = make_signs(K, seed + 17 * layer_index + group_index)
        for name in sources:
            N, K = shapes[(parent, name)]
            codes = torch.randint(-8, 8, (N, K), generator=gen, dtype=torch.int8)
            out[f"{parent}.{name}.packed"] = pack_int4(codes)
            out[f"{parent}.{name}.scale"] = (0.005 + 0.015 * torch.rand(N, K // 128, generator=gen)).to(torch.bfloat16)
    return out


def synthetic_base_model(base_dir, hf_config, seed: int = 0) -> Path:
    """A BF16 base directory for a random-init model: ``config.json`` and
    the parameters the W4A4 model keeps (embeddings and LM head ~N(0, 0.02),
    norms 1)."""
    root = Path(base_dir)
    root.mkdir(parents=True, exist_ok=True)
    hf_config.to_json_file(str(root / "config.json"))
    gen = torch.Generator("cpu").manual_seed(seed)
    head_dim = getattr(hf_config, "head_dim", None) or hf_config.hidden_size // hf_config.num_attention_heads
    tensors = {"model.embed_tokens.weight":
               (torch.randn(hf_config.vocab_size, hf_config.hidden_size, generator=gen) * 0.02).to(torch.bfloat16),
               "model.norm.weight": torch.ones(hf_config.hidden_size, dtype=torch.bfloat16)}
    if not hf_config.tie_word_embeddings:
        tensors["lm_head.weight"] = (torch.randn(hf_config.vocab_size, hf_config.hidden_size, generator=gen)
                                     * 0.02).to(torch.bfloat16)
    for i in range(hf_config.num_hidden_layers):
        p = f"model.layers.{i}."
        tensors[p + "input_layernorm.weight"] = torch.ones(hf_config.hidden_size, dtype=torch.bfloat16)
        tensors[p + "post_attention_layernorm.weight"] = torch.ones(hf_config.hidden_size, dtype=torch.bfloat16)
        tensors[p + "self_attn.q_norm.weight"] = torch.ones(head_dim, dtype=torch.bfloat16)
        tensors[p + "self_attn.k_norm.weight"] = torch.ones(head_dim, dtype=torch.bfloat16)
    save_file(tensors, str(root / "model.safetensors"))
    return root


def synthetic_w4a4_checkpoint(checkpoint_dir, base_dir, hf_config, seed: int = 0) -> dict:
    """A complete random-init checkpoint for ``hf_config`` whose manifest is
    tied to ``base_dir/config.json``."""
    layers = [synthetic_layer(hf_config, i, seed) for i in range(hf_config.num_hidden_layers)]
    return save_w4a4_checkpoint(checkpoint_dir, layers, Path(base_dir) / "config.json", seed)
