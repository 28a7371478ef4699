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
# Quantization settings the kernels implement, as the manifest must state
# them (``is`` comparison for the booleans the format requires literally).
_CONTRACT = (
    ("group_size", lambda v: v == 128),
    ("static_groups", bool),
    ("runtime_column_permutation", lambda v: v is False),
    ("evaluation_activation_group_size", lambda v: v == 128),
    ("evaluation_activation_clipping", lambda v: v == 0.9),
    ("layout_version", lambda v: v == LAYOUT_VERSION),
)


def sha256(path, block: int = 1 << 24) -> str:
    """Hex SHA-256 of a file, read in ``block``-byte pieces into one buffer."""
    digest, buf = hashlib.sha256(), bytearray(block)
    view = memoryview(buf)
    with open(path, "rb", buffering=0) as f:
        while True:
            n = f.readinto(view)
            if not n:
                return digest.hexdigest()
            digest.update(view[:n])


class Manifest:
    """``manifest.json`` of a checkpoint directory, checked against the
    format on construction; the other checks run when their inputs are
    known (base directory, model depth, shard files)."""

    def __init__(self, checkpoint: Path):
        self.root = checkpoint
        self.data = json.loads((checkpoint / "manifest.json").read_text())
        if self.data.get("format") != FORMAT or not self.data.get("complete"):
            raise ValueError("Incomplete or unsupported W4A4 checkpoint")
        self.config = self.data.get("config", {})
        if not all(ok(self.config.get(key)) for key, ok in _CONTRACT):
            raise ValueError("Checkpoint quantization contract differs from the native kernel")

    def require_base(self, base: Path) -> None:
        if sha256(base / "config.json") != self.config.get("model_config_sha256"):
            raise ValueError("Base model config does not match the calibrated checkpoint")

    def require_depth(self, num_layers: int) -> None:
        if sorted(self.data.get("layers", {})) != sorted(map(str, range(num_layers))):
            raise ValueError("Checkpoint layer set does not match the model")

    def shard(self, index: int) -> Path:
        """The verified shard file of layer ``index``: inside the checkpoint
        directory and hashing to its manifest entry."""
        entry = self.data["layers"][str(index)]
        path = (self.root / entry["file"]).resolve()
        if not path.is_relative_to(self.root) or sha256(path) != entry["sha256"]:
            raise ValueError(f"Invalid checkpoint shard: layer {index}")
        return path


def _load_base_parameters(model, base: Path) -> None:
    """Copy the BF16 parameters of the quantized model (embeddings, norms,
    LM head) from the base directory; the base files' projection weights
    are never read (their names match no parameter).  The first shard that
    holds a name supplies it."""
    params = dict(model.named_parameters())
    found: set[str] = set()
    for path in sorted(base.glob("*.safetensors")):
        with safe_open(str(path), framework="pt", device="cpu") as f:
            for name in sorted((set(f.keys()) & params.keys()) - found):
                tensor, param = f.get_tensor(name), params[name]
                if (tensor.dtype, param.dtype) != (torch.bfloat16, torch.bfloat16):
                    raise ValueError(f"Expected BF16 base parameter: {name}")
                getattr(param, "weight_loader", default_weight_loader)(param, tensor)
                found.add(name)
    if found != params.keys():
        raise ValueError(f"Missing base parameters: {sorted(params.keys() - found)}")


def _checked_signs(tensor, module: W4A4Linear, where: str):
    ok = tensor.dtype == torch.int8 and tuple(tensor.shape) == (module.in_features,)
    if not ok or bool(((tensor != 1) & (tensor != -1)).any()):
        raise ValueError(f"Invalid RHT signs at layer {where}")
    return tensor


def _checked_weights(codes, scales, module: W4A4Linear, where: str):
    """Concatenate the source projections along N and check the result
    against the fused module's buffers."""
    codes, scales = torch.cat(codes), torch.cat(scales)
    shapes_ok = (codes.dtype == torch.int8 and codes.shape == module.packed_weight.shape
                 and scales.dtype == torch.bfloat16 and scales.shape == module.weight_scale.shape)
    if not shapes_ok or not bool((torch.isfinite(scales) & (scales > 0)).all()):
        raise ValueError(f"Invalid weight/scale at layer {where}")
    return codes, scales


def _load_layer(index: int, layer, shard: Path) -> int:
    """Fill the four fused W4A4 modules of one decoder layer from its shard;
    returns the number of source projections read."""
    read = 0
    with safe_open(str(shard), framework="pt", device="cpu") as f:
        for parent, target, sources, sign_key in GROUPS:
            module = getattr(getattr(layer, parent), target)
            where = f"{index}/{target}"
            if not isinstance(module, W4A4Linear):
                raise TypeError(f"Expected W4A4Linear at layer {where}")
            signs = _checked_signs(f.get_tensor(f"signs.{sign_key}"), module, where)
            codes, scales = _checked_weights([f.get_tensor(f"{parent}.{s}.packed") for s in sources],
                                             [f.get_tensor(f"{parent}.{s}.scale") for s in sources], module, where)
            module.assign_quantized_(codes, scales, signs)
            read += len(sources)
    return read


@torch.no_grad()
def load_w4a4_model(model, model_path, checkpoint_path) -> dict:
    """Load a calibrated W4A4 checkpoint into a ``Qwen3ForCausalLM`` built
    with ``use_w4a4``: the manifest is checked against the kernels'
    quantization contract and the base model's ``config.json``, the BF16
    parameters come from the base directory, and each layer's projections
    from its verified shard (already in the MFMA-tiled order on a GPU
    model).  Returns the quantization summary the runner reports."""
    base = Path(resolve_model_path(str(model_path)))
    manifest = Manifest(Path(checkpoint_path).resolve())
    manifest.require_base(base)
    layers = model.model.layers
    manifest.require_depth(len(layers))
    _load_base_parameters(model, base)
    projections = sum(_load_layer(i, layer, manifest.shard(i)) for i, layer in enumerate(layers))
    return {"format": FORMAT, "projections": projections, "native_linear_modules": 4 * len(layers),
            "checkpoint_manifest_sha256": sha256(manifest.root / "manifest.json"),
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
