"""The W4A4 checkpoint format and loader (CPU).

Restates the reference's loader contract (nanovllm/utils/loader_w4a4.py:32-96)
on a synthetic checkpoint written in the reference's on-disk format
(benchmarks/calibrate_rht_gptq_grouped.py:63-87,131-136,189-237): the fused
modules receive q|k|v and gate|up concatenated along N, o and down as they
are, the signs and the BF16 base parameters; each violation of the contract
raises the reference's exception.  One decoder layer at the real
projection widths (hidden 4096, intermediate 12288) and a small vocabulary.
"""
import json
import shutil

import pytest
import torch
from safetensors import safe_open
from transformers import Qwen3Config

from nv4.qwen3 import Qwen3ForCausalLM
from nv4.utils import loader_w4a4 as L


def tiny_config(layers=1):
    return Qwen3Config(vocab_size=256, hidden_size=4096, intermediate_size=12288, num_hidden_layers=layers,
                       num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=512,
                       tie_word_embeddings=False, attention_bias=False)


def build(cfg):
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        return Qwen3ForCausalLM(cfg, use_w4a4=True)
    finally:
        torch.set_default_dtype(prev)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = tmp_path_factory.mktemp("w4a4")
    cfg = tiny_config()
    base = L.synthetic_base_model(root / "base", cfg, seed=3)
    manifest = L.synthetic_w4a4_checkpoint(root / "ckpt", base, cfg, seed=5)
    return cfg, root / "base", root / "ckpt", manifest


def test_format_and_manifest(ckpt):
    cfg, base, ck, manifest = ckpt
    assert manifest["format"] == L.FORMAT and manifest["complete"] and manifest["projections"] == 7
    assert manifest["config"]["layout_version"] == "row_DH_paley12_kron_sylvester_v1"
    with safe_open(str(ck / "weights" / "layer_00.safetensors"), "pt") as f:
        assert f.metadata() == {"format": L.FORMAT, "layer": "0"}
        keys = set(f.keys())
        assert keys == {"signs.qkv", "signs.o", "signs.gate_up", "signs.down",
                        *(f"self_attn.{n}.{t}" for n in ("q_proj", "k_proj", "v_proj", "o_proj")
                          for t in ("packed", "scale")),
                        *(f"mlp.{n}.{t}" for n in ("gate_proj", "up_proj", "down_proj") for t in ("packed", "scale"))}
        assert f.get_tensor("self_attn.k_proj.packed").shape == (1024, 2048)
        assert f.get_tensor("mlp.down_proj.scale").shape == (4096, 96)
    # signs seeded as the reference's calibration seeds them: seed + 17 * layer + group index
    from nv4.workloads import signs
    with safe_open(str(ck / "weights" / "layer_00.safetensors"), "pt") as f:
        assert torch.equal(f.get_tensor("signs.gate_up"), signs(4096, 5 + 2))
        assert torch.equal(f.get_tensor("signs.down"), signs(12288, 5 + 3))


def test_load_concatenates_along_n(ckpt):
    cfg, base, ck, _ = ckpt
    model = build(cfg)
    info = L.load_w4a4_model(model, str(base), str(ck))
    assert info["projections"] == 7 and info["native_linear_modules"] == 4 and info["split_k"] is False
    layer = model.model.layers[0]
    with safe_open(str(ck / "weights" / "layer_00.safetensors"), "pt") as f:
        g = f.get_tensor
        qkv = layer.self_attn.qkv_proj
        assert torch.equal(qkv.packed_weight, torch.cat([g("self_attn.q_proj.packed"), g("self_attn.k_proj.packed"),
                                                         g("self_attn.v_proj.packed")]))
        assert torch.equal(qkv.weight_scale, torch.cat([g("self_attn.q_proj.scale"), g("self_attn.k_proj.scale"),
                                                        g("self_attn.v_proj.scale")]))
        assert torch.equal(qkv.signs, g("signs.qkv"))
        gu = layer.mlp.gate_up_proj
        assert torch.equal(gu.packed_weight, torch.cat([g("mlp.gate_proj.packed"), g("mlp.up_proj.packed")]))
        assert torch.equal(layer.mlp.down_proj.weight_scale, g("mlp.down_proj.scale"))
        assert torch.equal(layer.self_attn.o_proj.signs, g("signs.o"))
    with safe_open(str(base / "model.safetensors"), "pt") as f:
        assert torch.equal(model.lm_head.weight, f.get_tensor("lm_head.weight"))
        assert torch.equal(model.model.embed_tokens.weight, f.get_tensor("model.embed_tokens.weight"))


def tampered(ckpt, tmp_path, edit):
    cfg, base, ck, _ = ckpt
    dst = tmp_path / "ck"
    shutil.copytree(ck, dst)
    edit(dst)
    return cfg, base, dst


def edit_manifest(**changes):
    def apply(dst):
        m = json.loads((dst / "manifest.json").read_text())
        for k, v in changes.items():
            if k.startswith("config."):
                m["config"][k[7:]] = v
            else:
                m[k] = v
        (dst / "manifest.json").write_text(json.dumps(m))
    return apply


@pytest.mark.parametrize("edit,message", [
    (edit_manifest(format="other"), "Incomplete or unsupported"),
    (edit_manifest(complete=False), "Incomplete or unsupported"),
    (edit_manifest(**{"config.evaluation_activation_clipping": 1.0}), "quantization contract"),
    (edit_manifest(**{"config.layout_version": "block128"}), "quantization contract"),
    (edit_manifest(**{"config.runtime_column_permutation": True}), "quantization contract"),
    (edit_manifest(**{"config.model_config_sha256": "0" * 64}), "Base model config"),
    (edit_manifest(layers={}), "layer set"),
])
def test_manifest_contract(ckpt, tmp_path, edit, message):
    cfg, base, dst = tampered(ckpt, tmp_path, edit)
    with pytest.raises(ValueError, match=message):
        L.load_w4a4_model(build(cfg), str(base), str(dst))


def test_shard_hash_and_tensor_checks(ckpt, tmp_path):
    cfg, base, dst = tampered(ckpt, tmp_path, lambda d: None)
    shard = dst / "weights" / "layer_00.safetensors"
    data = bytearray(shard.read_bytes())
    data[-1] ^= 1
    shard.write_bytes(bytes(data))
    with pytest.raises(ValueError, match="Invalid checkpoint shard"):
        L.load_w4a4_model(build(cfg), str(base), str(dst))
    # Rewrite the layer with a zero sign / a non-positive scale (hashes updated): rejected.
    layer = L.synthetic_layer(cfg, 0, 5)
    for key, bad in (("signs.o", "signs"), ("self_attn.q_proj.scale", "scale")):
        t = dict(layer)
        if bad == "signs":
            t[key] = t[key].clone()
            t[key][3] = 0
        else:
            t[key] = t[key].clone()
            t[key][0, 0] = 0
        L.save_w4a4_checkpoint(dst, [t], base / "config.json", seed=5)
        with pytest.raises(ValueError, match="Invalid RHT signs" if bad == "signs" else "Invalid weight/scale"):
            L.load_w4a4_model(build(cfg), str(base), str(dst))


def test_missing_base_parameters(ckpt, tmp_path):
    cfg, base, ck, _ = ckpt
    nb = tmp_path / "base"
    shutil.copytree(base, nb)
    from safetensors.torch import load_file, save_file
    t = load_file(str(nb / "model.safetensors"))
    del t["model.norm.weight"]
    save_file(t, str(nb / "model.safetensors"))
    with pytest.raises(ValueError, match="Missing base parameters"):
        L.load_w4a4_model(build(cfg), str(nb), str(ck))


def test_non_w4a4_projection_is_rejected(ckpt):
    """A BF16 model fails on its projection weights, absent from the base
    files (ValueError, as in the reference); a projection slot holding some
    other module type raises TypeError."""
    cfg, base, ck, _ = ckpt
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        bf16 = Qwen3ForCausalLM(cfg, use_w4a4=False)
    finally:
        torch.set_default_dtype(prev)
    with pytest.raises(ValueError, match="Missing base parameters"):
        L.load_w4a4_model(bf16, str(base), str(ck))
    model = build(cfg)
    model.model.layers[0].mlp.down_proj = torch.nn.Identity()
    with pytest.raises(TypeError, match="Expected W4A4Linear"):
        L.load_w4a4_model(model, str(base), str(ck))
