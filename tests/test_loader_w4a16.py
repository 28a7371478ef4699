"""The W4A16 model path on the CPU: GPTQ checkpoint loading and fusion.

The reference's W4A16 model (nanovllm/models/qwen3_w4a16.py:14-252) keeps
separate q/k/v/o/gate/up/down GPTQ projections and loads every checkpoint
tensor by name (nanovllm/utils/loader.py:12-34, ``g_idx`` skipped).  Here:
every parameter holds exactly the checkpoint tensor; ``fuse_projections_``
concatenates q/k/v and gate/up along N (qweight, qzeros, scales on dim 1)
with the parts left as views of the fused tensors (no copy), and the state
dict still equals the checkpoint.
"""
import torch
from safetensors.torch import load_file
from transformers import Qwen3Config

from nv4.qwen3 import W4A16Qwen3ForCausalLM
from nv4.utils.loader import load_w4a16_model, write_gptq_checkpoint


def small_cfg():
    return Qwen3Config(vocab_size=96, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=64,
                       rms_norm_eps=1e-6, tie_word_embeddings=False, attention_bias=False)


def test_gptq_checkpoint_loads_by_name_and_fuses(tmp_path):
    cfg = small_cfg()
    root = write_gptq_checkpoint(tmp_path / "gptq", cfg, seed=4)
    ref = load_file(str(tmp_path / "gptq" / "model.safetensors"))
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        model = W4A16Qwen3ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    load_w4a16_model(model, root)
    sd = model.state_dict()
    assert set(sd) == {k for k in ref if not k.endswith(".g_idx")}
    for k, v in sd.items():
        assert v.dtype == ref[k].dtype and torch.equal(v, ref[k]), k
    for layer in model.model.layers:
        a, m = layer.self_attn, layer.mlp
        for fused, parts in ((a.qkv_fused, (a.q_proj, a.k_proj, a.v_proj)), (m.gate_up_fused, (m.gate_proj, m.up_proj))):
            assert fused is not None and fused.out_features == sum(p.out_features for p in parts)
            for name in ("qweight", "qzeros", "scales"):
                cat = torch.cat([getattr(p, name).data for p in parts], dim=1)
                assert torch.equal(getattr(fused, name).data, cat)
                base = getattr(fused, name).data.untyped_storage().data_ptr()
                assert all(getattr(p, name).data.untyped_storage().data_ptr() == base for p in parts)
    assert a.qkv_fused.qweight.shape == (256 // 8, 256 + 2 * 128)
    assert not any("fused" in k for k in sd)
