"""The decoder and fixed-batch runner around the quantized path (GPU).

* BF16 decoder: the decode step (paged KV cache, paged decode attention,
  rotary positions from the step's context) reproduces the last-position
  logits of a prefill over the same tokens (flash prefill attention), within
  bf16 rounding.
* W4A4 decoder: its first qkv projection inside a prefill forward (input
  RMSNorm fused into the activation quantization) is bit-exact with the
  oracle chain on the normalised embeddings.
* W4A16 decoder (GPTQ, the reference's use_w4a16 model): the N-fused q/k/v
  and gate/up projections give the same logits, bit for bit, as the separate
  projections.
* All: the decode step replayed from the captured HIP graph gives logits
  bit-equal to the eager step (the reference checks the same,
  benchmarks/bench_nano_latency.py:96-107), finite, and a short run of the
  benchmark loop completes with in-vocabulary tokens.
Two decoder layers at the Qwen3-8B widths, vocabulary 1024.
"""
import numpy as np
import pytest
import torch
from transformers import Qwen3Config

import oracle
from conftest import bf16_bits
from nv4.engine import Engine, run_decode_benchmark, seeded_prompts

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def cfg():
    return Qwen3Config(vocab_size=1024, hidden_size=4096, intermediate_size=12288, num_hidden_layers=2,
                       num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=4096,
                       rms_norm_eps=1e-6, rope_theta=1_000_000.0, tie_word_embeddings=False, attention_bias=False)


@pytest.fixture(scope="module")
def engines():
    c = cfg()
    bf16 = Engine(c, use_w4a4=False, max_num_seqs=4, max_model_len=1024, device=DEV, seed=1)
    w4 = Engine(c, use_w4a4=True, max_num_seqs=4, max_model_len=1024, device=DEV, seed=2, kv_cache=bf16.kv_cache)
    w16 = Engine(c, use_w4a4=False, use_w4a16=True, max_num_seqs=4, max_model_len=1024, device=DEV, seed=3,
                 kv_cache=bf16.kv_cache)
    return bf16, w4, w16


def test_decode_step_matches_prefill_bf16(engines):
    eng = engines[0]
    prompt = seeded_prompts(1, 301, 1024, seed=5)[0]
    temps = torch.full((1,), 1.0, device=DEV)
    with torch.inference_mode():
        # prefill 300 tokens, then decode token 301 at position 300 ...
        eng.prefill(0, prompt[:300], 1.0)
        dec = eng.decode([0], [prompt[300]], [301], temps, eager=True, return_logits=True).float()
        # ... against a prefill of all 301 tokens (slot 1)
        from nv4.utils.context import reset_context, set_context
        n = 301
        ids = torch.tensor(prompt, device=DEV)
        pos = torch.arange(n, device=DEV)
        cu = torch.tensor([0, n], dtype=torch.int32, device=DEV)
        slots = torch.tensor(eng._slots(1, 0, n), dtype=torch.int32, device=DEV)
        set_context(True, cu, cu, n, n, slots, None, None, seqlens_q=(n,))
        ref = eng.model.compute_logits(eng.model(ids, pos)).float()
        reset_context()
    torch.cuda.synchronize()
    err = (dec - ref).abs().max().item()
    scale = ref.abs().max().item()
    assert err <= 0.03 * scale, f"decode vs prefill logits: max err {err:.4f} of max {scale:.4f}"


def test_w4a4_first_projection_matches_oracle(engines):
    """Capture the first layer's qkv projection output inside a real prefill
    forward of the W4A4 decoder (input RMSNorm fused into the activation
    quantization) and check it against the oracle chain on the normalised
    embeddings (nv4 RMSNorm, whose bits the fused kernel reproduces)."""
    from nv4.kernels.decoder_ops import rmsnorm
    eng = engines[1]
    layer = eng.model.model.layers[0]
    assert layer.fused
    seen = {}
    h = layer.self_attn.register_forward_pre_hook(lambda m, a, kw: seen.update(qkv=kw["qkv"].clone()),
                                                  with_kwargs=True)
    ids = seeded_prompts(1, 70, 1024, seed=9)[0]
    try:
        eng.prefill(2, ids, 1.0)
    finally:
        h.remove()
    with torch.inference_mode():
        emb = eng.model.model.embed_tokens(torch.tensor(ids, device=DEV))
        y = rmsnorm(emb, layer.input_layernorm.weight, layer.input_layernorm.eps)
    torch.cuda.synchronize()
    m = layer.self_attn.qkv_proj
    assert m.weights_tiled  # the runner's projections read the MFMA-tiled layout
    sd = m.state_dict()  # reference [out, in/2] layout
    packed, scale = oracle.rht_quant_pack(bf16_bits(y), sd["signs"].cpu().numpy())
    ref = oracle.w4a4_gemm(packed, sd["packed_weight"].cpu().numpy(), scale, bf16_bits(sd["weight_scale"]))
    assert np.array_equal(bf16_bits(seen["qkv"]), ref)


@pytest.mark.parametrize("n", [48, 90])
def test_w4a16_fused_projections_equal_separate(engines, n):
    """Fused q/k/v and gate/up (N-concatenated GPTQ tensors) against the
    separate projections.  Up to 64 rows the W4A16 GEMM is this library's
    kernel, whose per-element arithmetic does not depend on N: bit-exact.
    Above, the product is a library GEMM on the dequantized weight, whose
    reduction order may change with N: relative RMS difference <= 1e-2."""
    eng = engines[2]
    ids = seeded_prompts(1, n, 1024, seed=21)[0]

    def logits():
        from nv4.utils.context import reset_context, set_context
        cu = torch.tensor([0, n], dtype=torch.int32, device=DEV)
        slots = torch.tensor(eng._slots(3, 0, n), dtype=torch.int32, device=DEV)
        with torch.inference_mode():
            set_context(True, cu, cu, n, n, slots, None, None, seqlens_q=(n,))
            out = eng.model.compute_logits(eng.model(torch.tensor(ids, device=DEV), torch.arange(n, device=DEV)))
            reset_context()
        return out.clone()

    layers = eng.model.model.layers
    assert all(l.self_attn.qkv_fused is not None and l.mlp.gate_up_fused is not None for l in layers)
    fused = logits()
    saved = [(l.self_attn.qkv_fused, l.mlp.gate_up_fused) for l in layers]
    try:
        for l in layers:
            object.__setattr__(l.self_attn, "qkv_fused", None)
            object.__setattr__(l.mlp, "gate_up_fused", None)
        separate = logits()
    finally:
        for l, (q, gu) in zip(layers, saved):
            object.__setattr__(l.self_attn, "qkv_fused", q)
            object.__setattr__(l.mlp, "gate_up_fused", gu)
    torch.cuda.synchronize()
    assert torch.isfinite(fused).all()
    if n <= 64:
        assert torch.equal(fused, separate)
    else:
        rel = ((fused.float() - separate.float()).norm() / separate.float().norm()).item()
        assert rel <= 1e-2, f"relative RMS difference {rel:.3e}"


@pytest.mark.parametrize("which", ["bf16", "w4a4", "w4a16"])
def test_graph_equals_eager_and_benchmark_loop(engines, which):
    eng = engines[("bf16", "w4a4", "w4a16").index(which)]
    prompts = seeded_prompts(4, 200, 1024, seed=11)
    res = run_decode_benchmark(eng, prompts, output_tokens=6, temperature=0.6)
    assert res["graph_equals_eager"] and res["logits_finite"]
    assert len(res["decode_ms"]) == 5 and len(res["prefill_ms"]) == 4
    assert all(0 <= t < 1024 for t in res["last_tokens"])
