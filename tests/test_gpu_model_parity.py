"""Whole-model parity of the W4A4 decoder with the oracle (GPU).

Restates the reference's end-to-end check (benchmarks/verify_nano_w4a4.py):

* ``W4A4Linear.forward`` replaced by a forward computed by the oracle on the
  linear's bf16 input (K1 then the grouped-FMA GEMM, :55-68); prefill and
  decode logits of the native model must equal that model's bit for bit
  (:135-142).  Here the native layers run the fused producer + K1 kernels
  (add+RMSNorm before qkv and gate_up, SiLU-mul before down), and the
  oracle model runs the separate producers and hands their bf16 output to
  the oracle forward, so the check also covers the fusion.
* Graph replay against eager decode at batch 32, 7 and 1 (:113-124), full
  logits bit for bit.
* A synthetic two-layer checkpoint in the reference's on-disk format loaded
  onto the GPU (loader, concatenation along N and tiling): every projection
  of a prefill and a decode step equals the oracle on the checkpoint's own
  tensors, and every fused K1 equals the oracle K1 (``model_probe``).

Two decoder layers at the Qwen3-8B widths (hidden 4096, intermediate 12288,
32 q / 8 kv heads), vocabulary 1024; 32 ragged prompts of 3..9 tokens
(prefill M = 189, the int8 prefill GEMM), then a bs32 decode step (the
decode GEMMs).
"""
import numpy as np
import pytest
import torch
from transformers import Qwen3Config

import oracle
from conftest import bf16_bits, bits_to_bf16
from model_probe import ProjectionProbe, check_gemms, check_k1s, check_linears
from nv4.engine import Engine, seeded_prompts
from nv4.layers.linear_w4a4 import W4A4Linear
from nv4.utils.context import reset_context, set_context

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
VOCAB = 1024


def cfg(layers=2):
    return Qwen3Config(vocab_size=VOCAB, hidden_size=4096, intermediate_size=12288, num_hidden_layers=layers,
                       num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=4096,
                       rms_norm_eps=1e-6, rope_theta=1_000_000.0, tie_word_embeddings=False, attention_bias=False)


def prompts():
    toks = seeded_prompts(32, 9, VOCAB, seed=31)
    return [t[:3 + (i * 5) % 7] for i, t in enumerate(toks)]


def batched_prefill(eng, seqs):
    """One packed prefill forward of all sequences (sequence i in slot i);
    returns the last-position logits [B, vocab]."""
    lens = [len(s) for s in seqs]
    ids = torch.tensor([t for s in seqs for t in s], device=DEV)
    pos = torch.tensor([p for n in lens for p in range(n)], device=DEV)
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32, device=DEV)
    slots = torch.tensor([x for i, n in enumerate(lens) for x in eng._slots(i, 0, n)], dtype=torch.int32,
                         device=DEV)
    with torch.inference_mode():
        set_context(True, cu, cu, max(lens), max(lens), slots, None, None, seqlens_q=lens)
        logits = eng.model.compute_logits(eng.model(ids, pos)).clone()
        reset_context()
    return logits


class OracleForward:
    """W4A4Linear.forward computed by the oracle on the layer's bf16 input
    (RHT + quantize + pack, then the grouped GEMM; the reference's
    reference_forward, verify_nano_w4a4.py:55-68), with the model's layers
    switched to the unfused producers so that each linear sees its input."""

    def __init__(self, model):
        self.model = model
        self.weights = {}

    def forward(self, module, x):
        if id(module) not in self.weights:
            sd = module.state_dict()
            self.weights[id(module)] = (sd["signs"].cpu().numpy(), sd["packed_weight"].cpu().numpy(),
                                        bf16_bits(sd["weight_scale"]))
        signs, wp, sw = self.weights[id(module)]
        flat = bf16_bits(x.reshape(-1, module.in_features))
        packed, scale = oracle.rht_quant_pack(flat, signs)
        out = oracle.w4a4_gemm(packed, wp, scale, sw)
        return bits_to_bf16(out).to(x.device).reshape(*x.shape[:-1], module.out_features)

    def __enter__(self):
        self._native = W4A4Linear.forward
        runner = self
        W4A4Linear.forward = lambda module, x: runner.forward(module, x)
        self._fused = [layer.fused for layer in self.model.model.layers]
        for layer in self.model.model.layers:
            layer.fused = False
        return self

    def __exit__(self, *exc):
        W4A4Linear.forward = self._native
        for layer, f in zip(self.model.model.layers, self._fused):
            layer.fused = f
        return False


@pytest.fixture(scope="module")
def engine():
    eng = Engine(cfg(), use_w4a4=True, max_num_seqs=32, max_model_len=512, device=DEV, seed=41)
    for bs in (32, 7, 1):  # capture before any prefill (the capture's warm-up writes slot 0)
        eng.capture(bs)
    return eng


def forward_pair(eng):
    """Prefill logits, then the eager decode logits of the first step with
    the prefill's argmax tokens (teacher forcing, as the reference does)."""
    seqs = prompts()
    pre = batched_prefill(eng, seqs)
    teacher = pre.argmax(-1).tolist()
    lens = [len(s) + 1 for s in seqs]
    temps = torch.ones(32, device=DEV)
    dec = eng.decode(list(range(32)), teacher, lens, temps, eager=True, return_logits=True).clone()
    return pre, dec, teacher, lens


def test_whole_model_logits_equal_oracle_forward(engine):
    assert all(layer.fused for layer in engine.model.model.layers)
    native_pre, native_dec, teacher, lens = forward_pair(engine)
    with OracleForward(engine.model):
        ref_pre, ref_dec, ref_teacher, _ = forward_pair(engine)
    torch.cuda.synchronize()
    assert torch.isfinite(native_pre).all() and torch.isfinite(native_dec).all()
    assert torch.equal(native_pre, ref_pre), "prefill logits differ from the oracle-forward model"
    assert teacher == ref_teacher
    assert torch.equal(native_dec, ref_dec), "decode logits differ from the oracle-forward model"


@pytest.mark.parametrize("bs", [32, 7, 1])
def test_graph_equals_eager_decode(engine, bs):
    seqs = prompts()
    pre = batched_prefill(engine, seqs)
    teacher = pre.argmax(-1).tolist()
    lens = [len(s) + 1 for s in seqs]
    temps = torch.ones(bs, device=DEV)
    slots = list(range(bs))
    graph = engine.decode(slots, teacher[:bs], lens[:bs], temps, return_logits=True).clone()
    eager = engine.decode(slots, teacher[:bs], lens[:bs], temps, eager=True, return_logits=True).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(graph).all()
    assert torch.equal(graph, eager), f"bs={bs}: graph replay differs from the eager step"


def test_loaded_checkpoint_on_gpu_matches_oracle(tmp_path):
    """Synthetic checkpoint -> load_w4a4_model onto cuda:0 (tiling included)
    -> prefill and decode: every projection equals the oracle on the
    checkpoint file's tensors, every fused K1 the oracle K1."""
    from safetensors import safe_open

    from nv4.qwen3 import Qwen3ForCausalLM
    from nv4.utils import loader_w4a4 as L

    c = cfg()
    base = L.synthetic_base_model(tmp_path / "base", c, seed=7)
    L.synthetic_w4a4_checkpoint(tmp_path / "ckpt", base, c, seed=9)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(DEV):
            model = Qwen3ForCausalLM(c, use_w4a4=True)
    finally:
        torch.set_default_dtype(prev)
    info = L.load_w4a4_model(model, str(base), str(tmp_path / "ckpt"))
    assert info["projections"] == 14 and info["native_linear_modules"] == 8
    assert all(m.weights_tiled for m in model.modules() if isinstance(m, W4A4Linear))
    # The loaded layers keep no fp6 copy of their weights by default; on request they keep it
    # where it pays (qkv, o, down of Qwen3-8B), matching the weights just loaded.
    from nv4.kernels.w4a4_grouped import keep_weights_f6, weights_to_f6
    for m in model.modules():
        if isinstance(m, W4A4Linear):
            assert m.weight_f6 is None and m._f6() is None
            m.keep_weights_f6_(True)
            keep = keep_weights_f6(m.out_features, m.in_features)
            assert (m._f6() is not None) == keep
            if keep:
                assert torch.equal(m.weight_f6, weights_to_f6(m.packed_weight, True))

    # Weights straight from the files, concatenated along N as the reference's loader does.
    weights = {}
    for i in range(2):
        with safe_open(str(tmp_path / "ckpt" / "weights" / f"layer_{i:02d}.safetensors"), "pt") as f:
            for name, parent, sources in (("qkv", "self_attn", ("q_proj", "k_proj", "v_proj")),
                                          ("o", "self_attn", ("o_proj",)),
                                          ("gate_up", "mlp", ("gate_proj", "up_proj")),
                                          ("down", "mlp", ("down_proj",))):
                wp = torch.cat([f.get_tensor(f"{parent}.{s}.packed") for s in sources]).numpy()
                sw = bf16_bits(torch.cat([f.get_tensor(f"{parent}.{s}.scale") for s in sources]))
                weights[f"layer{i}.{name}"] = (wp, sw)

    eng = Engine(c, use_w4a4=True, max_num_seqs=32, max_model_len=64, device=DEV, model=model)
    with ProjectionProbe(model, [0, 1]) as probe:
        forward_pair(eng)
    torch.cuda.synchronize()
    # per layer and pass: qkv, gate_up and down from fused K1s, o as a whole
    # forward; 2 layers x (prefill + decode)
    assert check_gemms(probe, weights=weights) == 12
    assert check_linears(probe, weights=weights) == 4
    assert check_k1s(probe) == 12
