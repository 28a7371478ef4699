"""Records the quantized-linear calls of chosen decoder layers during a real
forward, and checks each one against the oracle (test helper, GPU).

In the W4A4 decoder every projection's activations are quantized by a fused
producer + K1 launch (add+RMSNorm before qkv and gate_up, SiLU-mul before
down) and multiplied by the grouped INT4 GEMM on the MFMA-tiled weights
(``W4A4Linear.forward_quantized``).  At decode sizes SiLU-mul may run in the
gate/up GEMM's epilogue instead (``forward_quantized_silu``), followed by
down's plain row-tiled K1 (``rht_quant_pack_rowtiled``).  ``ProjectionProbe`` wraps both for the
layers it is given and keeps copies of what went in and came out; the
``check_*`` functions then compare:

* every GEMM output with the oracle's grouped GEMM on the recorded codes and
  scales and the weights in the reference layout (bit for bit); a gate/up
  GEMM with SiLU-mul in its epilogue with the separate SiLU-mul kernel on the
  oracle's GEMM output;
* every whole ``W4A4Linear.forward`` (o_proj, whose input is the attention
  output in bf16) with the oracle's K1 + GEMM chain on the same input;
* every fused K1 output with the oracle's K1 on the producer's bf16 output
  computed by this library's separate producer kernel (bit for bit; the
  separate kernel equals the fused prologue bit for bit and matches the
  reference's fp32 formulation within one bf16 ulp, both tested elsewhere),
  and the residual written back with bf16(x + residual).

``rows`` restricts the oracle to a subset of rows (prefill-sized M).
"""
from __future__ import annotations

import numpy as np
import torch

import oracle
from conftest import bf16_bits

import nv4.qwen3 as qwen3
from nv4.kernels.decoder_ops import rmsnorm, silu_mul
from nv4.layers.linear_w4a4 import W4A4Linear


def rowtiled_to_reference(packed, m):
    """Row-tiled packed codes [ceil(M/16)*16, K/2] -> the [M, K/2] layout (torch,
    same device): unit (rb*G + g)*64 + 16*part + r of the row-tiled buffer holds
    bytes 64*g + 16*part .. +15 of row 16*rb + r."""
    rows, kb = packed.shape
    g = kb // 64
    t = packed.reshape(rows // 16, g, 4, 16, 16).permute(0, 3, 1, 2, 4).reshape(rows, kb)
    return t[:m].contiguous()


class ProjectionProbe:
    def __init__(self, model, layer_ids):
        self.model = model
        self.layers = {i: model.model.layers[i] for i in layer_ids}
        self.gemms = []   # (name, module, packed, scale, out): forward_quantized calls
        self.linears = []  # (name, module, x, out): whole-forward calls (o_proj takes bf16 input)
        self.k1s = []     # (name, kind, inputs dict, packed, scale)
        self._by_signs = {}
        for i, layer in self.layers.items():
            for name, m in (("qkv", layer.self_attn.qkv_proj), ("o", layer.self_attn.o_proj),
                            ("gate_up", layer.mlp.gate_up_proj), ("down", layer.mlp.down_proj)):
                assert isinstance(m, W4A4Linear)
                self._by_signs[m.signs.data_ptr()] = (f"layer{i}.{name}", m)

    def __enter__(self):
        self._saved = (qwen3.rmsnorm_rht_quant_pack, qwen3.silu_mul_rht_quant_pack, qwen3.rht_quant_pack_rowtiled)
        rms_k1, silu_k1, plain_k1 = self._saved
        probe = self

        def rms_wrap(x, weight, eps, signs, residual=None, **kw):
            hit = probe._by_signs.get(signs.data_ptr())
            if hit is None:
                return rms_k1(x, weight, eps, signs, residual, **kw)
            inputs = {"x": x.clone(), "weight": weight, "eps": eps, "signs": signs,
                      "residual": None if residual is None else residual.clone()}
            out = rms_k1(x, weight, eps, signs, residual, **kw)
            inputs["residual_out"] = None if residual is None else out[2].clone()
            packed = rowtiled_to_reference(out[0], x.shape[0]) if kw.get("rowtiled") else out[0].clone()
            probe.k1s.append((hit[0], "rmsnorm", inputs, packed, out[1].clone()))
            return out

        def silu_wrap(gate_up, signs, **kw):
            hit = probe._by_signs.get(signs.data_ptr())
            out = silu_k1(gate_up, signs, **kw)
            if hit is not None:
                packed = rowtiled_to_reference(out[0], gate_up.shape[0]) if kw.get("rowtiled") else out[0].clone()
                probe.k1s.append((hit[0], "silu_mul", {"gate_up": gate_up.clone(), "signs": signs},
                                  packed, out[1].clone()))
            return out

        def plain_wrap(x, signs, **kw):
            hit = probe._by_signs.get(signs.data_ptr())
            out = plain_k1(x, signs, **kw)
            if hit is not None:
                probe.k1s.append((hit[0], "plain", {"x": x.clone(), "signs": signs},
                                  rowtiled_to_reference(out[0], x.shape[0]), out[1].clone()))
            return out

        qwen3.rmsnorm_rht_quant_pack, qwen3.silu_mul_rht_quant_pack = rms_wrap, silu_wrap
        qwen3.rht_quant_pack_rowtiled = plain_wrap
        self._patched = []
        for name, m in self._by_signs.values():
            def fq(packed, scale, rowtiled=False, _m=m, _name=name, _orig=m.forward_quantized):
                out = _orig(packed, scale, rowtiled=rowtiled)
                ref_packed = rowtiled_to_reference(packed, scale.shape[0]) if rowtiled else packed.clone()
                probe.gemms.append((_name, _m, ref_packed, scale.clone(), out.clone(), False))
                return out
            def fqs(packed, scale, _m=m, _name=name, _orig=m.forward_quantized_silu):
                out = _orig(packed, scale)
                ref_packed = rowtiled_to_reference(packed, scale.shape[0])
                probe.gemms.append((_name, _m, ref_packed, scale.clone(), out.clone(), True))
                return out
            def fw(x, _m=m, _name=name, _orig=m.forward):
                out = _orig(x)
                probe.linears.append((_name, _m, x.clone(), out.clone()))
                return out
            m.forward_quantized = fq
            m.forward_quantized_silu = fqs
            m.forward = fw
            self._patched.append(m)
        return self

    def __exit__(self, *exc):
        qwen3.rmsnorm_rht_quant_pack, qwen3.silu_mul_rht_quant_pack, qwen3.rht_quant_pack_rowtiled = self._saved
        for m in self._patched:
            del m.forward_quantized
            del m.forward_quantized_silu
            del m.forward
        return False


def _rows(t, rows):
    return t if rows is None else t[rows]


def reference_weights(module: W4A4Linear):
    """(packed int8 [N, K/2], bf16 scale bits [N, K/128]) in the reference layout."""
    sd = module.state_dict()
    return sd["packed_weight"].cpu().numpy(), bf16_bits(sd["weight_scale"])


def check_gemms(probe: ProjectionProbe, rows=None, weights=None):
    """Every recorded GEMM output equals the oracle's, bit for bit.
    ``weights`` maps a recorded name to (packed, scale bits) to use instead
    of the module's own (e.g. tensors read from a checkpoint file)."""
    assert probe.gemms, "no W4A4 GEMM was recorded"
    cache = {}
    for name, m, packed, scale, out, silu in probe.gemms:
        if name not in cache:
            cache[name] = weights[name] if weights and name in weights else reference_weights(m)
        wp, sw = cache[name]
        a = _rows(packed, rows).cpu().numpy()
        sa = bf16_bits(_rows(scale, rows))
        ref = oracle.w4a4_gemm(a, wp, sa, sw)
        if silu:  # SiLU-mul in the epilogue: the separate kernel on the oracle's gate/up output
            ref = bf16_bits(silu_mul(torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).to(out.device)))
        got = bf16_bits(_rows(out, rows))
        assert np.array_equal(got, ref), f"{name}: GEMM output differs from the oracle " \
                                         f"({int((got != ref).sum())} of {ref.size} elements)"
    return len(probe.gemms)


def check_linears(probe: ProjectionProbe, rows=None, weights=None):
    """Every recorded whole W4A4Linear forward (bf16 input -> K1 -> GEMM)
    equals the oracle chain on the same input, bit for bit."""
    assert probe.linears, "no W4A4Linear forward was recorded"
    for name, m, x, out in probe.linears:
        wp, sw = weights[name] if weights and name in weights else reference_weights(m)
        flat = _rows(x.reshape(-1, m.in_features), rows)
        packed, scale = oracle.rht_quant_pack(bf16_bits(flat), m.signs.cpu().numpy())
        ref = oracle.w4a4_gemm(packed, wp, scale, sw)
        got = bf16_bits(_rows(out.reshape(-1, m.out_features), rows))
        assert np.array_equal(got, ref), f"{name}: linear output differs from the oracle chain"
    return len(probe.linears)


def check_k1s(probe: ProjectionProbe, rows=None):
    """Every recorded fused K1 equals the oracle K1 on the separate producer's
    output, bit for bit; the written-back residual equals bf16(x + residual)."""
    assert probe.k1s, "no fused K1 was recorded"
    for name, kind, inp, packed, scale in probe.k1s:
        if kind == "rmsnorm":
            x = _rows(inp["x"], rows).contiguous()
            res = None if inp["residual"] is None else _rows(inp["residual"], rows).contiguous()
            if res is not None:
                expect = (x.float() + res.float()).to(torch.bfloat16)
                assert torch.equal(_rows(inp["residual_out"], rows), expect), f"{name}: residual write-back"
                y, _ = rmsnorm(x, inp["weight"], inp["eps"], residual=res.clone())
            else:
                y = rmsnorm(x, inp["weight"], inp["eps"])
        elif kind == "plain":
            y = _rows(inp["x"], rows).contiguous()
        else:
            y = silu_mul(_rows(inp["gate_up"], rows).contiguous())
        p_ref, s_ref = oracle.rht_quant_pack(bf16_bits(y), inp["signs"].cpu().numpy())
        assert np.array_equal(_rows(packed, rows).cpu().numpy(), p_ref), f"{name}: fused K1 codes differ"
        assert np.array_equal(bf16_bits(_rows(scale, rows)), s_ref), f"{name}: fused K1 scales differ"
    return len(probe.k1s)
