"""Qwen3 decoder around the quantized linears: the caller side of the hot path.

The module tree, parameter names and numerics follow the reference's
nanovllm/models/qwen3.py:14-233 (BF16 and W4A4 variants behind
``use_w4a4``), so state dicts, the BF16 loader and the W4A4 checkpoint
loader address the same names:

* ``W4A4Linear`` (RHT + group-128 INT4 activations, grouped INT4 GEMM) for
  the fused qkv / o / gate_up / down projections when ``use_w4a4``;
  ``W4A16Linear`` (GPTQ) for separate q/k/v/o/gate/up/down projections when
  ``use_w4a16`` (``W4A16Qwen3ForCausalLM``, the reference's
  nanovllm/models/qwen3_w4a16.py:14-252); plain
  BF16 linears (torch ``F.linear``, i.e. hipBLASLt on ROCm) otherwise, with
  the reference's q/k/v and gate/up shard loaders
  (nanovllm/layers/linear.py:54-156, one GPU).
* RMSNorm with the fused residual add (nanovllm/layers/layernorm.py:16-50),
  the per-head q/k RMSNorm + rotary embedding + KV-cache store
  (nanovllm/models/qwen3.py:78-94, nanovllm/layers/rotary_embedding.py:6-59,
  nanovllm/layers/attention.py:10-40) and SiLU·mul
  (nanovllm/layers/activation.py:8-11): one HIP launch each
  (``nv4.kernels.decoder_ops``), with the rounding points of the
  reference's PyTorch formulation.
* W4A4 layers fuse the input and post-attention add+RMSNorm into the qkv
  and gate_up activation quantization, and SiLU-mul into down's
  (``rmsnorm_rht_quant_pack``, ``silu_mul_rht_quant_pack``): same bits,
  one launch and one activation round trip less per fused pair.  At decode
  sizes SiLU-mul runs in the gate/up GEMM's epilogue instead
  (``W4A4Linear.forward_quantized_silu``), spread over every CU, and down
  takes the plain row-tiled K1: same bits again.
* Embedding and LM head, the head reading only each sequence's last
  position in prefill (nanovllm/layers/embed_head.py:56-66).
* Attention through ``nv4.attention.Attention`` (paged KV cache).

The reference wraps the small ops in ``torch.compile`` (Triton); here they
are hand-written HIP kernels, and the decode step is captured in a HIP graph
by the runner.
"""
from __future__ import annotations

import functools

import torch
import torch.nn.functional as F
from torch import nn

from .attention import Attention
from .kernels.decoder_ops import (lm_head, lm_head_fits, qk_norm_rope_store, rmsnorm, rmsnorm_rht_quant_pack,
                                  silu_mul, silu_mul_rht_quant_pack)
from .kernels.rht_a4 import rht_quant_pack_rowtiled
from .layers.linear_w4a4 import W4A4Linear
from .layers.linear_w4a16 import W4A16Linear, fuse_w4a16
from .utils.context import get_context


class RMSNorm(nn.Module):
    """RMSNorm with the fused residual add (nanovllm/layers/layernorm.py:16-50)
    as one HIP launch (``nv4_rmsnorm``): fp32 arithmetic, the normalised
    value rounded to bf16 before the weight product, the residual kept in
    bf16.  With ``residual`` the sum is written into ``residual`` in place and
    returned as the new residual."""

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x, residual=None):
        return rmsnorm(x.contiguous(), self.weight, self.eps, residual)


class RotaryEmbedding(nn.Module):
    """cos/sin table of the rotary embedding (nanovllm/layers/rotary_embedding.py:
    6-48): ``cos_sin_cache`` fp32 [max_position, 1, head_size], cos in the first
    half, sin in the second.  The rotation itself is applied inside
    ``qk_norm_rope_store``."""

    def __init__(self, head_size: int, max_position: int, base: float) -> None:
        super().__init__()
        inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float) / head_size))
        t = torch.arange(max_position, dtype=torch.float)
        freqs = t[:, None] * inv_freq[None, :]
        cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)
        self.register_buffer("cos_sin_cache", cache, persistent=False)


@functools.lru_cache(maxsize=None)
def _rope(head_size: int, max_position: int, base: float, device: str) -> RotaryEmbedding:
    # One table shared by every layer, as the reference's lru_cache'd get_rope
    # (nanovllm/layers/rotary_embedding.py:51-59); 20 MiB at 40960 positions.
    with torch.device(device):
        return RotaryEmbedding(head_size, max_position, base)


def get_rope(head_size: int, max_position: int, base: float) -> RotaryEmbedding:
    return _rope(head_size, max_position, float(base), str(torch.empty(0).device))


class BF16Linear(nn.Module):
    """One-GPU BF16 linear; ``shards`` maps a shard id to (row offset, rows)
    for the fused q/k/v or gate/up weight (nanovllm/layers/linear.py:54-156)."""

    def __init__(self, input_size: int, output_size: int, shards: dict | None = None) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.empty(output_size, input_size))
        self.shards = shards or {}
        self.weight.weight_loader = self.weight_loader

    def weight_loader(self, param, loaded_weight, shard_id=None):
        if shard_id is None:
            param.data.copy_(loaded_weight)
        else:
            offset, rows = self.shards[shard_id]
            param.data.narrow(0, offset, rows).copy_(loaded_weight)

    def forward(self, x):
        return F.linear(x, self.weight)


class Qwen3Attention(nn.Module):
    def __init__(self, hidden_size, num_heads, num_kv_heads, max_position, head_dim=None, rms_norm_eps=1e-6,
                 rope_theta=1_000_000.0, use_w4a4=False, use_w4a16=False) -> None:
        super().__init__()
        self.num_heads, self.num_kv_heads = num_heads, num_kv_heads
        self.head_dim = head_dim or hidden_size // num_heads
        self.q_size, self.kv_size = num_heads * self.head_dim, num_kv_heads * self.head_dim
        self.scaling = self.head_dim ** -0.5
        qkv_out = self.q_size + 2 * self.kv_size
        self.use_w4a16 = use_w4a16
        if use_w4a16:  # separate GPTQ projections, as the reference's W4A16 model (qwen3_w4a16.py:56-74)
            self.q_proj = W4A16Linear(hidden_size, self.q_size)
            self.k_proj = W4A16Linear(hidden_size, self.kv_size)
            self.v_proj = W4A16Linear(hidden_size, self.kv_size)
            self.o_proj = W4A16Linear(self.q_size, hidden_size)
            object.__setattr__(self, "qkv_fused", None)  # derived by fuse_projections_(), not in the state dict
        elif use_w4a4:
            self.qkv_proj = W4A4Linear(hidden_size, qkv_out)
            self.o_proj = W4A4Linear(self.q_size, hidden_size)
        else:
            self.qkv_proj = BF16Linear(hidden_size, qkv_out, {"q": (0, self.q_size),
                                                              "k": (self.q_size, self.kv_size),
                                                              "v": (self.q_size + self.kv_size, self.kv_size)})
            self.o_proj = BF16Linear(self.q_size, hidden_size)
        self.rotary_emb = get_rope(self.head_dim, max_position, rope_theta)
        self.attn = Attention(num_heads, self.head_dim, self.scaling, num_kv_heads)
        self.q_norm = RMSNorm(self.head_dim, eps=rms_norm_eps)
        self.k_norm = RMSNorm(self.head_dim, eps=rms_norm_eps)

    def fuse_projections_(self):
        """W4A16: q/k/v as one N-concatenated GPTQ linear (same bits)."""
        if self.use_w4a16 and self.qkv_fused is None:
            object.__setattr__(self, "qkv_fused", fuse_w4a16([self.q_proj, self.k_proj, self.v_proj]))

    def forward(self, positions, hidden_states=None, qkv=None):
        if qkv is None and self.use_w4a16:
            h = hidden_states
            qkv = (self.qkv_fused(h) if self.qkv_fused is not None
                   else torch.cat([self.q_proj(h), self.k_proj(h), self.v_proj(h)], dim=-1))
        elif qkv is None:
            qkv = self.qkv_proj(hidden_states)
        ctx = get_context()
        if not ctx.is_prefill and self.attn.k_cache.numel() > 0:
            # Decode: q/k RMSNorm + rotary + KV store inside the attention launch.
            o = self.attn.decode_qkv(qkv, self.q_norm.weight, self.k_norm.weight, self.rotary_emb.cos_sin_cache,
                                     positions, self.q_norm.eps)
            return self.o_proj(o.flatten(1, -1))
        # q/k RMSNorm + rotary + KV-cache store in one launch; prefill also
        # needs the rotated keys and the values as tensors.
        out = qk_norm_rope_store(qkv, self.num_heads, self.num_kv_heads, self.q_norm.weight, self.k_norm.weight,
                                 self.rotary_emb.cos_sin_cache, positions, self.q_norm.eps,
                                 slot_mapping=ctx.slot_mapping, k_cache=self.attn.k_cache,
                                 v_cache=self.attn.v_cache, return_kv=ctx.is_prefill)
        q, k, v = out if ctx.is_prefill else (out, None, None)
        o = self.attn(q, k, v)
        return self.o_proj(o.flatten(1, -1))


class Qwen3MLP(nn.Module):
    def __init__(self, hidden_size, intermediate_size, use_w4a4=False, use_w4a16=False) -> None:
        super().__init__()
        self.use_w4a16 = use_w4a16
        if use_w4a16:  # reference qwen3_w4a16.py:136-160
            self.gate_proj = W4A16Linear(hidden_size, intermediate_size)
            self.up_proj = W4A16Linear(hidden_size, intermediate_size)
            self.down_proj = W4A16Linear(intermediate_size, hidden_size)
            object.__setattr__(self, "gate_up_fused", None)
        elif use_w4a4:
            self.gate_up_proj = W4A4Linear(hidden_size, 2 * intermediate_size)
            self.down_proj = W4A4Linear(intermediate_size, hidden_size)
        else:
            self.gate_up_proj = BF16Linear(hidden_size, 2 * intermediate_size,
                                           {0: (0, intermediate_size), 1: (intermediate_size, intermediate_size)})
            self.down_proj = BF16Linear(intermediate_size, hidden_size)

    def fuse_projections_(self):
        """W4A16: gate/up as one N-concatenated GPTQ linear (same bits)."""
        if self.use_w4a16 and self.gate_up_fused is None:
            object.__setattr__(self, "gate_up_fused", fuse_w4a16([self.gate_proj, self.up_proj]))

    def forward(self, x):
        if self.use_w4a16:
            gate_up = (self.gate_up_fused(x) if self.gate_up_fused is not None
                       else torch.cat([self.gate_proj(x), self.up_proj(x)], dim=-1))
            return self.down_proj(silu_mul(gate_up))
        return self.down_proj(silu_mul(self.gate_up_proj(x)))

    def forward_fused(self, x, residual, norm):
        """W4A4: post-attention add+RMSNorm inside gate_up's quantization,
        SiLU-mul inside down's; returns (output, residual)."""
        # Decode-sized M: row-tiled codes, and each K1 reads the weights of
        # the GEMM that follows it into the Infinity Cache.
        m = x.shape[0]
        rt = self.gate_up_proj.uses_rowtiled(m)
        packed, scale, residual = rmsnorm_rht_quant_pack(x, norm.weight, norm.eps, self.gate_up_proj.signs, residual,
                                                         rowtiled=rt, prefetch=self.gate_up_proj.prefetch_target(rt))
        if self.gate_up_proj.uses_rowtiled_silu(m) and self.down_proj.uses_rowtiled(m):
            # Decode: SiLU-and-mul in the gate/up GEMM's epilogue (spread over
            # every CU), then down's plain row-tiled K1.
            act = self.gate_up_proj.forward_quantized_silu(packed, scale)
            packed, scale = rht_quant_pack_rowtiled(act, self.down_proj.signs,
                                                    prefetch=self.down_proj.prefetch_target(True))
            return self.down_proj.forward_quantized(packed, scale, rowtiled=True), residual
        gate_up = self.gate_up_proj.forward_quantized(packed, scale, rowtiled=rt)
        rt = self.down_proj.uses_rowtiled(m)
        packed, scale = silu_mul_rht_quant_pack(gate_up, self.down_proj.signs, rowtiled=rt,
                                                prefetch=self.down_proj.prefetch_target(rt))
        return self.down_proj.forward_quantized(packed, scale, rowtiled=rt), residual


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, config, use_w4a4=False, use_w4a16=False) -> None:
        super().__init__()
        self.self_attn = Qwen3Attention(
            config.hidden_size, config.num_attention_heads, config.num_key_value_heads,
            config.max_position_embeddings, getattr(config, "head_dim", None), config.rms_norm_eps,
            getattr(config, "rope_theta", 1_000_000.0), use_w4a4, use_w4a16)
        self.mlp = Qwen3MLP(config.hidden_size, config.intermediate_size, use_w4a4, use_w4a16)
        self.input_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        # W4A4 with the 4096-wide hidden state: the norms and SiLU-mul run
        # inside the projections' activation quantization (one launch each).
        self.fused = use_w4a4 and config.hidden_size == 4096

    def forward(self, positions, hidden_states, residual):
        if self.fused:
            attn = self.self_attn
            norm = self.input_layernorm
            rt = attn.qkv_proj.uses_rowtiled(hidden_states.shape[0])
            pf = attn.qkv_proj.prefetch_target(rt)
            if residual is None:
                packed, scale = rmsnorm_rht_quant_pack(hidden_states, norm.weight, norm.eps, attn.qkv_proj.signs,
                                                       rowtiled=rt, prefetch=pf)
                residual = hidden_states
            else:
                packed, scale, residual = rmsnorm_rht_quant_pack(hidden_states, norm.weight, norm.eps,
                                                                 attn.qkv_proj.signs, residual, rowtiled=rt,
                                                                 prefetch=pf)
            hidden_states = attn(positions, qkv=attn.qkv_proj.forward_quantized(packed, scale, rowtiled=rt))
            return self.mlp.forward_fused(hidden_states, residual, self.post_attention_layernorm)
        if residual is None:
            hidden_states, residual = self.input_layernorm(hidden_states), hidden_states
        else:
            hidden_states, residual = self.input_layernorm(hidden_states, residual)
        hidden_states = self.self_attn(positions, hidden_states)
        hidden_states, residual = self.post_attention_layernorm(hidden_states, residual)
        return self.mlp(hidden_states), residual


class Qwen3Model(nn.Module):
    def __init__(self, config, use_w4a4=False, use_w4a16=False) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([Qwen3DecoderLayer(config, use_w4a4, use_w4a16)
                                     for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, input_ids, positions):
        hidden_states, residual = self.embed_tokens(input_ids), None
        for layer in self.layers:
            hidden_states, residual = layer(positions, hidden_states, residual)
        hidden_states, _ = self.norm(hidden_states, residual)
        return hidden_states


class Qwen3ForCausalLM(nn.Module):
    packed_modules_mapping = {
        "q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"), "v_proj": ("qkv_proj", "v"),
        "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1),
    }

    def __init__(self, config, use_w4a4=False, use_w4a16=False) -> None:
        super().__init__()
        if use_w4a4 and use_w4a16:
            raise ValueError("W4A16 and W4A4 cannot be enabled together")
        self.model = Qwen3Model(config, use_w4a4, use_w4a16)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids, positions):
        return self.model(input_ids, positions)

    def compute_logits(self, hidden_states):
        ctx = get_context()
        if ctx.is_prefill and ctx.cu_seqlens_q is not None:
            hidden_states = hidden_states[ctx.cu_seqlens_q[1:] - 1].contiguous()
        if lm_head_fits(hidden_states, self.lm_head.weight):  # decode-sized: one HIP launch
            return lm_head(hidden_states, self.lm_head.weight)
        return F.linear(hidden_states, self.lm_head.weight)


class W4A16Qwen3ForCausalLM(Qwen3ForCausalLM):
    """The reference's GPTQ model (nanovllm/models/qwen3_w4a16.py:228-252):
    separate q/k/v and gate/up W4A16 projections under the checkpoint's names
    (no packed-module mapping, so ``load_model`` copies every GPTQ tensor by
    name).  ``fuse_projections_()`` (after loading) concatenates q/k/v and
    gate/up along N into one GPTQ linear each -- one launch instead of three
    and two, the fused QKV at N = 6144 -- with the parts' parameters kept as
    views, so the state dict is unchanged and the outputs are the same bits."""
    packed_modules_mapping = {}

    def __init__(self, config) -> None:
        super().__init__(config, use_w4a16=True)

    def fuse_projections_(self):
        for layer in self.model.layers:
            layer.self_attn.fuse_projections_()
            layer.mlp.fuse_projections_()
        return self
