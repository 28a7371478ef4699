"""Paged-KV attention for the Qwen3 decoder on MI355X.

Replaces the reference's Attention (nanovllm/layers/attention.py:44-75),
whose KV store is a Triton kernel and whose attention is flash-attn, neither
of which this build uses:

* KV store: each new token's K and V rows go to ``slot_mapping`` slots of
  the caches ``[num_blocks, block_size, num_kv_heads, head_dim]`` (the
  reference's store_kvcache, :10-40).  Here the store is fused into the
  producer of the rotated keys (``nv4.kernels.decoder_ops.qk_norm_rope_store``,
  called by Qwen3Attention before this module), so ``Attention.forward``
  receives caches that already hold the step's tokens.
* Prefill (causal, GQA): ``prefill_attention``, the HIP kernel
  ``nv4_prefill_attention`` (flash-style online softmax on the matrix cores,
  all packed sequences in one launch; replaces flash_attn_varlen_func,
  :64-70).
* Decode: ``paged_decode_attention``, the HIP kernel ``nv4_paged_decode_attention``
  (split over the context, one workgroup per (sequence, KV head, split);
  online softmax in fp32; a second pass merges the splits).  The decoder
  calls ``paged_decode_attention_qkv`` (``Attention.decode_qkv``) instead:
  the same kernel also takes the step's raw qkv rows, normalises and rotates
  q and k itself and stores the step's key and value, so no separate
  ``qk_norm_rope_store`` launch precedes it.
"""
from __future__ import annotations

import ctypes
import functools

import torch
from torch import nn

from . import _lib
from .utils.context import get_context

SPLIT_TOKENS = 256  # context tokens per decode workgroup


def decode_workspace(batch: int, num_heads: int, max_context: int, head_dim: int, device) -> torch.Tensor:
    """fp32 scratch for the split partials of ``paged_decode_attention``."""
    splits = (max_context + SPLIT_TOKENS - 1) // SPLIT_TOKENS
    return torch.empty(batch * num_heads * splits * (head_dim + 2), dtype=torch.float32, device=device)


def paged_decode_attention(q, k_cache, v_cache, block_tables, context_lens, scale, out=None, workspace=None,
                           max_context=None):
    """q [B, Hq, D] bf16 (rows may be strided), caches [nb, bs, Hkv, D] bf16,
    block_tables [B, max_blocks] int32, context_lens [B] int32 -> [B, Hq, D] bf16.
    ``max_context`` bounds every context length (default: the block table's
    capacity)."""
    B, Hq, D = q.shape
    nb, bs, Hkv, Dk = k_cache.shape
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("q and the caches must be BF16")
    if (Dk != D or v_cache.shape != k_cache.shape or block_tables.dtype != torch.int32
            or context_lens.dtype != torch.int32 or tuple(context_lens.shape) != (B,)
            or block_tables.shape[0] != B or q.stride(2) != 1 or q.stride(1) != D):
        raise ValueError("Inconsistent paged attention arguments")
    if max_context is None:
        max_context = block_tables.shape[1] * bs
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=q.device)
    if workspace is None:
        workspace = decode_workspace(B, Hq, max_context, D, q.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(q.device).cuda_stream
    with torch.cuda.device(q.device):
        rc = lib.nv4_paged_decode_attention(
            ctypes.c_void_p(q.data_ptr()), q.stride(0), ctypes.c_void_p(k_cache.data_ptr()),
            ctypes.c_void_p(v_cache.data_ptr()), ctypes.c_void_p(block_tables.data_ptr()), block_tables.shape[1],
            ctypes.c_void_p(context_lens.data_ptr()), ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(workspace.data_ptr()), workspace.numel() * 4, B, Hq, Hkv, D, bs, max_context,
            ctypes.c_float(scale), ctypes.c_void_p(stream))
    _lib.check(rc, "paged_decode_attention")
    return out


def paged_decode_attention_qkv(qkv, num_heads, num_kv_heads, q_norm_w, k_norm_w, cos_sin, positions, slot_mapping,
                               eps, k_cache, v_cache, block_tables, context_lens, scale, out=None, workspace=None,
                               max_context=None):
    """The decode step's q/k RMSNorm + rotary + KV store and the paged decode
    attention in one launch (``nv4_paged_decode_attention_qkv``): the same
    bits as ``qk_norm_rope_store`` followed by ``paged_decode_attention`` on
    its q.  qkv bf16 [B, (Hq + 2 Hkv) * 128] (one token per sequence, rows may
    be strided), positions int64 [B], slot_mapping int32 [B] -> [B, Hq, 128];
    the step's keys and values are stored in the caches."""
    B = qkv.shape[0]
    D = 128
    if qkv.dtype != torch.bfloat16 or qkv.ndim != 2 or qkv.stride(1) != 1:
        raise TypeError("qkv must be BF16 [B, heads*128] with unit column stride")
    if qkv.shape[1] != (num_heads + 2 * num_kv_heads) * D:
        raise ValueError("qkv width does not match the head counts (head_dim 128)")
    if cos_sin.dtype != torch.float32 or cos_sin.shape[-1] != D or not cos_sin.is_contiguous():
        raise TypeError("cos_sin must be a contiguous FP32 [max_position, 128] table")
    if positions.dtype != torch.int64 or tuple(positions.shape) != (B,):
        raise TypeError("positions must be int64 [B]")
    if slot_mapping.dtype != torch.int32 or tuple(slot_mapping.shape) != (B,):
        raise TypeError("slot_mapping must be int32 [B]")
    for w in (q_norm_w, k_norm_w):
        if w.dtype != torch.bfloat16 or tuple(w.shape) != (D,) or not w.is_contiguous():
            raise TypeError("q/k norm weights must be contiguous BF16 [128]")
    nb, bs, Hkv, Dk = k_cache.shape
    if k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("the caches must be BF16")
    if (Dk != D or Hkv != num_kv_heads or v_cache.shape != k_cache.shape or not k_cache.is_contiguous()
            or not v_cache.is_contiguous() or block_tables.dtype != torch.int32
            or context_lens.dtype != torch.int32 or tuple(context_lens.shape) != (B,)
            or block_tables.shape[0] != B):
        raise ValueError("Inconsistent paged attention arguments")
    dev = qkv.device
    for t in (q_norm_w, k_norm_w, cos_sin, positions, slot_mapping, k_cache, v_cache, block_tables, context_lens):
        if t.device != dev:
            raise ValueError("all tensors must be on the device of qkv")
    if max_context is None:
        max_context = block_tables.shape[1] * bs
    if out is None:
        out = torch.empty((B, num_heads, D), dtype=torch.bfloat16, device=dev)
    if workspace is None:
        workspace = decode_workspace(B, num_heads, max_context, D, dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    P = ctypes.c_void_p
    with torch.cuda.device(dev):
        rc = lib.nv4_paged_decode_attention_qkv(
            P(qkv.data_ptr()), qkv.stride(0), P(q_norm_w.data_ptr()), P(k_norm_w.data_ptr()),
            P(cos_sin.data_ptr()), cos_sin.numel() // D, P(positions.data_ptr()), P(slot_mapping.data_ptr()),
            nb * bs, P(k_cache.data_ptr()), P(v_cache.data_ptr()), P(block_tables.data_ptr()),
            block_tables.shape[1], P(context_lens.data_ptr()), P(out.data_ptr()), P(workspace.data_ptr()),
            workspace.numel() * 4, B, num_heads, num_kv_heads, D, bs, max_context, ctypes.c_float(eps),
            ctypes.c_float(scale), P(stream))
    _lib.check(rc, "paged_decode_attention_qkv")
    return out


@functools.lru_cache(maxsize=64)
def _cu_seqlens(lens, device):
    """int32 [B+1] sequence starts on ``device``, made once per batch shape
    (every layer of a prefill reuses it instead of copying it again)."""
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.tensor(lens, dtype=torch.int32).cumsum(0)
    return cu.to(device)


def prefill_attention(q, k, v, seqlens, scale):
    """Causal GQA attention over packed sequences of lengths ``seqlens``
    (q [T, Hq, 128], k/v [T, Hkv, 128] bf16, rows of each tensor contiguous
    in its last two dims) -> bf16 [T, Hq, 128], in one launch of
    ``nv4_prefill_attention``."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3 or q.shape[2] != 128 or k.shape != v.shape:
        raise ValueError("Expected q [T, Hq, 128] and k, v [T, Hkv, 128]")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("q, k and v must be bf16")
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    lens = [int(n) for n in seqlens]
    if k.shape[0] != T or sum(lens) != T or any(n < 1 for n in lens):
        raise ValueError("seqlens must be positive and sum to the number of rows")
    for t in (q, k, v):
        if not t.is_cuda or t.device != q.device or t.stride(2) != 1 or t.stride(1) != D:
            raise ValueError("q, k and v must be CUDA tensors on one device with contiguous heads")
    cu = _cu_seqlens(tuple(lens), q.device)
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    lib = _lib.load()
    stream = torch.cuda.current_stream(q.device).cuda_stream
    with torch.cuda.device(q.device):
        rc = lib.nv4_prefill_attention(
            ctypes.c_void_p(q.data_ptr()), q.stride(0), ctypes.c_void_p(k.data_ptr()), k.stride(0),
            ctypes.c_void_p(v.data_ptr()), v.stride(0), ctypes.c_void_p(out.data_ptr()), out.stride(0),
            ctypes.c_void_p(cu.data_ptr()), len(lens), max(lens), Hq, Hkv, D, ctypes.c_float(scale),
            ctypes.c_void_p(stream))
    _lib.check(rc, "prefill_attention")
    return out


class Attention(nn.Module):
    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads, self.head_dim, self.scale, self.num_kv_heads = num_heads, head_dim, scale, num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.workspace = None  # set by the runner for decode
        self.max_context = None

    def forward(self, q, k, v):
        """q [T, Hq, D]; k, v [T, Hkv, D] in prefill (None in decode, which
        reads the keys and values from the caches)."""
        ctx = get_context()
        if ctx.is_prefill:
            return prefill_attention(q, k, v, ctx.seqlens_q, self.scale)
        return paged_decode_attention(q, self.k_cache, self.v_cache, ctx.block_tables, ctx.context_lens,
                                      self.scale, workspace=self.workspace, max_context=self.max_context)

    def decode_qkv(self, qkv, q_norm_w, k_norm_w, cos_sin, positions, eps):
        """Decode from the raw fused qkv rows: q/k norm, rotary, KV store and
        attention in one launch (``paged_decode_attention_qkv``)."""
        ctx = get_context()
        return paged_decode_attention_qkv(qkv, self.num_heads, self.num_kv_heads, q_norm_w, k_norm_w, cos_sin,
                                          positions, ctx.slot_mapping, eps, self.k_cache, self.v_cache,
                                          ctx.block_tables, ctx.context_lens, self.scale, workspace=self.workspace,
                                          max_context=self.max_context)
