"""Next-token sampler (MI355X): the reference's Sampler in one HIP launch.

The reference (nanovllm/layers/sampler.py:5-12) samples
``argmax(softmax(logits / T) / clamp(Exp(1), 1e-10))`` -- the Gumbel-max
form of drawing from softmax(logits / T) -- with seven torch operations over
the [B, vocab] logits.  ``gumbel_sample`` draws from the same distribution in
one pass over the logits (``nv4_gumbel_sample_ws``: column chunks of every row
in parallel, then a merge of their maxima): argmax of ``logits / T - log(E)`` with
E = -log(U) and U from a counter-based Philox4x32-10 stream keyed by
(seed, offset), so a step's draws are reproducible.  ``Sampler`` keeps the
reference's module interface and advances the offset once per call.
"""
from __future__ import annotations

import ctypes

import torch
from torch import nn

from . import _lib


def gumbel_sample(logits: torch.Tensor, temperatures: torch.Tensor, seed: int, offset: int,
                  out: torch.Tensor | None = None, split: bool = True) -> torch.Tensor:
    """logits [B, V] (bf16 or fp32, rows may be strided), temperatures fp32 [B]
    -> int64 [B] token ids.  ``split`` spreads each row over several
    workgroups (two launches, nv4_gumbel_sample_ws); the tokens are the same
    as the one-launch form's."""
    if logits.shape[0] > 65535:
        split = False
    if logits.ndim != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [B, V] with unit column stride")
    if logits.dtype == torch.bfloat16:
        code = _lib.BF16
    elif logits.dtype == torch.float32:
        code = _lib.FP32
    else:
        raise TypeError("logits must be BF16 or FP32")
    B, V = logits.shape
    if temperatures.dtype != torch.float32 or tuple(temperatures.shape) != (B,) or not temperatures.is_contiguous():
        raise TypeError("temperatures must be contiguous FP32 [B]")
    if out is None:
        out = torch.empty((B,), dtype=torch.int64, device=logits.device)
    if any(not t.is_cuda or t.device != logits.device for t in (temperatures, out)):
        raise ValueError("All tensors must be on one CUDA device")
    lib = _lib.load()
    stream = torch.cuda.current_stream(logits.device).cuda_stream
    seed_c, off_c = ctypes.c_uint64(seed & (2**64 - 1)), ctypes.c_uint64(offset & (2**64 - 1))
    with torch.cuda.device(logits.device):
        if split:
            # each row spread over several workgroups, partials from torch's caching allocator
            P = lib.nv4_gumbel_sample_chunks(B, V)
            ws = torch.empty((2 * B * P,), dtype=torch.int32, device=logits.device)
            rc = lib.nv4_gumbel_sample_ws(ctypes.c_void_p(logits.data_ptr()), logits.stride(0), code,
                                          ctypes.c_void_p(temperatures.data_ptr()), B, V, seed_c, off_c,
                                          ctypes.c_void_p(ws.data_ptr()), ws.numel() * 4,
                                          ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream))
        else:
            rc = lib.nv4_gumbel_sample(ctypes.c_void_p(logits.data_ptr()), logits.stride(0), code,
                                       ctypes.c_void_p(temperatures.data_ptr()), B, V, seed_c, off_c,
                                       ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream))
    _lib.check(rc, "gumbel_sample")
    return out


class Sampler(nn.Module):
    """Drop-in for nanovllm.layers.sampler.Sampler: forward(logits,
    temperatures) -> sampled token ids.  ``seed`` defaults to a draw from
    torch's CPU generator (so torch.manual_seed fixes the stream)."""

    def __init__(self, seed: int | None = None):
        super().__init__()
        self.seed = seed
        self.offset = 0

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor) -> torch.Tensor:
        if self.seed is None:
            self.seed = int(torch.randint(0, 2**62, (1,)).item())
        tokens = gumbel_sample(logits, temperatures, self.seed, self.offset)
        self.offset += 1
        return tokens
