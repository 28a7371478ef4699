"""Single-GPU RHT-aware W4A4 linear, W128/A128, clipping 0.9 (MI355X).

Drop-in for ``nanovllm.layers.linear_w4a4.W4A4Linear`` (reference
nanovllm/layers/linear_w4a4.py:15-36): same constructor checks, the same
buffers (``packed_weight`` int8 [out, in/2], ``weight_scale`` bf16
[out, in/128], ``signs`` int8 [in]) so state dicts and the checkpoint loader
carry over, and the same forward: RHT + quantize + pack the activations
(K1), then the grouped INT4 GEMM (K2), on the current stream through one C
ABI call (``nv4_w4a4_linear``).  Temporary buffers come from torch's caching
allocator, so the forward can be captured in a HIP graph.

``tile_weights_()`` (called by the loaders once the weights are in) reorders
``packed_weight`` in place into the MFMA-tiled order that the decode
kernels read in whole cache lines; the forward then uses the tiled entry
point, with bit-identical results.

On request (``keep_weights_f6_(True)``, or ``Engine(keep_weights_f6=True)``)
a layer also keeps ``weight_f6``, the fp6 tile form the prefill GEMM reads
(0.75 bytes per weight on top of the 0.5 of the INT4 codes, rebuilt whenever
the weights are loaded), so prefill-sized calls convert only their
activations -- for weights up to ``KEEP_F6_MAX_BYTES`` of fp6 tiles
(``keep_weights_f6``: qkv, o and down of Qwen3-8B; gate_up converts per
call).  It is off by default: it buys about 3 % per prefill GEMM call for
+72 % of those layers' weight bytes.  The copy is used only while
``packed_weight`` is the tensor version it was made from; weights without a
version counter (inference tensors) never keep one, so no in-place write can
leave it stale.  ``state_dict()`` and ``load_state_dict()`` still see the
reference [out, in/2] layout and do not hold ``weight_f6``.
"""
import torch
from torch import nn
import torch.distributed as dist

from .. import _lib
from ..kernels.w4a4_grouped import (ROWTILED_MAX_M, keep_weights_f6, rowtiled_silu_fits, tile_weights, untile_weights,
                                   w4a4_gemm_rowtiled, w4a4_gemm_rowtiled_silu, w4a4_grouped_gemm, weights_to_f6)
from ..kernels.w4a4_linear import w4a4_linear


def _version_of(t):
    try:
        return t._version
    except RuntimeError:  # inference tensors track no version
        return None


class W4A4Linear(nn.Module):
    def __init__(self, input_size: int, output_size: int, bias: bool = False, keep_weights_f6: bool = False):
        super().__init__()
        if dist.is_available() and dist.is_initialized() and dist.get_world_size() != 1:
            raise ValueError("W4A4Linear supports one GPU only")
        if bias or input_size not in (4096, 12288) or output_size % 8:
            raise ValueError("W4A4 requires bias-free Qwen3-8B projection shapes")
        self.in_features, self.out_features = input_size, output_size
        self.register_buffer("packed_weight", torch.empty(output_size, input_size // 2, dtype=torch.int8))
        self.register_buffer("weight_scale", torch.empty(output_size, input_size // 128, dtype=torch.bfloat16))
        self.register_buffer("signs", torch.empty(input_size, dtype=torch.int8))
        self.register_buffer("weight_f6", None, persistent=False)
        self.weights_tiled = False
        self.keep_f6 = keep_weights_f6
        # Decode-sized forwards: the K1 launch reads this layer's weights into
        # the Infinity Cache while its one-workgroup-per-row transform runs.
        self.prefetch_weights = True

    @torch.no_grad()
    def tile_weights_(self) -> "W4A4Linear":
        """Reorder ``packed_weight`` into the MFMA-tiled layout (GPU, once) and
        build its fp6 tile form for prefill."""
        if not self.weights_tiled and self.out_features % 16 == 0 and self.packed_weight.is_cuda:
            self.packed_weight.copy_(tile_weights(self.packed_weight))
            self.weights_tiled = True
        self._refresh_f6()
        return self

    @torch.no_grad()
    def keep_weights_f6_(self, enable: bool = True) -> "W4A4Linear":
        """Keep (or drop) the fp6 tile form of the weights for prefill-sized
        calls; made now if the weights are loaded and tiled."""
        self.keep_f6 = enable
        self._refresh_f6()
        return self

    @torch.no_grad()
    def _refresh_f6(self) -> None:
        version = _version_of(self.packed_weight)
        keep = (self.keep_f6 and self.packed_weight.is_cuda and version is not None
                and keep_weights_f6(self.out_features, self.in_features))
        self.weight_f6 = weights_to_f6(self.packed_weight, self.weights_tiled) if keep else None
        self._f6_version = version

    def _f6(self):
        """``weight_f6`` while ``packed_weight`` is unchanged since it was made
        (an in-place write bumps the tensor's version); otherwise None, and
        prefill calls convert the weights themselves."""
        version = _version_of(self.packed_weight)
        if self.weight_f6 is None or version is None or getattr(self, "_f6_version", -1) != version:
            return None
        return self.weight_f6

    def weight_bytes(self) -> int:
        """Device bytes of the layer's tensors: INT4 codes, scales, signs and
        (when kept) the fp6 tile form."""
        n = sum(t.numel() * t.element_size() for t in (self.packed_weight, self.weight_scale, self.signs))
        return n + (self.weight_f6.numel() if self.weight_f6 is not None else 0)

    @torch.no_grad()
    def assign_quantized_(self, packed: torch.Tensor, scale: torch.Tensor, signs: torch.Tensor) -> "W4A4Linear":
        """Install checkpoint tensors in the reference layout (packed int8
        [out, in/2], bf16 scales [out, in/128], int8 signs [in]) onto this
        module's device; on a GPU the weights are then tiled in place."""
        self.packed_weight.copy_(packed)
        self.weight_scale.copy_(scale)
        self.signs.copy_(signs)
        self.weights_tiled = False
        return self.tile_weights_()

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        if self.weights_tiled:
            destination[prefix + "packed_weight"] = untile_weights(self.packed_weight)

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)
        if self.weights_tiled and prefix + "packed_weight" in state_dict:
            with torch.no_grad():
                self.packed_weight.copy_(tile_weights(self.packed_weight))
        if self.weight_f6 is not None and prefix + "packed_weight" in state_dict:
            self._refresh_f6()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.in_features or x.dtype != torch.bfloat16:
            raise ValueError("W4A4Linear requires BF16 activations with the configured input width")
        flat = x.reshape(-1, self.in_features).contiguous()
        # RHT + quantize + pack, then the grouped INT4 GEMM; packed codes and
        # scales come from the caching allocator, so the forward can be
        # captured in a HIP graph.
        out = w4a4_linear(flat, self.signs, self.packed_weight, self.weight_scale, weights_tiled=self.weights_tiled,
                          weights_f6=self._f6())
        return out.reshape(*x.shape[:-1], self.out_features)

    def uses_rowtiled(self, m: int) -> bool:
        """Whether a call with M rows takes the row-tiled decode path
        (tiled weights and M <= 32), so its producer should quantize with
        ``rowtiled=True``."""
        return self.weights_tiled and m <= ROWTILED_MAX_M

    def prefetch_target(self, rowtiled: bool):
        """What the K1 producing this layer's row-tiled codes should prefetch:
        the head of its packed weights (``nv4_w4a4_prefetch_bytes``), or None
        off the row-tiled path."""
        if not (rowtiled and self.prefetch_weights):
            return None
        n = _lib.load().nv4_w4a4_prefetch_bytes(self.out_features, self.in_features)
        return self.packed_weight.view(-1)[:n] if n > 0 else None

    def forward_quantized(self, packed: torch.Tensor, scale: torch.Tensor, rowtiled: bool = False) -> torch.Tensor:
        """The GEMM half of ``forward`` on activations already quantized by
        ``rht_quant_pack`` (or a fused producer + K1: ``nv4.kernels.decoder_ops``)
        with this module's signs: packed int8 [M, in/2], scale bf16 [M, in/128]
        -> bf16 [M, out].  ``rowtiled``: the codes are in the row-tiled order
        ([ceil(M/16)*16, in/2], ``rht_quant_pack_rowtiled``; needs
        ``uses_rowtiled(M)``)."""
        if rowtiled:
            return w4a4_gemm_rowtiled(packed, self.packed_weight, scale, self.weight_scale)
        return w4a4_grouped_gemm(packed, self.packed_weight, scale, self.weight_scale,
                                 weights_tiled=self.weights_tiled, weights_f6=self._f6())

    def uses_rowtiled_silu(self, m: int) -> bool:
        """For a fused gate/up projection (gate rows, then up rows): whether
        ``forward_quantized_silu`` serves M rows (row-tiled path and the paired
        decode kernel's sizes)."""
        return self.uses_rowtiled(m) and rowtiled_silu_fits(m, self.out_features, self.in_features,
                                                             self.packed_weight.device)

    def forward_quantized_silu(self, packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        """SiLU-and-mul of this fused gate/up projection on row-tiled codes:
        bf16 [M, out/2], the same bits as ``silu_mul(forward_quantized(packed,
        scale, rowtiled=True))`` in one launch (needs ``uses_rowtiled_silu(M)``)."""
        return w4a4_gemm_rowtiled_silu(packed, self.packed_weight, scale, self.weight_scale)
