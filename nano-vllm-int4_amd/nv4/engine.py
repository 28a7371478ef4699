"""A fixed-batch runner for the end-to-end decode workload of the quantized path.

It reproduces the steps the reference's engine takes for its latency
benchmark (benchmarks/bench_nano_latency.py:32-121 on nanovllm/engine/*):
requests are prefilled one at a time (serial prefill, each prompt one
forward), then the whole batch decodes together, one token per sequence per
step, the decode forward replayed from a HIP graph captured for that batch
size (nanovllm/engine/model_runner.py:211-276).  A step prepares the
inputs on the host and copies them in (:144-203), runs the model, the LM
head on each sequence's last hidden state and the sampler at the request
temperature (nanovllm/layers/sampler.py:7-12, one HIP launch here), and returns the
tokens to the host; the decode step time is measured around all of it,
and decode tokens/s = batch * 1000 / mean step ms over the pure-decode
steps (bench_nano_latency.py:118).

Scope: a fixed set of requests that all fit (the reference's continuous
batching, preemption and prefix cache are outside the quantized path), the
KV cache laid out as ``max_num_seqs`` contiguous runs of blocks (sequence
slot s owns blocks s*B .. s*B+B-1), and one GPU.
"""
from __future__ import annotations

import math
import time

import numpy as np
import torch

from .attention import decode_workspace
from .layers.linear_w4a4 import W4A4Linear
from .layers.linear_w4a16 import W4A16Linear
from .qwen3 import BF16Linear, Qwen3ForCausalLM, W4A16Qwen3ForCausalLM
from .sampler import Sampler
from .utils.context import get_context, reset_context, set_context


def qwen3_8b_config(num_hidden_layers: int = 36):
    """Qwen3-8B dimensions (random weights: nothing is downloaded)."""
    from transformers import Qwen3Config
    return Qwen3Config(vocab_size=151936, hidden_size=4096, intermediate_size=12288,
                       num_hidden_layers=num_hidden_layers, num_attention_heads=32, num_key_value_heads=8,
                       head_dim=128, max_position_embeddings=40960, rms_norm_eps=1e-6, rope_theta=1_000_000.0,
                       tie_word_embeddings=False, attention_bias=False, hidden_act="silu", torch_dtype="bfloat16")


@torch.no_grad()
def random_init(model: Qwen3ForCausalLM, seed: int) -> None:
    """Random-init weights of the workload: embeddings and LM head ~N(0,
    0.02), norms 1, W4A4 projections with codes uniform in [-8, 7] (random
    bytes), group-128 scales uniform in [0.005, 0.02] and RHT signs +-1, BF16
    projections ~N(0, 0.02), GPTQ projections with uniform nibbles and zero
    points and scales uniform in [0.005, 0.02].  W4A4 weights end in the
    MFMA-tiled order, as after the checkpoint loader."""
    dev = next(model.parameters()).device
    g = torch.Generator(device=dev).manual_seed(seed)
    for name, p in model.named_parameters():
        if not p.dtype.is_floating_point or p.dtype == torch.float16:  # GPTQ tensors: below
            continue
        if name.endswith("norm.weight"):
            p.fill_(1.0)
        else:
            p.copy_(torch.randn(p.shape, generator=g, device=dev, dtype=torch.float32).mul_(0.02))
    for m in model.modules():
        if isinstance(m, W4A16Linear):  # uniform nibbles and zero points, scales in [0.005, 0.02]
            m.qweight.copy_(torch.randint(-2**31, 2**31, m.qweight.shape, generator=g, device=dev, dtype=torch.int64))
            m.qzeros.copy_(torch.randint(-2**31, 2**31, m.qzeros.shape, generator=g, device=dev, dtype=torch.int64))
            m.scales.copy_(0.005 + 0.015 * torch.rand(m.scales.shape, generator=g, device=dev))
    for m in model.modules():
        if isinstance(m, W4A4Linear):
            m.packed_weight.copy_(torch.randint(-128, 128, m.packed_weight.shape, generator=g, device=dev,
                                                dtype=torch.int16))
            m.weight_scale.copy_(0.005 + 0.015 * torch.rand(m.weight_scale.shape, generator=g, device=dev))
            m.signs.copy_(torch.randint(0, 2, m.signs.shape, generator=g, device=dev, dtype=torch.int16) * 2 - 1)
            m.weights_tiled = False
            m.tile_weights_()


def model_tensor_bytes(model) -> int:
    """Bytes of every parameter and registered buffer of ``model``, each
    storage counted once."""
    seen, total = set(), 0
    for t in list(model.parameters()) + list(model.buffers()):
        if t is None or t.numel() == 0:
            continue
        key = (t.untyped_storage().data_ptr(), t.device)
        if key in seen:
            continue
        seen.add(key)
        total += t.untyped_storage().nbytes()
    return total


class Engine:
    def __init__(self, hf_config, use_w4a4: bool, max_num_seqs: int, max_model_len: int, block_size: int = 256,
                 device="cuda:0", model: Qwen3ForCausalLM | None = None, kv_cache: torch.Tensor | None = None,
                 seed: int = 0, use_w4a16: bool = False, keep_weights_f6: bool = False):
        self.cfg, self.device = hf_config, torch.device(device)
        self.max_num_seqs, self.max_model_len, self.block_size = max_num_seqs, max_model_len, block_size
        self.blocks_per_seq = math.ceil(max_model_len / block_size)
        if model is None:
            prev = torch.get_default_dtype()
            torch.set_default_dtype(torch.bfloat16)
            try:
                with torch.device(self.device):
                    model = W4A16Qwen3ForCausalLM(hf_config) if use_w4a16 else Qwen3ForCausalLM(hf_config, use_w4a4)
            finally:
                torch.set_default_dtype(prev)
            random_init(model, seed)
            if use_w4a16:
                model.fuse_projections_()
        self.model = model.eval()
        if keep_weights_f6:  # fp6 tiles of the W4A4 weights for prefill-sized calls (opt-in)
            for m in self.model.modules():
                if isinstance(m, W4A4Linear):
                    m.keep_weights_f6_(True)
        cfg = hf_config
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        nblocks = max_num_seqs * self.blocks_per_seq
        shape = (2, cfg.num_hidden_layers, nblocks, block_size, cfg.num_key_value_heads, head_dim)
        if kv_cache is None or tuple(kv_cache.shape) != shape:
            kv_cache = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
        self.kv_cache = kv_cache
        ws = decode_workspace(max_num_seqs, cfg.num_attention_heads, max_model_len, head_dim, self.device)
        for i, layer in enumerate(self.model.model.layers):
            attn = layer.self_attn.attn
            attn.k_cache, attn.v_cache = kv_cache[0, i], kv_cache[1, i]
            attn.workspace, attn.max_context = ws, max_model_len
        self.block_tables = torch.arange(nblocks, dtype=torch.int32, device=self.device).view(
            max_num_seqs, self.blocks_per_seq)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.graph_vars: dict[str, torch.Tensor] = {}
        self._stage: dict[int, dict] = {}
        self.sampler = Sampler()

    def model_bytes(self) -> int:
        """Device bytes of the model's tensors (parameters and buffers: quantized
        codes, scales, signs, kept fp6 weight tiles, embeddings, norms, LM
        head), without the KV cache and the attention workspace -- the figure
        the reference reports as model tensor bytes."""
        return model_tensor_bytes(self.model)

    # ------------------------------------------------------------ helpers
    def _slots(self, seq_slot: int, start: int, end: int):
        base = seq_slot * self.blocks_per_seq * self.block_size
        return list(range(base + start, base + end))

    def _check_fits(self, seq_slots, lengths) -> None:
        """Every sequence slot must exist and every length fit the slot's run
        of blocks: a longer sequence would write its keys and values into the
        next slot's blocks and attend to a truncated context.  Host lists
        only, so the check costs no device synchronisation."""
        for s, n in zip(seq_slots, lengths):
            if not 0 <= s < self.max_num_seqs:
                raise ValueError(f"sequence slot {s} outside [0, {self.max_num_seqs})")
            if not 1 <= n <= self.max_model_len:
                raise ValueError(f"sequence length {n} outside [1, max_model_len={self.max_model_len}]")

    def _to_dev(self, values, dtype):
        return torch.tensor(values, dtype=dtype, pin_memory=True).to(self.device, non_blocking=True)

    def sample(self, logits: torch.Tensor, temperatures: torch.Tensor) -> torch.Tensor:
        return self.sampler(logits, temperatures)

    # -------------------------------------------------------------- steps
    @torch.inference_mode()
    def prefill(self, seq_slot: int, token_ids: list[int], temperature: float) -> int:
        n = len(token_ids)
        self._check_fits([seq_slot], [n])
        input_ids = self._to_dev(token_ids, torch.int64)
        positions = self._to_dev(list(range(n)), torch.int64)
        cu = self._to_dev([0, n], torch.int32)
        slot_mapping = self._to_dev(self._slots(seq_slot, 0, n), torch.int32)
        set_context(True, cu, cu, n, n, slot_mapping, None, None, seqlens_q=(n,))
        logits = self.model.compute_logits(self.model(input_ids, positions))
        token = self.sample(logits, self._to_dev([temperature], torch.float32)).tolist()[0]
        reset_context()
        return token

    def _staging(self, bs: int) -> dict:
        """The decode inputs of batch size ``bs`` in one pinned host buffer and
        its device twin, so a step moves them in one copy: int64 input_ids
        [bs] and positions [bs], then int32 context_lens [bs] and slot_mapping
        [bs].  The device views are the captured graph's static inputs; the
        block tables stay in place until the step's sequence slots change."""
        st = self._stage.get(bs)
        if st is None:
            host = torch.empty(3 * bs, dtype=torch.int64, pin_memory=True)
            dev = torch.zeros(3 * bs, dtype=torch.int64, device=self.device)
            i32 = dev[2 * bs:].view(torch.int32)
            i32[:bs].fill_(1)  # a valid context for the capture's warm-up forward
            st = {"host": host, "np": host.numpy(), "dev": dev, "input_ids": dev[:bs], "positions": dev[bs:2 * bs],
                  "context_lens": i32[:bs], "slot_mapping": i32[bs:], "block_tables": self.block_tables[:bs].clone(),
                  "slots": tuple(range(bs)), "copied": torch.cuda.Event()}
            st["copied"].record(torch.cuda.current_stream(self.device))
            self._stage[bs] = st
        return st

    def _set_decode_inputs(self, seq_slots, last_tokens, lengths):
        bs = len(seq_slots)
        if len(last_tokens) != bs or len(lengths) != bs or bs < 1:
            raise ValueError("decode needs one last token and one length per sequence slot")
        self._check_fits(seq_slots, lengths)
        st = self._staging(bs)
        st["copied"].synchronize()  # the previous step's copy has read the host buffer
        h = st["np"]
        n = np.asarray(lengths, dtype=np.int64)
        h[:bs] = last_tokens
        h[bs:2 * bs] = n - 1
        h32 = h[2 * bs:].view(np.int32)
        h32[:bs] = n
        h32[bs:] = np.asarray(seq_slots, dtype=np.int64) * (self.blocks_per_seq * self.block_size) + n - 1
        st["dev"].copy_(st["host"], non_blocking=True)
        st["copied"].record(torch.cuda.current_stream(self.device))
        slots = tuple(int(s) for s in seq_slots)
        if slots != st["slots"]:
            st["block_tables"].copy_(self.block_tables[torch.tensor(slots, device=self.device)])
            st["slots"] = slots
        return st["input_ids"], st["positions"], st["context_lens"], st["slot_mapping"], st["block_tables"]

    @torch.inference_mode()
    def capture(self, bs: int) -> None:
        """Capture the decode forward (model only, as the reference does) for
        batch size ``bs`` with static input buffers."""
        st = self._staging(bs)
        gv = {k: st[k] for k in ("input_ids", "positions", "slot_mapping", "context_lens", "block_tables")}
        set_context(False, slot_mapping=gv["slot_mapping"], context_lens=gv["context_lens"],
                    block_tables=gv["block_tables"])
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.model(gv["input_ids"], gv["positions"])  # warm-up outside the graph
        torch.cuda.current_stream(self.device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            gv["outputs"] = self.model(gv["input_ids"], gv["positions"])
        reset_context()
        self.graphs[bs], self.graph_vars[bs] = graph, gv

    @torch.inference_mode()
    def decode(self, seq_slots, last_tokens, lengths, temperatures: torch.Tensor, eager: bool = False,
               return_logits: bool = False):
        """One decode step for the sequences in ``seq_slots`` whose current
        lengths (prompt + generated, including the new input token) are
        ``lengths``; returns the sampled tokens (a host list)."""
        bs = len(seq_slots)
        input_ids, positions, context_lens, slot_mapping, block_tables = self._set_decode_inputs(
            seq_slots, last_tokens, lengths)
        if eager or bs not in self.graphs:
            set_context(False, slot_mapping=slot_mapping, context_lens=context_lens, block_tables=block_tables)
            hidden = self.model(input_ids, positions)
        else:  # the inputs already sit in the graph's static buffers
            gv = self.graph_vars[bs]
            self.graphs[bs].replay()
            hidden = gv["outputs"]
            set_context(False)
        logits = self.model.compute_logits(hidden)
        reset_context()
        if return_logits:
            return logits
        return self.sample(logits, temperatures).tolist()


def run_decode_benchmark(engine: Engine, prompts: list[list[int]], output_tokens: int, temperature: float = 0.6,
                         seed: int = 20261108, check_graph: bool = True) -> dict:
    """Serial prefill of every prompt, then ``output_tokens - 1`` pure-decode
    steps of the whole batch; wall-clock milliseconds of each step."""
    bs = len(prompts)
    torch.manual_seed(seed)
    temps = torch.full((bs,), temperature, dtype=torch.float32, device=engine.device)
    if bs not in engine.graphs:
        engine.capture(bs)
    lengths = [len(p) for p in prompts]
    last, prefill_ms = [], []
    for s, p in enumerate(prompts):
        torch.cuda.synchronize(engine.device)
        t0 = time.perf_counter()
        last.append(engine.prefill(s, p, temperature))
        prefill_ms.append((time.perf_counter() - t0) * 1e3)
    lengths = [n + 1 for n in lengths]
    result = {"prefill_ms": prefill_ms}
    if check_graph:  # graph replay must reproduce the eager step exactly
        slots = list(range(bs))
        a = engine.decode(slots, last, lengths, temps, eager=True, return_logits=True).clone()
        b = engine.decode(slots, last, lengths, temps, return_logits=True).clone()
        result["graph_equals_eager"] = bool(torch.equal(a, b))
        result["logits_finite"] = bool(torch.isfinite(b).all())
    decode_ms = []
    for _ in range(output_tokens - 1):
        torch.cuda.synchronize(engine.device)
        t0 = time.perf_counter()
        last = engine.decode(list(range(bs)), last, lengths, temps)
        decode_ms.append((time.perf_counter() - t0) * 1e3)
        lengths = [n + 1 for n in lengths]
    mean = sum(decode_ms) / len(decode_ms)
    result.update(decode_ms=decode_ms, decode_ms_mean=mean, tokens_per_s=bs * 1000.0 / mean,
                  last_tokens=last)
    return result


def seeded_prompts(batch: int, length: int, vocab: int, seed: int = 20261108) -> list[list[int]]:
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randint(0, vocab, (batch, length), generator=g).tolist()


def count_w4a4(model) -> int:
    return sum(isinstance(m, W4A4Linear) for m in model.modules())


def count_bf16(model) -> int:
    return sum(isinstance(m, BF16Linear) for m in model.modules())


def count_w4a16(model) -> int:
    return sum(isinstance(m, W4A16Linear) for m in model.modules())
