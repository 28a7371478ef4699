"""The end-to-end workload at its own size (GPU): the Qwen3-8B-shaped W4A4
decoder with random weights (36 layers, hidden 4096, intermediate 12288,
32 q / 8 kv heads, head_dim 128, vocabulary 151936), 32 requests of 4096
seeded token ids prefilled one at a time, then batch-32 decode from the HIP
graph, as the reference's latency benchmark runs it
(benchmarks/bench_nano_latency.py:32-121).

* Prefill: every request's first token is in the vocabulary; inside the
  first request's prefill (M = 4096: the fp6 matrix-core prefill GEMM, the
  size-chosen path), every W4A4
  projection of the first and the last layer equals the oracle on a sample
  of rows, and every fused K1 the oracle K1 (``model_probe``).
* Decode at ~4.1k context: the graph-replayed step's full logits equal the
  eager step's bit for bit and are finite (bench_nano_latency.py:96-107);
  inside the eager step (row-tiled codes from the fused K1s into the decode
  GEMM), every W4A4 projection of the first and last layer equals the oracle
  on all 32 rows; a few more graph steps sample tokens in the vocabulary.
"""
import pytest
import torch

from model_probe import ProjectionProbe, check_gemms, check_k1s, check_linears
from nv4.engine import Engine, qwen3_8b_config, seeded_prompts

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
PROMPT, BATCH, OUT = 4096, 32, 256
ROWS = [0, 1, 255, 256, 1000, 2047, 2048, 3333, 4094, 4095]


@pytest.fixture(scope="module")
def run():
    cfg = qwen3_8b_config(36)
    print("[e2e] building the 36-layer engine", flush=True)
    eng = Engine(cfg, use_w4a4=True, max_num_seqs=BATCH, max_model_len=PROMPT + OUT, device=DEV, seed=1)
    eng.capture(BATCH)  # before any prefill: the capture's warm-up writes slot 0
    prompts = seeded_prompts(BATCH, PROMPT, cfg.vocab_size)
    state = {"eng": eng, "cfg": cfg, "prompts": prompts}
    with ProjectionProbe(eng.model, [0, 35]) as probe:
        first = [eng.prefill(0, prompts[0], 0.6)]
    state["prefill_probe"] = probe
    print("[e2e] prefilling 31 more requests", flush=True)
    for s in range(1, BATCH):
        first.append(eng.prefill(s, prompts[s], 0.6))
    torch.cuda.synchronize()
    state["first"] = first
    return state


def test_prefill_tokens_and_projections(run):
    vocab = run["cfg"].vocab_size
    assert all(0 <= t < vocab for t in run["first"])
    probe = run["prefill_probe"]
    # layers 0 and 35: qkv, gate_up, down through fused K1s; o as a whole forward
    assert check_gemms(probe, rows=ROWS) == 6
    assert check_linears(probe, rows=ROWS) == 2
    assert check_k1s(probe, rows=ROWS) == 6


def test_decode_graph_equals_eager_and_projections(run):
    eng, cfg = run["eng"], run["cfg"]
    slots = list(range(BATCH))
    lengths = [PROMPT + 1] * BATCH
    temps = torch.full((BATCH,), 0.6, device=DEV)
    graph = eng.decode(slots, run["first"], lengths, temps, return_logits=True).clone()
    with ProjectionProbe(eng.model, [0, 35]) as probe:
        eager = eng.decode(slots, run["first"], lengths, temps, eager=True, return_logits=True).clone()
    torch.cuda.synchronize()
    assert graph.shape == (BATCH, cfg.vocab_size)
    assert torch.isfinite(graph).all()
    assert torch.equal(graph, eager), "graph replay of the bs32 decode step differs from the eager step"
    assert check_gemms(probe) == 6
    assert check_linears(probe) == 2
    assert check_k1s(probe) == 6
    last = run["first"]
    for step in range(3):
        last = eng.decode(slots, last, [n + step for n in lengths], temps)
        assert len(last) == BATCH and all(0 <= t < cfg.vocab_size for t in last)
