#!/usr/bin/env python3
"""Benchmark of the W4A4 quantized-linear hot path on one MI355X.

A step is one decode-sized pass of the W4A4 linear chain of one Qwen3-8B
decoder layer: for each fused projection (qkv 4096->6144, o 4096->4096,
gate_up 4096->24576, down 12288->4096) the W4A4Linear forward -- RHT +
group-128 INT4 quantization + packing of the activations, then the grouped
INT4 GEMM -- on M = 32 rows of synthetic activations (the reference's
operator table, benchmarks/README.md:121-133, times exactly this chain at
M = 32 and M = 4096).

Timing rules:
* Every step is a HIP-graph replay (captured once per weight set), so the
  numbers are GPU time, not Python launch overhead.
* Steps rotate through ``--rotate`` distinct weight sets (~92 MB each, 6 by
  default = 550 MB), more than the 256 MB Infinity Cache, so weights stream
  from HBM as they would across the 36 layers of the model.
* The dominant kernel (the grouped INT4 GEMM) is also timed on its own: a
  graph of back-to-back launches over the rotating weight sets, replayed
  between HIP events on the stream it runs on; its algorithmic bytes
  (M*K/2 + M*K/64 + N*K/2 + N*K/64 + 2*M*N per launch) over that time give
  the roofline fraction against the 8 TB/s HBM peak.
* The CPU baseline is the repository's C oracle (the same chain, and one
  entry per workload configuration), timed on this host's cores on a
  bounded number of steps.
* ``e2e_decode``: the decoder around the hot path, end to end -- the
  reference's latency benchmark (32 x 4096-token prompts, serial prefill,
  bs32 decode of 256 tokens with HIP-graph steps) on the Qwen3-8B-shaped
  model with random weights, W4A4 projections against BF16 hipBLASLt ones.

Prints ONE JSON line.  ``--gpus`` above 1 is rejected: this path runs on one
GPU (rows of M are independent; see the design notes for sharding).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "nano-vllm-int4_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PROJECTIONS = ("qkv", "o", "gate_up", "down")
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, published (no sparsity)
FP6_PEAK_TOPS = 10100.0        # MI355X dense fp6 / fp4 MFMA, published (no sparsity)
# Published reference numbers (one RTX A6000), full RHT+quant+pack+GEMM chain
# at M = 32, benchmarks/README.md:126-129, in microseconds.
PUBLISHED_CHAIN_M32_US = {"qkv": 28.12, "o": 21.87, "gate_up": 86.85, "down": 64.65}
PUBLISHED_GEMM_M32_US = {"qkv": 21.25, "o": 14.97, "gate_up": 79.86, "down": 46.06}
PUBLISHED_GEMM_M4096_US = {"qkv": 861.77, "o": 505.62, "gate_up": 3293.68, "down": 1550.64}
# Published bs32 decode tokens/s of the real Qwen3-8B (one RTX A6000, 32 x 4096
# prompts, 256 output tokens), benchmarks/README.md:65.
PUBLISHED_E2E_TOKS = {"bf16": 564.57, "w4a4": 766.71, "w4a16": None}


def k2_bytes(M, N, K):
    return M * K // 2 + M * K // 64 + N * K // 2 + N * K // 64 + 2 * M * N


def k1_bytes(M, K):
    return 2 * M * K + K + M * K // 2 + M * K // 64


def k3_bytes(M, N, K):
    return 2 * M * K + N * K // 2 + 2 * N * K // 128 + 4 * (K // 128) * (N // 8) + 2 * M * N


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=600)
    ap.add_argument("--warmup", type=int, default=60)
    ap.add_argument("--m", type=int, default=32, help="rows per step (decode batch)")
    ap.add_argument("--rotate", type=int, default=6, help="distinct weight sets cycled through")
    ap.add_argument("--no-detail", action="store_true", help="skip the per-projection M=32/M=4096 table")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured matrix-core / HBM peaks")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="target CPU baseline sample length")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end bs32 decode of the decoder")
    ap.add_argument("--e2e-layers", type=int, default=36, help="decoder layers of the end-to-end model")
    ap.add_argument("--e2e-tokens", type=int, default=256, help="output tokens per request (end to end)")
    ap.add_argument("--pmc-prefill", action="store_true",
                    help="for rocprofv3 --pmc: three launches of the fp6 prefill GEMM at gate_up M=4096 "
                         "(after its operand conversion) and three 256 MiB device copies, then exit")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="for rocprofv3 --pmc: eager decode GEMM launches (3 rounds over the rotating sets) "
                         "and three plain 256 MiB device copies as the counter calibration, then exit")
    return ap.parse_args()


# ----------------------------------------------------------------- inputs
def make_layer_sets(torch, W, M, rotate, dev):
    """Weight sets: set 0 is the seeded CPU workload (shared with the oracle),
    the others are drawn on the GPU with the same recipe.  Packed weights are
    stored in the MFMA-tiled order, as W4A4Linear keeps them after loading."""
    import nv4
    acts, sets = {}, []
    base = {}
    for p in PROJECTIONS:
        case = W.w4a4_case(p, M)
        acts[p] = case.x.to(dev)
        base[p] = (case.signs.to(dev), nv4.tile_weights(case.w_packed.to(dev)), case.w_scale.to(dev))
    sets.append(base)
    g = torch.Generator(device=dev)
    g.manual_seed(W.BASE_SEED + 1000)
    for _ in range(1, rotate):
        layer = {}
        for p in PROJECTIONS:
            N, K = W.PROJECTIONS[p]
            sg = (torch.randint(0, 2, (K,), generator=g, device=dev, dtype=torch.int8) * 2 - 1)
            wp = torch.randint(-128, 128, (N, K // 2), generator=g, device=dev, dtype=torch.int16).to(torch.int8)
            sw = (0.005 + 0.015 * torch.rand(N, K // 128, generator=g, device=dev)).to(torch.bfloat16)
            layer[p] = (sg.contiguous(), nv4.tile_weights(wp.contiguous()), sw.contiguous())
        sets.append(layer)
    return acts, sets


def make_gemm_sets(torch, W, p, dev):
    """Tiled weight sets (and scales) of one projection for its GEMM-alone
    timing, drawn on the GPU with the workload recipe, rotation_sets(N, K)
    of them."""
    import nv4
    N, K = W.PROJECTIONS[p]
    g = torch.Generator(device=dev)
    g.manual_seed(W.BASE_SEED + 5000 + N + K)
    out = []
    for _ in range(rotation_sets(N, K)):
        wp = torch.randint(-128, 128, (N, K // 2), generator=g, device=dev, dtype=torch.int16).to(torch.int8)
        sw = (0.005 + 0.015 * torch.rand(N, K // 128, generator=g, device=dev)).to(torch.bfloat16)
        out.append((nv4.tile_weights(wp), sw))
    return out


STEPS_PER_GRAPH = 60


# ------------------------------------------------------------- graph timing
GRAPH_MIN_LAUNCHES = 48   # launches per captured graph (the list is repeated up to this)


def graph_launch_us(torch, launches, replays):
    """Average microseconds per launch of ``launches`` (callables that each
    enqueue exactly one kernel on the current stream), captured back to back
    in one HIP graph and replayed between two HIP events on the capturing
    stream.  Inside a graph consecutive kernels start as the previous one
    ends, so this is kernel time, not host launch time.  The list is repeated
    until the graph holds at least GRAPH_MIN_LAUNCHES launches (the replays
    shrink to keep about ``replays`` x the original launch count): a graph of
    a few short kernels replays faster on the GPU than the host can submit
    it, and would otherwise time the host (an empty kernel measured 3.3 us per
    launch in 6-launch graphs against 1.7 us in 48-launch ones)."""
    rep = max(1, -(-GRAPH_MIN_LAUNCHES // len(launches)))
    launches = list(launches) * rep
    replays = max(2, -(-replays // rep))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in launches:
            fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in launches:
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * len(launches))
    del g
    return us


# ------------------------------------------------------------ counter pass
COPY_BYTES = 256 << 20


def pmc_pass(torch, linear, R):
    """Kernels for a hardware-counter run: the W4A4 linear (K1 + K2) of every
    projection and weight set, three rounds, then three device-to-device
    copies of exactly COPY_BYTES (read COPY_BYTES, write COPY_BYTES) to scale
    FETCH_SIZE and WRITE_SIZE into bytes."""
    for _ in range(3):
        for l in range(R):
            for p in PROJECTIONS:
                linear(l, p)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"pmc pass done: {3 * R * len(PROJECTIONS)} linear launches, 3 copies of {COPY_BYTES} bytes", flush=True)


DECODE_GEMM_SOURCES = ("nano-vllm-int4_amd/csrc/w4a4_gemm.hip", "nano-vllm-int4_amd/csrc/nv4_common.h",
                       "nano-vllm-int4_amd/csrc/norm_ops.h", "nano-vllm-int4_amd/csrc/k2_launch.h",
                       "nano-vllm-int4_amd/Makefile")


def decode_gemm_source_sha():
    """SHA-256 over the sources of the decode GEMM kernels (the recorded
    counter traffic belongs to exactly these)."""
    import hashlib
    h = hashlib.sha256()
    for rel in DECODE_GEMM_SOURCES:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()


def pmc_prefill(torch, W, dev):
    """Kernels for a hardware-counter run of the prefill GEMM: the W4A4
    grouped GEMM at gate_up M=4096 (K1 codes of seeded activations, MFMA-tiled
    weights), three launches on the fp6 path (each: the operand conversion
    kernel, then k2_prefill_f6), then three copies of COPY_BYTES for the
    FETCH_SIZE / WRITE_SIZE calibration."""
    import nv4
    M, (N, K) = 4096, W.PROJECTIONS["gate_up"]
    g = torch.Generator(device=dev)
    g.manual_seed(W.BASE_SEED + 3000)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    sg = torch.randint(0, 2, (K,), generator=g, device=dev, dtype=torch.int8) * 2 - 1
    wp = nv4.tile_weights(torch.randint(-128, 128, (N, K // 2), generator=g, device=dev,
                                        dtype=torch.int16).to(torch.int8))
    sw = (0.005 + 0.015 * torch.rand(N, K // 128, generator=g, device=dev)).to(torch.bfloat16)
    pk = torch.empty((M, K // 2), dtype=torch.int8, device=dev)
    sc = torch.empty((M, K // 128), dtype=torch.bfloat16, device=dev)
    nv4.rht_quant_pack(x, sg, out_packed=pk, out_scale=sc)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    for _ in range(3):
        nv4.w4a4_grouped_gemm(pk, wp, sc, sw, out=out, weights_tiled=True, path="fp6")
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc prefill pass done: 3 fp6 prefill GEMMs at gate_up M=4096, 3 copies of "
          f"{COPY_BYTES} bytes", flush=True)


def measured_traffic():
    """HBM bytes per decode-GEMM launch from the committed counter summary
    (two rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled by the
    copy calibration).  The summary records the hash of the kernel sources it
    was measured on; when those sources have changed since, the figure is
    stale and is reported as None with the reason."""
    path = ROOT / "profiles" / "decode_gemm_m32_traffic.json"
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return {"bytes_per_launch": None, "source": "no counter summary committed"}
    if rec.get("kernel_source_sha256") != decode_gemm_source_sha():
        return {"bytes_per_launch": None,
                "source": f"{path.name} was measured on other kernel sources (stale): re-run the --pmc passes"}
    return rec


ROTATE_BYTES = 320 << 20   # distinct weight bytes a per-projection timing rotates through (> 256 MB MALL)


def rotation_sets(N, K):
    """Weight sets one projection's GEMM timing rotates through: enough that
    their bytes exceed the 256 MB Infinity Cache, so every launch streams its
    weights from HBM."""
    return max(2, -(-ROTATE_BYTES // (N * K // 2 + N * K // 64)))


def k2_medians(torch, gemm, nsets, rounds=9, replays=20):
    """Per projection, the median over ``rounds`` rounds of the decode GEMM's
    microseconds per launch (a graph of back-to-back launches over the
    projection's ``nsets[p]`` rotating weight sets, replayed between HIP
    events), the projections in a freshly shuffled order every round."""
    import random
    rng = random.Random(20261108)
    samples = {p: [] for p in PROJECTIONS}
    order = list(PROJECTIONS)
    for _ in range(rounds):
        rng.shuffle(order)
        for p in order:
            samples[p].append(graph_launch_us(torch, [lambda l=l, p=p: gemm(l, p) for l in range(nsets[p])],
                                              replays))
    return {p: statistics.median(v) for p, v in samples.items()}


# -------------------------------------------------------------- end to end
def e2e_decode(torch, layers, out_tokens):
    """The reference's latency benchmark on the Qwen3-8B-shaped decoder with
    random weights: 32 requests of 4096 seeded token ids, serial prefill, then
    bs32 decode of ``out_tokens`` tokens (HIP-graph steps), for the W4A4, the
    BF16 (hipBLASLt) and the W4A16 (GPTQ, fused q/k/v and gate/up) projections;
    decode tokens/s = 32 * 1000 / mean step ms over the pure-decode steps
    (benchmarks/bench_nano_latency.py:32-121)."""
    from nv4.engine import Engine, qwen3_8b_config, run_decode_benchmark, seeded_prompts
    cfg = qwen3_8b_config(layers)
    prompts = seeded_prompts(32, 4096, cfg.vocab_size)
    res, kv = {}, None
    for which in ("w4a4", "bf16", "w4a16"):
        eng = Engine(cfg, use_w4a4=(which == "w4a4"), use_w4a16=(which == "w4a16"), max_num_seqs=32,
                     max_model_len=4096 + out_tokens, device="cuda:0", seed=1, kv_cache=kv)
        kv = eng.kv_cache
        r = run_decode_benchmark(eng, prompts, output_tokens=out_tokens)
        if not (r["graph_equals_eager"] and r["logits_finite"]):
            raise RuntimeError(f"end-to-end {which}: graph replay differs from eager or logits not finite")
        steps = sorted(r["decode_ms"])
        model_bytes = eng.model_bytes()
        res[which] = {"tokens_per_s": round(r["tokens_per_s"], 1), "decode_ms_mean": round(r["decode_ms_mean"], 4),
                      "model_tensor_bytes": model_bytes, "model_tensor_gib": round(model_bytes / 2**30, 3),
                      "decode_ms_p50": round(steps[len(steps) // 2], 4),
                      "prefill_ms_mean": round(sum(r["prefill_ms"][1:]) / (len(r["prefill_ms"]) - 1), 2),
                      "published_a6000_tokens_per_s": PUBLISHED_E2E_TOKS[which]}
        print(f"[e2e] {which}: {res[which]['tokens_per_s']} tok/s, {res[which]['decode_ms_mean']} ms/step",
              file=sys.stderr, flush=True)
        del eng
        torch.cuda.empty_cache()
    del kv
    torch.cuda.empty_cache()
    res["w4a4_over_bf16"] = round(res["w4a4"]["tokens_per_s"] / res["bf16"]["tokens_per_s"], 4)
    res["model_tensor_gib_published_a6000"] = {"bf16": 15.28, "w4a4": 5.67}  # benchmarks/README.md:68-69
    res["model_tensor_bytes_note"] = ("parameters and buffers of the model on the GPU (no KV cache); W4A4 "
                                      "without the opt-in fp6 prefill copies of the weights")
    res["w4a16_over_bf16"] = round(res["w4a16"]["tokens_per_s"] / res["bf16"]["tokens_per_s"], 4)
    res["workload"] = (f"Qwen3-8B-shaped decoder ({layers} layers, hidden 4096, intermediate 12288, 32 q / 8 kv "
                       "heads, vocab 151936), random weights; 32 requests x 4096 seeded token ids, serial "
                       f"prefill, bs32 decode of {out_tokens} tokens (HIP graph), KV cache bf16 paged "
                       "(block 256); tokens/s over the pure-decode steps")
    return res


# ---------------------------------------------------------------- CPU leg
def cpu_threads():
    """Host threads for the CPU baseline: every core this process may run on
    (its affinity set), bounded by OMP_NUM_THREADS when the host sets it (a
    host that shares its cores among GPU jobs sets it to the job's share, 16
    cores per GPU)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(cap)) if cap.isdigit() and int(cap) > 0 else n, n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, warmups=2, min_runs=5, seconds=2.0, max_runs=200):
    for _ in range(warmups):
        fn()
    times = []
    start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - start < seconds and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(M, seconds):
    """The oracle (the repository's C restatement of the reference's numerics,
    OpenMP over rows) on this host's cores, on the same seeded workloads:
    the bench step (the W4A4 chain of the four projections at M), and one
    entry per workload configuration -- o_proj chain at M = 32, the W4A16
    fused-QKV GEMM at M = 1 / 8 / 32, gate_up and down at M = 4096 (a
    64-row sample, scaled by 4096 / 64: rows are independent in both K1 and
    K2) and down at M = 32.  Medians of >= 5 runs after 2 warm-ups."""
    import numpy as np
    import torch

    import oracle
    from nv4 import workloads as W

    threads, affinity = cpu_threads()
    torch.set_num_threads(threads)

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    def chain_fn(projections, rows):
        cases = []
        for p in projections:
            c = W.w4a4_case(p, rows)
            cases.append((bits(c.x), c.signs.numpy(), c.w_packed.numpy(), bits(c.w_scale)))

        def run():
            for x, sg, wp, sw in cases:
                pk, sc = oracle.rht_quant_pack(x, sg, threads=threads)
                oracle.w4a4_gemm(pk, wp, sc, sw, threads=threads)
        return run

    model = cpu_model()
    med, n = _median_time(chain_fn(PROJECTIONS, M), seconds=seconds)
    entry = {
        "value": round(med * 1e6, 1), "unit": "us/step", "cores": threads, "kind": "port",
        "sample": (f"{n} steps (after 2 warm-ups) of the oracle's W4A4 chain, M={M}, qkv/o/gate_up/down, "
                   f"median; {threads} OpenMP threads (affinity {affinity}) on {model}"),
        "cpu_model": model, "affinity_cores": affinity,
    }
    configs = {}
    med, n = _median_time(chain_fn(["o"], 32), seconds=1.0)
    configs["config0_o_chain_M32"] = {"value_us": round(med * 1e6, 1), "runs": n}
    for m16 in (1, 8, 32):
        c = W.w4a16_case(m16)
        args = (bits(c.x), c.qweight.numpy(), c.qzeros.numpy(), c.scales.numpy().view(np.uint16))
        med, n = _median_time(lambda a=args: oracle.w4a16_gemm(*a, x_dtype=oracle.X_FP16, threads=threads),
                              seconds=1.0)
        configs[f"config1_w4a16_qkv_M{m16}"] = {"value_us": round(med * 1e6, 1), "runs": n}
    for proj, key in (("gate_up", "config2_gate_up_M4096"), ("down", "config3_down_M4096")):
        med, n = _median_time(chain_fn([proj], 64), seconds=2.0)
        configs[key] = {"value_us": round(med * 1e6 * 4096 / 64, 1), "runs": n,
                        "sample": "64 of 4096 rows (K1 + K2), scaled x64"}
    med, n = _median_time(chain_fn(["down"], 32), seconds=1.0)
    configs["config3_down_chain_M32"] = {"value_us": round(med * 1e6, 1), "runs": n}
    entry["configs"] = configs
    return entry


# -------------------------------------------------------------------- main
def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this hot path runs on one GPU "
              "(one MI355X per box); rows of M shard across GPUs with no exchange.", file=sys.stderr)
        sys.exit(2)

    import torch

    import nv4
    from nv4 import workloads as W

    nv4._lib.load()  # raises if the HIP library is missing: there is no fallback
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.pmc_prefill:
        pmc_prefill(torch, W, dev)
        return
    from nv4.kernels.rht_a4 import rowtiled_rows
    from nv4.kernels.w4a4_grouped import ROWTILED_MAX_M, w4a4_gemm_rowtiled

    M, R = args.m, max(1, args.rotate)
    # Decode-sized M runs as W4A4Linear runs it: K1 writes the codes in the
    # row-tiled order that the decode GEMM reads.
    rt = M <= ROWTILED_MAX_M
    acts, sets = make_layer_sets(torch, W, M, R, dev)
    pk = {p: torch.empty((rowtiled_rows(M) if rt else M, W.PROJECTIONS[p][1] // 2), dtype=torch.int8, device=dev)
          for p in PROJECTIONS}
    sc = {p: torch.empty((M, W.PROJECTIONS[p][1] // 128), dtype=torch.bfloat16, device=dev) for p in PROJECTIONS}
    out = {p: torch.empty((M, W.PROJECTIONS[p][0]), dtype=torch.bfloat16, device=dev) for p in PROJECTIONS}

    def linear(l, p):  # W4A4Linear.forward: RHT+quant+pack, then the grouped GEMM (tiled weights)
        nv4.w4a4_linear(acts[p], sets[l][p][0], sets[l][p][1], sets[l][p][2],
                        out=out[p], out_packed=pk[p], out_scale=sc[p], weights_tiled=True, packed_rowtiled=rt)

    def step(l):
        for p in PROJECTIONS:
            linear(l, p)

    if args.pmc_pass:
        pmc_pass(torch, linear, R)
        return

    # The GEMM alone, on the codes the last linear call left in pk/sc, over
    # each projection's own rotation of weight sets (> 256 MB per projection).
    k2sets = {p: make_gemm_sets(torch, W, p, dev) for p in PROJECTIONS}
    nsets = {p: len(v) for p, v in k2sets.items()}

    def gemm(l, p):
        w, sw = k2sets[p][l]
        if rt:
            w4a4_gemm_rowtiled(pk[p], w, sc[p], sw, out=out[p])
        else:
            nv4.w4a4_grouped_gemm(pk[p], w, sc[p], sw, out=out[p], weights_tiled=True)


    # Eager reference outputs of set 0, then one graph per weight set.
    step(0)
    torch.cuda.synchronize()
    eager = {p: out[p].clone() for p in PROJECTIONS}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for l in range(R):
            step(l)
    torch.cuda.current_stream().wait_stream(side)
    graphs = []
    for l in range(R):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(l)
        graphs.append(g)
    graphs[0].replay()
    torch.cuda.synchronize()
    for p in PROJECTIONS:
        if not torch.equal(out[p].view(torch.int16), eager[p].view(torch.int16)):
            raise RuntimeError(f"graph replay of {p} differs from the eager launch")

    del graphs
    # Timed steps: graphs of up to STEPS_PER_GRAPH consecutive steps (weight
    # set i % R for step i), so the GPU, not the host's graph submission,
    # sets the pace; exactly --steps steps between the events.
    chunk = min(args.steps, STEPS_PER_GRAPH)

    def steps_graph(n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                step(i % R)
        return g
    g_chunk = steps_graph(chunk)
    g_rem = steps_graph(args.steps % chunk) if args.steps % chunk else None
    for _ in range(-(-args.warmup // chunk)):
        g_chunk.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps // chunk):
        g_chunk.replay()
    if g_rem is not None:
        g_rem.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    step_us = ms_per_step * 1e3
    del g_chunk, g_rem

    # Dominant kernel: the decode GEMM, timed per projection over the rotating
    # weight sets (equal launch counts per projection, so the mean of the
    # per-projection averages is the kernel's average launch).
    k2_us = k2_medians(torch, gemm, nsets, rounds=9, replays=20)
    avg_launch_us = statistics.mean(k2_us.values())
    avg_bytes = statistics.mean(k2_bytes(M, *W.PROJECTIONS[p]) for p in PROJECTIONS)
    achieved = avg_bytes / (avg_launch_us * 1e-6) / 1e9       # GB/s

    traffic = measured_traffic()
    line = {
        "metric": "INT4 GEMM us & % roofline at Qwen3-8B shapes; bs32 decode tokens/s",
        "value": round(step_us, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(step_us / sum(PUBLISHED_CHAIN_M32_US.values()), 4),
        "vs_baseline_note": ("value / the reference's published M=32 chain time summed over the four "
                             "projections (201.49 us, RTX A6000, benchmarks/README.md:126-129)"),
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": (f"W4A4 linear chain of one Qwen3-8B decoder layer at M={M}: RHT+group-128 "
                         "INT4 quant+pack then grouped INT4 GEMM for qkv (6144x4096), o (4096x4096), "
                         "gate_up (24576x4096), down (4096x12288); HIP-graph replays rotating "
                         f"{R} weight sets ({R * 92} MB) past the 256 MB Infinity Cache"),
            "M": M, "rotate": R,
        },
        "roofline": {
            "kernel": ("decode grouped INT4 GEMM on row-tiled activations and MFMA-tiled weights (k2_dec for "
                       "qkv/o/down, k2_wide for gate_up), M=32"),
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (traffic or {}).get("bytes_per_launch"),
            "traffic_source": (traffic or {}).get("source"),
            "avg_launch_us": round(avg_launch_us, 3), "algorithmic_bytes_per_launch": int(avg_bytes),
            "per_projection_us": {p: round(v, 3) for p, v in k2_us.items()},
            "timing": ("median over 9 rounds (projections in shuffled order each round) of HIP events "
                       "around replays of a graph of >= 48 back-to-back launches per projection, cycling "
                       f"through the projection's own weight sets ({nsets}, > 256 MB each)"),
        },
    }

    if not args.no_peaks:
        peaks = measured_peaks(torch, dev)
        line["roofline"]["measured_peak"] = peaks["hbm_read_gbs"]
        line["roofline"]["frac_of_measured"] = round(achieved / peaks["hbm_read_gbs"], 4)
        line["measured_peaks"] = peaks
    if not args.no_detail:
        line["detail"] = detail_table(torch, nv4, W, dev, R)
    del sets, acts, k2sets
    torch.cuda.empty_cache()
    if not args.no_e2e:
        line["e2e_decode"] = e2e_decode(torch, args.e2e_layers, args.e2e_tokens)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(M, args.cpu_seconds)
        line["cpu_baseline"]["gpu_speedup"] = round(line["cpu_baseline"]["value"] / step_us, 1)
    print(json.dumps(line), flush=True)


def measured_peaks(torch, dev):
    """The device's sustained rates, measured by the library's probe kernels
    (`nv4_probe_mfma`, `nv4_probe_read`): int8, fp8 and fp6 matrix-core
    operations per second with every SIMD's matrix pipe fed by eight waves of
    four independent products, and the HBM streaming-read rate over a 1 GiB
    buffer (four times the Infinity Cache).  Medians of 5 timed launches after
    one warm-up; reported beside the published peaks, not instead of them."""
    import ctypes
    from nv4 import _lib
    lib = _lib.load()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    wgs = 8 * cus
    sink = torch.zeros(max(wgs, 1024), dtype=torch.int32, device=dev)
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def timed(launch, reps=5):
        launch()
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            launch()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e-3)
        return statistics.median(ts)

    out = {}
    for kind, name, iters, ops_per in ((0, "int8_mfma_tops", 2000, 2 * 16 * 16 * 64),
                                       (1, "fp8_mfma_tops", 500, 2 * 32 * 32 * 64),
                                       (2, "fp6_mfma_tops", 1000, 2 * 32 * 32 * 64)):
        def run(kind=kind, iters=iters):
            rc = lib.nv4_probe_mfma(kind, iters, wgs, ctypes.c_void_p(sink.data_ptr()), stream())
            if rc != 0:
                raise RuntimeError(f"nv4_probe_mfma failed: {rc}")
        sec = timed(run)
        out[name] = round(wgs * 4 * iters * 4 * ops_per / sec / 1e12, 1)
    buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    buf.fill_(1)

    def rd():
        rc = lib.nv4_probe_read(ctypes.c_void_p(buf.data_ptr()), buf.numel(), ctypes.c_void_p(sink.data_ptr()),
                                stream())
        if rc != 0:
            raise RuntimeError(f"nv4_probe_read failed: {rc}")
    out["hbm_read_gbs"] = round(buf.numel() / timed(rd, reps=9) / 1e9, 1)
    del buf
    out["published"] = {"int8_mfma_tops": 5000.0, "fp8_mfma_tops": 5000.0, "fp6_mfma_tops": FP6_PEAK_TOPS,
                        "hbm_read_gbs": HBM_PEAK_GBS}
    out["method"] = (f"{wgs} workgroups x 4 waves, 4 independent MFMAs per round (16x16x64 i8: 2000 rounds; "
                     "32x32x64 f8: 500 rounds; 32x32x64 f6: 1000 rounds); streaming read of 1 GiB, "
                     "16 nontemporal 16-byte loads per "
                     "thread; HIP events, median of 5 (9 for the read)")
    return out


def detail_table(torch, nv4, W, dev, R):
    """Per projection at M = 32 and M = 4096: K1 and K2 microseconds (graph
    replays of back-to-back launches, weights rotated past the Infinity
    Cache), their roofline fractions, and the BF16 hipBLASLt GEMM (torch.mm)
    on the same shape; then the W4A16 GPTQ GEMM on the fused QKV at M = 1, 8,
    32 (fp16 activations, microseconds per call and HBM fraction)."""
    from nv4.kernels.rht_a4 import rht_quant_pack_rowtiled, rowtiled_rows
    from nv4.kernels.w4a4_grouped import keep_weights_f6, w4a4_gemm_rowtiled
    res = {}
    g = torch.Generator(device=dev)
    g.manual_seed(W.BASE_SEED + 2000)
    for M in (32, 4096):
        reps = 20 if M == 32 else 3
        for p in PROJECTIONS:
            N, K = W.PROJECTIONS[p]
            # Decode: the projection's own weights rotate past the Infinity
            # Cache; prefill is matrix-core bound and rotates two sets.
            rot = rotation_sets(N, K) if M == 32 else 2
            x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
            sg = (torch.randint(0, 2, (K,), generator=g, device=dev, dtype=torch.int8) * 2 - 1)
            wsets = []
            for _ in range(rot):
                wp = torch.randint(-128, 128, (N, K // 2), generator=g, device=dev,
                                   dtype=torch.int16).to(torch.int8)
                sw = (0.005 + 0.015 * torch.rand(N, K // 128, generator=g, device=dev)).to(torch.bfloat16)
                wt = nv4.tile_weights(wp)
                # As W4A4Linear keeps them: tiled INT4 weights and, for the
                # prefill sizes of qkv, o and down, their fp6 tile form
                # (converted once; gate_up's weights are converted per call).
                keep = M > 32 and keep_weights_f6(N, K)
                wsets.append((wt, sw, nv4.weights_to_f6(wt, True) if keep else None))
            scb = torch.empty((M, K // 128), dtype=torch.bfloat16, device=dev)
            ob = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            if M == 32:  # as W4A4Linear runs decode sizes: row-tiled codes
                pkb = torch.empty((rowtiled_rows(M), K // 2), dtype=torch.int8, device=dev)
                l1 = [lambda: rht_quant_pack_rowtiled(x, sg, out_packed=pkb, out_scale=scb)] * rot
                l2 = [lambda w=w: w4a4_gemm_rowtiled(pkb, w[0], scb, w[1], out=ob) for w in wsets]
            else:
                pkb = torch.empty((M, K // 2), dtype=torch.int8, device=dev)
                l1 = [lambda: nv4.rht_quant_pack(x, sg, out_packed=pkb, out_scale=scb)] * rot
                l2 = [lambda w=w: nv4.w4a4_grouped_gemm(pkb, w[0], scb, w[1], out=ob, weights_tiled=True,
                                                        weights_f6=w[2]) for w in wsets]
            us1 = graph_launch_us(torch, l1, reps)
            us2 = graph_launch_us(torch, l2, reps)
            del wsets
            nb = max(2, -(-ROTATE_BYTES // (2 * N * K))) if M == 32 else 2
            wb = [torch.randn(N, K, generator=g, device=dev).to(torch.bfloat16) for _ in range(nb)]
            ob16 = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            l3 = [lambda w=w: torch.mm(x, w.t(), out=ob16) for w in wb]
            us3 = graph_launch_us(torch, l3, reps)
            del wb
            entry = {"k1_us": round(us1, 2), "k2_us": round(us2, 2), "chain_us": round(us1 + us2, 2),
                     "bf16_mm_us": round(us3, 2),
                     "k1_hbm_frac": round(k1_bytes(M, K) / (us1 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
            if M == 32:
                entry["k2_hbm_frac"] = round(k2_bytes(M, N, K) / (us2 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                entry["ref_a6000_gemm_us"] = PUBLISHED_GEMM_M32_US[p]
            else:
                # The size-chosen kernel runs on the fp6 matrix cores (exact for
                # INT4 codes); reported against the int8 peak the target names
                # and against the fp6 peak of the units it uses.
                entry["k2_path"] = "fp6"
                entry["k2_int8_frac"] = round(2 * M * N * K / (us2 * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4)
                entry["k2_fp6_frac"] = round(2 * M * N * K / (us2 * 1e-6) / 1e12 / FP6_PEAK_TOPS, 4)
                entry["ref_a6000_gemm_us"] = PUBLISHED_GEMM_M4096_US[p]
            res[f"M{M}_{p}"] = entry
            print(f"[detail] M={M} {p}: {entry}", file=sys.stderr, flush=True)
    # W4A16 GPTQ GEMM on the fused QKV (N = 6144, K = 4096, fp16 activations), decode sizes;
    # 24 rotating weight sets (315 MB) past the Infinity Cache.
    for M in (1, 8, 32):
        N, K = 6144, 4096
        x = torch.randn(M, K, generator=g, device=dev).to(torch.float16)
        wsets = []
        for _ in range(24):
            qw = torch.randint(-2**31, 2**31, (K // 8, N), generator=g, device=dev, dtype=torch.int64).to(torch.int32)
            qz = torch.randint(-2**31, 2**31, (K // 128, N // 8), generator=g, device=dev,
                               dtype=torch.int64).to(torch.int32)
            sc = (0.005 + 0.015 * torch.rand(K // 128, N, generator=g, device=dev)).to(torch.float16)
            wsets.append((qw, qz, sc))
        o16 = torch.empty((M, N), dtype=torch.float16, device=dev)
        l4 = [lambda w=w: nv4.dequant_matmul_w4a16(x, w[0], w[1], w[2], out=o16) for w in wsets]
        us4 = graph_launch_us(torch, l4, 20)
        del wsets
        entry = {"k3_us": round(us4, 2), "k3_hbm_frac": round(k3_bytes(M, N, K) / (us4 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        res[f"W4A16_M{M}_qkv"] = entry
        print(f"[detail] W4A16 M={M} qkv: {entry}", file=sys.stderr, flush=True)
    return res


if __name__ == "__main__":
    main()
