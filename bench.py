"""Benchmark: AI.IF prefill of Qwen3-4B FP8 on one MI355X.

One step = one AI.IF stage over the whole synthetic corpus: 512 documents
(lognormal lengths, median 256, sigma 0.8, clipped 32..2048) behind a
64-token shared instruction prefix held once in the paged KV arena, packed
into 16384-row packs, each pack's prefill forward pass through the 36
layers, and the yes/no answer read at every document's last row. Weights
are seeded random-init with the Qwen3-4B architecture (no checkpoint is
available offline); token ids are seeded uniform.

Prints ONE JSON line: AI.IF rows/s (`value`), prefill tokens/s, the FP8
GEMM's measured TFLOP/s against the MFMA peak (HIP events around every
GEMM launch of the timed region), and the CPU baseline: the oracle's torch
restatement of the reference path timed on this host on a bounded sample.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--cpu-seconds S]
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "AI.IF rows/sec + prefill tok/s, Qwen3-4B FP8, 1 MI355X; % FP8 MFMA peak"
PEAK_FP8 = 5.0e15        # MI355X dense FP8 MFMA, FLOP/s
PEAK_BF16 = 2.5e15       # dense bf16 MFMA
PEAK_HBM = 8.0e12        # HBM3E bytes/s
WORKLOAD = "qwen3-4b"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--workload", default=WORKLOAD)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="target wall time of the CPU baseline sample (0 skips it)")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads() -> int:
    share = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    return min(share, int(env)) if env and env.isdigit() else share


def attention_pairs(run_packs):
    """(q, k) pairs the causal paged calls evaluate, summed over packs."""
    pairs = 0
    for cu, used in run_packs:
        for s in range(len(used)):
            q_len = cu[s + 1] - cu[s]
            u = used[s]
            # query i sees u - q_len + i + 1 keys
            pairs += q_len * (u - q_len) + q_len * (q_len + 1) // 2
    return pairs


def cpu_baseline(model, workload, target_s):
    """The oracle (the torch restatement of the reference path, fp32
    contractions, the reference's own CPU arithmetic) on this host: whole
    documents of the corpus through the first layers, scaled to all layers
    and reported per fresh token and per document."""
    import torch

    from oracle import qwen3_ref as ref
    from tests.helpers import ref_model

    threads = cpu_threads()
    torch.set_num_threads(threads)
    ref.set_precision(torch.float32)
    cfg = model.config
    # the first layers' weights and the embedding on the host
    sample_layers = 1
    sub = type(model)(**vars(model))
    inner = type(model.model)(**vars(model.model))
    inner.layers = model.model.layers[:sample_layers]
    sub.model = inner
    m = ref_model(sub)
    docs = []
    tokens = 0
    for prompt in workload.prompts:
        docs.append(list(prompt))
        tokens += len(prompt)
        if tokens >= 1024:
            break
    t0 = time.perf_counter()
    ref.forward_documents(m, docs, layers=sample_layers)
    one = time.perf_counter() - t0
    # grow the sample to about target_s of CPU work
    reps = max(1, int(target_s / max(one, 1e-3)))
    reps = min(reps, 20)
    t0 = time.perf_counter()
    for _ in range(reps):
        ref.forward_documents(m, docs, layers=sample_layers)
    elapsed = time.perf_counter() - t0
    ref.set_precision(torch.float64)
    per_token_layer = elapsed / (reps * tokens * sample_layers)
    tok_s = 1.0 / (per_token_layer * cfg.layers)
    docs_per_token = workload.documents / sum(len(p) for p in workload.prompts)
    return dict(value=round(tok_s * docs_per_token, 3), unit="rows/s", cores=threads,
                kind="port", tok_s=round(tok_s, 1),
                sample=(f"{len(docs)} whole documents ({tokens} tokens) x {sample_layers} of "
                        f"{cfg.layers} layers x {reps} reps, {elapsed:.1f} s, scaled to all "
                        f"layers; rows/s = tok/s x documents per token of the corpus"))


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this benchmark runs on one GPU; "
                                   "the path shards by documents with no exchange, so N GPUs "
                                   "are N independent copies of this run"}))
        sys.exit(2)

    import torch

    from quail_amd.arena import KVArena
    from quail_amd.executor import StageRun
    from quail_amd.model import CONFIGS, build_synthetic, retain_answer_head
    from quail_amd.qwen3 import Qwen3Pipeline
    from quail_amd.readout import AnswerRows, AsyncAnswers
    from quail_amd.workload import make_workload

    assert torch.cuda.is_available(), "bench needs a GPU"
    wl = make_workload(args.workload, seed=args.seed)
    cfg = CONFIGS[wl.model]
    t_build = time.perf_counter()
    model = build_synthetic(cfg, seed=args.seed, device="cuda")
    retain_answer_head(model, wl.label_ids[:2])
    num_pages = 3 * wl.chunk_budget // wl.page_tokens + 64
    arena = KVArena(cfg.layers, num_pages, wl.page_tokens, cfg.kv_heads, cfg.head_dim)
    pipe = Qwen3Pipeline(model, arena)
    readout = AsyncAnswers(AnswerRows(model, [wl.label_ids[0]], [wl.label_ids[1]]))
    prefixes, suffixes = wl.groups_input()
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t_build

    def step(record=None):
        run = StageRun(pipe, arena, readout, prefixes, suffixes, wl.chunk_budget)
        if record is not None:
            orig = pipe.forward_chunk

            def forward(chunk):
                u = chunk.host["unified"]
                record.append(([int(x) for x in u["cu_q"]], [int(x) for x in u["used"]]))
                return orig(chunk)
            pipe.forward_chunk = forward
        try:
            answers = run.run()
        finally:
            pipe.forward_chunk = Qwen3Pipeline.forward_chunk.__get__(pipe)
        return answers, run.stats

    log(f"setup {t_build:.1f} s: {wl.documents} documents, {cfg.layers} layers, "
        f"{num_pages} KV pages")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log("warmup done")

    packs = []
    timer = []
    pipe.engine.gemm_timer = timer
    stats = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        answers, st = step(record=packs if i == 0 else None)
        stats.append(st)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    pipe.engine.gemm_timer = None

    gemm_ms = 0.0
    gemm_flops = 0.0
    per_shape = {}
    for m, n, k, start, end in timer:
        ms = start.elapsed_time(end)
        gemm_ms += ms
        gemm_flops += 2.0 * m * n * k
        s = per_shape.setdefault(f"{k}x{n}", [0.0, 0.0, 0])
        s[0] += 2.0 * m * n * k
        s[1] += ms
        s[2] += 1
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12
    launches = len(timer)

    fresh = stats[0]["fresh_tokens"]
    docs = wl.documents
    ms_step = elapsed * 1e3 / args.steps
    rows_s = docs * args.steps / elapsed
    tok_s = fresh * args.steps / elapsed
    pairs = attention_pairs(packs)
    f_gemm = cfg.gemm_flops_per_token() * fresh
    f_attn = cfg.attention_flops_per_pair() * pairs
    h, i_, hq, hk, d = cfg.hidden, cfg.intermediate, cfg.heads, cfg.kv_heads, cfg.head_dim
    # streaming HBM bytes per token per layer as the reference fuses them:
    # two add_rms_norm_quant (x, res in; res, e4m3, scales out: 14h + h/16),
    # qk_norm_rope (q, k in and out: 4 (hq + hk) d), the KV scatter (k, v in
    # and out: 8 hk d), the attention-output quant (bf16 in, e4m3 out: 3 hq d)
    # and silu_mul_quant (gate_up in, e4m3 out: 5 i)
    b_layer = 14 * h + h // 16 + 4 * (hq + hk) * d + 8 * hk * d + 3 * hq * d + 5 * i_
    b_stream = b_layer * cfg.layers * fresh
    t_roof = f_gemm / PEAK_FP8 + f_attn / PEAK_BF16 + b_stream / PEAK_HBM
    e2e_frac = t_roof / (elapsed / args.steps)

    log(f"timed {args.steps} steps: {elapsed:.3f} s")
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(model, wl, args.cpu_seconds)
        log(f"cpu baseline: {cpu['sample']}")

    line = {
        "metric": METRIC,
        "value": round(rows_s, 2),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 (fp32 accumulate), bf16 activations",
        "data": "synthetic (seeded random-init Qwen3-4B weights, uniform token ids)",
        "config": {
            "workload": ("Qwen3-4B FP8 AI.IF prefill: 512 documents, lognormal(256, 0.8) "
                         "clipped 32..2048 tokens, 64-token shared prefix in the paged arena, "
                         "16384-row packs"),
            "documents": docs, "fresh_tokens": fresh, "packs": stats[0]["chunks"],
            "borrowed_tokens": stats[0]["borrowed_tokens"], "attention_pairs": pairs,
            "parallelism": "none (1 GPU)",
        },
        "prefill_tok_s": round(tok_s, 1),
        "e2e_roofline_frac": round(e2e_frac, 4),
        "roofline": {
            "bound": "mfma",
            "kernel": "qx_gemm_fp8_blockscaled (all four Qwen3-4B shapes)",
            "achieved": round(gemm_tflops, 2),
            "peak": PEAK_FP8 / 1e12,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops * 1e12 / PEAK_FP8, 4),
            "traffic": None,
            "launches": launches,
            "avg_launch_us": round(gemm_ms * 1e3 / max(launches, 1), 2),
            "gemm_time_share": round(gemm_ms * 1e-3 / elapsed, 4),
            "per_shape_tflops": {s: round(v[0] / (v[1] * 1e-3) / 1e12, 1)
                                 for s, v in per_shape.items()},
        },
        "cpu_baseline": cpu,
        "setup_s": round(t_build, 1),
    }
    print(json.dumps(line, default=lambda o: o.item() if hasattr(o, "item") else str(o)))


if __name__ == "__main__":
    main()
