"""Benchmark: AI.IF prefill of Qwen3-4B FP8 on one MI355X.

One step = one AI.IF stage over the whole synthetic corpus: 512 documents
(lognormal lengths, median 256, sigma 0.8, clipped 32..2048) behind a
64-token shared instruction prefix held once in the paged KV arena, packed
into 16384-row packs, each pack's prefill forward pass through the 36
layers, and the yes/no answer read at every document's last row. Weights
are seeded random-init with the Qwen3-4B architecture (no checkpoint is
available offline); token ids are seeded uniform.

Prints ONE JSON line: AI.IF rows/s (`value`), prefill tokens/s, the FP8
GEMM's measured TFLOP/s against the MFMA peak (HIP events on the launch
stream around one GEMM launch in 13 of the timed region, a sample that
rotates over the four shapes, the layers and the packs: the events around
every launch would add ~18 ms of idle GPU to a step), and the CPU baseline:
the oracle's torch restatement of the reference path timed on this host on
a bounded sample.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--cpu-seconds S]
                  [--attention unified|tree]
                                          tree: the tree attention path (each
                                          document one causal segment, the
                                          shared prefix read from its parent's
                                          pages, LSE merge) instead of the
                                          unified paged call
  python bench.py --copy-mib 1024 ...     also run one plain copy of that size
                                          (qx_embed over identity ids) before
                                          the warmup, to calibrate HBM counters
  python bench.py --summarize DIR [--copy-mib 1024]
                                          print the summary of a rocprofv3 CSV
                                          output directory (kernel stats or
                                          FETCH_SIZE / WRITE_SIZE counters)
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
PEAK_CLOCK_GHZ = 2.4     # the clock the dense peaks are quoted at
XCDS = 8                 # MI355X: 8 XCDs of 32 CUs
SIMDS = 1024             # 256 CUs x 4 SIMDs
PEAK_HBM = 8.0e12        # HBM3E bytes/s
WORKLOAD = "qwen3-4b"
# HBM bytes per GEMM launch of this workload, from the FETCH_SIZE and
# WRITE_SIZE counter runs summarized in this file (copy-calibrated)
TRAFFIC_FILE = ROOT / "profiles" / "gemm_fp8_qwen3_4b_ai_if_traffic.txt"
COPY_ROW_ELEMS = 2048    # bf16 elements per row of the calibration copy


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--workload", default=WORKLOAD)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--attention", choices=("unified", "tree"), default="unified")
    p.add_argument("--v-dtype", choices=("fp16", "bf16"), default="fp16",
                   help="type of the arena's V pages: fp16 (this engine's arena) or bf16 "
                        "(the reference KVArena's layout)")
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="target wall time of the CPU baseline sample (0 skips it)")
    p.add_argument("--copy-mib", type=int, default=0,
                   help="size of the counter-calibration copy (0: none)")
    p.add_argument("--summarize", default=None,
                   help="summarize a rocprofv3 CSV directory and exit")
    p.add_argument("--gemm-alone-reps", type=int, default=20,
                   help="launches per shape of the GEMM-alone record (0 skips it)")
    p.add_argument("--gemm-sample", type=int, default=13,
                   help="time one GEMM launch in this many inside the timed steps (1: all; "
                        "each timed launch adds two event records to the stream)")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_name(cfg) -> str:
    """qwen3-4b -> Qwen3-4B."""
    return "Qwen3" + cfg.name[len("qwen3"):].upper() if cfg.name.startswith("qwen3") else cfg.name


def describe(wl, cfg, attention) -> str:
    """The workload line of the JSON record."""
    text = (f"{model_name(cfg)} FP8 AI.{wl.function.upper()} prefill: {wl.documents} documents, "
            f"{wl.describe_lengths()}, {wl.prefix_tokens}-token shared prefix in the paged "
            f"arena, {wl.chunk_budget}-row packs")
    return text + ("" if attention == "unified" else ", tree attention path")


def issued_work(cfg, fresh, finals, final_pairs, pairs):
    """(GEMM FLOP, attention FLOP, streaming HBM bytes) the engine issues for
    a stage: every layer but the last on every fresh row; the last layer's
    qkv projection, q/k norm and RoPE and KV write on every row (later packs
    read that KV), its attention, o_proj, MLP and norms on the final rows
    only (the rows an answer is read from). pairs: (query, key) pairs of all
    rows in one layer; final_pairs: those of the final rows."""
    h, i_, hq, hk, d = cfg.hidden, cfg.intermediate, cfg.heads, cfg.kv_heads, cfg.head_dim
    shapes = dict(zip(("qkv", "o", "gate_up", "down"), cfg.linear_shapes()))
    per_row = {k: 2.0 * kk * n for k, (kk, n) in shapes.items()}
    layer = sum(per_row.values())
    f_gemm = (cfg.layers - 1) * layer * fresh + per_row["qkv"] * fresh + (
        per_row["o"] + per_row["gate_up"] + per_row["down"]) * finals
    per_pair = 4.0 * hq * d
    f_attn = per_pair * ((cfg.layers - 1) * pairs + final_pairs)
    norm = 7 * h + h // 32                       # one add_rms_norm_quant
    qk = 4 * (hq + hk) * d                       # qk_norm_rope
    kv = 8 * hk * d                              # KV scatter
    tail = 3 * hq * d + norm + 5 * i_            # attention quant, post norm, silu_mul_quant
    b_stream = (cfg.layers - 1) * (2 * norm + qk + kv + 3 * hq * d + 5 * i_) * fresh + (
        norm + qk + kv) * fresh + tail * finals
    return f_gemm, f_attn, b_stream


def cpu_threads() -> int:
    share = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    return min(share, int(env)) if env and env.isdigit() else share


def attention_pairs(run_packs):
    """(q, k) pairs the attention calls evaluate, summed over packs: each
    entry is (cu_q, used, causal) of one call."""
    pairs = 0
    for cu, used, causal in run_packs:
        for s in range(len(used)):
            q_len = cu[s + 1] - cu[s]
            u = used[s]
            if causal:
                # query i sees u - q_len + i + 1 keys
                pairs += q_len * (u - q_len) + q_len * (q_len + 1) // 2
            else:
                pairs += q_len * u
    return pairs


def cpu_baseline(model, workload, target_s):
    """The oracle (the torch restatement of the reference path, fp32
    contractions, the reference's own CPU arithmetic) on this host: one pack's
    worth of whole documents (up to the pack budget of rows) through the first
    layer, after one warm-up pass, repeated to about target_s, scaled to all
    layers and reported per fresh token and per document."""
    import torch

    from oracle import qwen3_ref as ref
    from tests.helpers import ref_model

    threads = cpu_threads()
    torch.set_num_threads(threads)
    ref.set_precision(torch.float32)
    cfg = model.config
    sample_layers = 1
    sub = type(model)(**vars(model))
    inner = type(model.model)(**vars(model.model))
    inner.layers = model.model.layers[:sample_layers]
    sub.model = inner
    m = ref_model(sub)
    docs = []
    tokens = 0
    for prompt in workload.prompts:
        if tokens + len(prompt) > workload.chunk_budget:
            break
        docs.append(list(prompt))
        tokens += len(prompt)
    ref.forward_documents(m, docs[:2], layers=sample_layers)   # warm-up
    reps = 0
    t0 = time.perf_counter()
    while True:
        ref.forward_documents(m, docs, layers=sample_layers)
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= target_s or elapsed * (reps + 1) / reps > 2 * target_s:
            break
    ref.set_precision(torch.float64)
    per_token_layer = elapsed / (reps * tokens * sample_layers)
    tok_s = 1.0 / (per_token_layer * cfg.layers)
    docs_per_token = workload.documents / sum(len(p) for p in workload.prompts)
    return dict(value=round(tok_s * docs_per_token, 3), unit="rows/s", cores=threads,
                kind="port", tok_s=round(tok_s, 1),
                sample=(f"one-pack subset: {len(docs)} whole documents ({tokens} tokens, "
                        f"shared prefix included) x {sample_layers} of {cfg.layers} layers x "
                        f"{reps} reps, {elapsed:.1f} s, scaled to all layers; rows/s = tok/s x "
                        f"documents per prompt token of the corpus"))


GEMM_ALONE_M = 8192
# (K, N) of the four Qwen3-4B projections: qkv, o_proj, gate_up, down
GEMM_ALONE_SHAPES = ((2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560))


def gemm_alone(reps: int = 20, seed: int = 0):
    """The FP8 block-scaled GEMM alone at the Qwen3-4B projection shapes,
    M = 8192 tokens: activations bf16 N(0, 1) quantized per token per 128
    columns (qx_group_quant), weights N(0, 0.02) quantized per 128 x 128
    block, bf16 output; each shape timed over `reps` launches with HIP events
    on the launch stream after 3 untimed ones. Returns the sub-record."""
    import torch

    from quail_amd.engine import Engine, gemm_config
    from quail_amd.model import quantize_blocks

    eng = Engine(None, num_q_heads=1, num_kv_heads=1, head_dim=128, rotary=None)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    shapes = {}
    m = GEMM_ALONE_M
    for k, n in GEMM_ALONE_SHAPES:
        x = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16)
        q, s = eng.quant(x)
        w, sw = quantize_blocks(torch.randn(n, k, generator=g, device="cuda") * 0.02)
        lin = type("Linear", (), {})()
        lin.weight, lin.weight_scale_inv = w, sw
        out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        for _ in range(3):
            eng.gemm(q, s, lin, out=out)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            eng.gemm(q, s, lin, out=out)
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1e3 / reps
        tflops = 2.0 * m * n * k / (us * 1e-6) / 1e12
        shapes[f"{k}x{n}"] = dict(us=round(us, 2), tflops=round(tflops, 1),
                                  frac=round(tflops * 1e12 / PEAK_FP8, 4),
                                  config=gemm_config(n, k, m))
        del x, q, s, w, sw, out
    total_flops = sum(2.0 * m * n * k for k, n in GEMM_ALONE_SHAPES)
    total_us = sum(v["us"] for v in shapes.values())
    return dict(workload=f"FP8 block-scaled GEMM alone, Qwen3-4B projection shapes (K x N), "
                         f"M = {m} tokens, bf16 output",
                m=m, reps=reps, shapes=shapes,
                tflops_all=round(total_flops / (total_us * 1e-6) / 1e12, 1),
                frac_all=round(total_flops / (total_us * 1e-6) / PEAK_FP8, 4))


def _short(name: str) -> str:
    """A kernel name without its parameter list, at most 110 characters."""
    name = name.strip('"').replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            name = name[:i]
            break
    return name if len(name) <= 110 else name[:107] + "..."


def summarize(directory: str, copy_mib: int) -> None:
    """Print a rocprofv3 CSV directory as text: kernel statistics, and for
    counter runs the mean FETCH_SIZE / WRITE_SIZE per dispatch of each kernel,
    the calibration factor of the plain copy (qx_embed over identity ids,
    copy_mib MiB read and written) and the copy-calibrated HBM bytes per FP8
    GEMM launch."""
    import csv
    from collections import defaultdict

    root = Path(directory)
    stats = sorted(root.rglob("*kernel_stats.csv"))
    counters = sorted(root.rglob("*counter_collection.csv"))
    if stats:
        rows = list(csv.DictReader(open(stats[0])))
        total = sum(float(r["TotalDurationNs"]) for r in rows)
        print(f"{'calls':>7} {'total ms':>10} {'avg us':>10} {'share':>6}  kernel")
        gemm_ns, gemm_calls = 0.0, 0
        for r in rows:
            ns, calls = float(r["TotalDurationNs"]), int(r["Calls"])
            print(f"{calls:7d} {ns / 1e6:10.2f} {ns / calls / 1e3:10.2f} "
                  f"{ns / total:6.1%}  {_short(r['Name'])}")
            if "gemm_fp8" in r["Name"]:
                gemm_ns += ns
                gemm_calls += calls
        if gemm_calls:
            print(f"fp8 gemm, all launches (plain and SwiGLU epilogue): {gemm_calls} launches, "
                  f"avg {gemm_ns / gemm_calls / 1e3:.2f} us")
    for path in counters:
        per = defaultdict(lambda: defaultdict(list))
        dispatch = defaultdict(dict)     # (kernel, dispatch id) -> counter values
        for r in csv.DictReader(open(path)):
            kernel = _short(r["Kernel_Name"])
            per[r["Counter_Name"]][kernel].append(float(r["Counter_Value"]))
            d = dispatch[(kernel, r["Dispatch_Id"])]
            d[r["Counter_Name"]] = float(r["Counter_Value"])
            d["_ns"] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
        if "MfmaUtil" in per or "SQ_INSTS_MFMA" in per or "GRBM_GUI_ACTIVE" in per:
            summarize_mfma(dispatch)
            continue
        for counter, kernels in per.items():
            copy = [v for k, v in kernels.items() if "embed_kernel" in k]
            factor = None
            if copy and copy_mib:
                # the calibration copy is the largest embed dispatch
                factor = copy_mib * 2**20 / (max(copy[0]) * 1024)
            # mean dispatch duration of each kernel (every dispatch runs alone
            # under --pmc), for the calibrated GB/s
            ns = defaultdict(list)
            for (kernel, _), d in dispatch.items():
                ns[kernel].append(d["_ns"])
            print(f"\n{counter} (KiB per dispatch; calibrated: x the copy's factor)")
            print(f"{'calls':>7} {'mean KiB':>14} {'calib. MB':>10} {'avg us':>9} {'GB/s':>8}  "
                  f"kernel")
            for k, v in sorted(kernels.items(), key=lambda kv: -sum(kv[1])):
                kib = sum(v) / len(v)
                us = sum(ns[k]) / len(ns[k]) / 1e3 if ns[k] else 0.0
                cal = kib * 1024 * factor if factor else float("nan")
                rate = cal / (us * 1e-6) / 1e9 if us and factor else float("nan")
                print(f"{len(v):7d} {kib:14.1f} {cal / 1e6:10.2f} {us:9.2f} {rate:8.1f}  {k}")
            gemm = [x for k, v in kernels.items() if "gemm_fp8" in k for x in v]
            if factor and gemm:
                mean = sum(gemm) / len(gemm) * 1024 * factor
                print(f"copy calibration: {copy_mib} MiB moved, counter reads "
                      f"{max(copy[0]) * 1024 / 2**20:.1f} MiB, factor {factor:.4f}")
                print(f"{counter}_bytes_per_gemm_launch = {mean:.0f}")


def summarize_mfma(dispatch) -> None:
    """Per-kernel means of an MFMA/VALU/LDS counter pass: MfmaUtil and
    VALUBusy are rocprofv3's own derived metrics (counter_defs.yaml:
    SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * SIMDs) and
    SQ_ACTIVE_INST_VALU / (CUs * GRBM_GUI_ACTIVE), in %); FP8 TFLOP/s is
    SQ_INSTS_VALU_MFMA_MOPS_F8 * 512 FLOP over the dispatch's duration under
    the profiler; VALU/MFMA is SQ_INSTS_VALU (which counts the MFMAs too)
    per SQ_INSTS_MFMA."""
    from collections import defaultdict

    groups = defaultdict(list)
    for (kernel, _), d in dispatch.items():
        groups[kernel].append(d)
    if any("GRBM_GUI_ACTIVE" in d for d in dispatch.values()):
        summarize_clock(groups)
        return
    cols = ("MfmaUtil", "VALUBusy", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_INSTS_LDS",
            "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_VALU_MFMA_MOPS_F8",
            "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F16")
    print(f"{'calls':>6} {'avg us':>9} {'MFMA%':>6} {'VALU%':>6} {'VALU/MFMA':>9} "
          f"{'LDS inst':>10} {'LDS confl':>10} {'TFLOP/s':>8}  kernel")
    for kernel, ds in sorted(groups.items(), key=lambda kv: -sum(d["_ns"] for d in kv[1])):
        mean = {c: sum(d.get(c, 0.0) for d in ds) / len(ds) for c in cols + ("_ns",)}
        ns = mean["_ns"]
        mops = (mean["SQ_INSTS_VALU_MFMA_MOPS_F8"] + mean["SQ_INSTS_VALU_MFMA_MOPS_BF16"] +
                mean["SQ_INSTS_VALU_MFMA_MOPS_F16"])
        tflops = mops * 512 / (ns * 1e-9) / 1e12 if ns else 0.0
        ratio = (mean["SQ_INSTS_VALU"] / mean["SQ_INSTS_MFMA"]
                 if mean["SQ_INSTS_MFMA"] else float("nan"))
        print(f"{len(ds):6d} {ns / 1e3:9.2f} {mean['MfmaUtil']:6.1f} {mean['VALUBusy']:6.1f} "
              f"{ratio:9.2f} {mean['SQ_INSTS_LDS']:10.3g} {mean['SQ_LDS_BANK_CONFLICT']:10.3g} "
              f"{tflops:8.1f}  {kernel}")


def summarize_clock(groups) -> None:
    """Per-kernel means of a clock pass: GRBM_GUI_ACTIVE (busy cycles at the
    shader clock, summed by rocprofv3 over the 8 XCDs) over the dispatch's
    duration gives the clock the kernel ran at; SQ_VALU_MFMA_BUSY_CYCLES
    (summed over the 1024 SIMDs) over those cycles gives the fraction of
    time the matrix cores were busy, and MOPS x 512 over the duration the
    achieved TFLOP/s; the clocked peak is the dense peak scaled by the clock
    over 2.4 GHz."""
    print(f"{'calls':>6} {'avg us':>9} {'clock GHz':>9} {'MFMA busy':>9} {'TFLOP/s':>8} "
          f"{'of peak':>7} {'of clocked':>10}  kernel")
    for kernel, ds in sorted(groups.items(), key=lambda kv: -sum(d["_ns"] for d in kv[1])):
        ns = sum(d["_ns"] for d in ds) / len(ds)
        grbm = sum(d.get("GRBM_GUI_ACTIVE", 0.0) for d in ds) / len(ds) / XCDS
        busy = sum(d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) for d in ds) / len(ds)
        f8 = sum(d.get("SQ_INSTS_VALU_MFMA_MOPS_F8", 0.0) for d in ds) / len(ds)
        b16 = sum(d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) + d.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0)
                  for d in ds) / len(ds)
        clock = grbm / ns if ns else 0.0
        mfma = busy / (grbm * SIMDS) if grbm else 0.0
        tflops = (f8 + b16) * 512 / (ns * 1e-9) / 1e12 if ns else 0.0
        peak = PEAK_FP8 if f8 >= b16 else PEAK_BF16
        frac = tflops * 1e12 / peak
        clocked = frac * PEAK_CLOCK_GHZ / clock if clock else 0.0
        print(f"{len(ds):6d} {ns / 1e3:9.2f} {clock:9.3f} {mfma:9.1%} {tflops:8.1f} {frac:7.1%} "
              f"{clocked:10.1%}  {kernel}")


def load_traffic():
    """HBM bytes per FP8 GEMM launch (FETCH + WRITE, copy-calibrated) from the
    committed counter summary, or None when it is absent."""
    if not TRAFFIC_FILE.exists():
        return None
    vals = {}
    for line in TRAFFIC_FILE.read_text().splitlines():
        if "_bytes_per_gemm_launch =" in line:
            key, val = line.split("=")
            vals[key.strip()] = float(val)
    fetch = vals.get("FETCH_SIZE_bytes_per_gemm_launch")
    write = vals.get("WRITE_SIZE_bytes_per_gemm_launch")
    if fetch is None or write is None:
        return None
    return dict(fetch=fetch, write=write, total=fetch + write)


def copy_calibration(mib: int) -> None:
    """One plain copy of mib MiB (qx_embed over identity ids: every row read
    once, written once), for counter calibration."""
    import torch

    from quail_amd import _lib
    rows = mib * 2**20 // (2 * COPY_ROW_ELEMS)
    src = torch.empty((rows, COPY_ROW_ELEMS), dtype=torch.bfloat16, device="cuda")
    src.fill_(1.0)
    dst = torch.empty_like(src)
    ids = torch.arange(rows, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()

    def copy():
        _lib.call("qx_embed", src.data_ptr(), COPY_ROW_ELEMS, ids.data_ptr(), dst.data_ptr(),
                  COPY_ROW_ELEMS, rows, COPY_ROW_ELEMS, torch.cuda.current_stream().cuda_stream)
    copy()
    torch.cuda.synchronize()
    log(f"calibration copy: {rows} rows x {2 * COPY_ROW_ELEMS} B = {mib} MiB")
    # the same copy timed: the practical bandwidth of a read + write stream
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(5):
        copy()
    end.record()
    torch.cuda.synchronize()
    seconds = start.elapsed_time(end) * 1e-3 / 5
    log(f"copy bandwidth: {2 * mib * 2**20 / seconds / 1e12:.2f} TB/s (read + write)")
    del src, dst, ids


def main():
    args = parse()
    if args.summarize:
        summarize(args.summarize, args.copy_mib)
        return
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
    from quail_amd.readout import AnswerRows, AsyncAnswers, AsyncLabelLogprobs, AsyncScores
    from quail_amd.workload import make_workload

    assert torch.cuda.is_available(), "bench needs a GPU"
    wl = make_workload(args.workload, seed=args.seed)
    cfg = CONFIGS[wl.model]
    t_build = time.perf_counter()
    model = build_synthetic(cfg, seed=args.seed, device="cuda")
    if wl.function != "classify":
        retain_answer_head(model, wl.label_ids[:2])
    num_pages = 3 * wl.chunk_budget // wl.page_tokens + 64
    v_dtype = torch.bfloat16 if args.v_dtype == "bf16" else torch.float16
    arena = KVArena(cfg.layers, num_pages, wl.page_tokens, cfg.kv_heads, cfg.head_dim,
                    v_dtype=v_dtype)
    pipe = Qwen3Pipeline(model, arena)
    # the stage's AI function: AI.IF bits, AI.SCORE values, or the
    # AI.CLASSIFY label logits at each document's last row
    if wl.function == "classify":
        readout = AsyncLabelLogprobs(model.lm_head.weight, list(wl.label_ids), normalize=False)
    else:
        rows = AnswerRows(model, [wl.label_ids[0]], [wl.label_ids[1]])
        readout = (AsyncScores if wl.function == "score" else AsyncAnswers)(rows)
    prefixes, suffixes = wl.groups_input()
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t_build

    def step(record=None):
        run = StageRun(pipe, arena, readout, prefixes, suffixes, wl.chunk_budget,
                       attention_mode=args.attention)
        if record is not None:
            orig = pipe.forward_chunk

            def forward(chunk):
                calls = ([chunk.host["unified"]] if chunk.attention_mode == "unified" else
                         [t for t in (chunk.host["segments"], chunk.host["reads"]) if t])
                for u in calls:
                    record.append(([int(x) for x in u["cu_q"]], [int(x) for x in u["used"]],
                                   bool(u.get("causal", True))))
                return orig(chunk)
            pipe.forward_chunk = forward
        try:
            answers = run.run()
        finally:
            pipe.forward_chunk = Qwen3Pipeline.forward_chunk.__get__(pipe)
        return answers, run.stats

    log(f"setup {t_build:.1f} s: {wl.documents} documents, {cfg.layers} layers, "
        f"{num_pages} KV pages")
    if args.copy_mib:
        copy_calibration(args.copy_mib)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log("warmup done")

    packs = []
    timer = []
    pipe.engine.gemm_timer = timer
    pipe.engine.gemm_timer_every = max(1, args.gemm_sample)
    pipe.engine.gemm_launches = 0
    stats = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        answers, st = step(record=packs if i == 0 else None)
        stats.append(st)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    pipe.engine.gemm_timer = None
    host = {k: sum(st.get(k, 0.0) for st in stats) / len(stats) * 1e3
            for k in ("admission_s", "pack_s")}
    log("host work per step (overlapped with the GPU after the first pack): " +
        ", ".join(f"{k[:-2]} {v:.1f} ms" for k, v in host.items()))

    gemm_ms = 0.0
    gemm_flops = 0.0
    per_shape = {}
    for m, n, k, start, end, swiglu in timer:
        ms = start.elapsed_time(end)
        gemm_ms += ms
        gemm_flops += 2.0 * m * n * k
        s = per_shape.setdefault(f"{k}x{n}" + ("+swiglu" if swiglu else ""), [0.0, 0.0, 0])
        s[0] += 2.0 * m * n * k
        s[1] += ms
        s[2] += 1
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12
    launches = len(timer)
    all_launches = pipe.engine.gemm_launches
    # operands read once and the result written once: A (M x K e4m3), W (N x K
    # e4m3) and both scale arrays in; C (M x N bf16) out, or with the SwiGLU
    # epilogue M x N/2 e4m3 and its M x N/256 scales
    gemm_bytes = sum(m * k + n * k + 4 * (m * k // 128 + n * k // 16384) +
                     (m * n // 2 + 4 * (m * n // 256) if swiglu else 2 * m * n)
                     for m, n, k, _, _, swiglu in timer)
    # the counter runs behind TRAFFIC_FILE are of the Qwen3-4B workload
    traffic = load_traffic() if args.workload == WORKLOAD else None

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
    e2e_model = t_roof / (elapsed / args.steps)
    # the same over the work the engine issues (the last layer past its KV
    # on final rows only): one final row per question asked
    finals = sum(len(s) for s in suffixes)
    final_pairs = sum(len(p) + len(q) for p, sufs in zip(prefixes, suffixes) for q in sufs)
    i_gemm, i_attn, i_stream = issued_work(cfg, fresh, finals, final_pairs, pairs)
    t_issued = i_gemm / PEAK_FP8 + i_attn / PEAK_BF16 + i_stream / PEAK_HBM
    e2e_frac = t_issued / (elapsed / args.steps)

    log(f"timed {args.steps} steps: {elapsed:.3f} s")
    alone = None
    if args.gemm_alone_reps > 0:
        alone = gemm_alone(args.gemm_alone_reps, args.seed)
        log(f"gemm alone: {alone['shapes']}")
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(model, wl, args.cpu_seconds)
        log(f"cpu baseline: {cpu['sample']}")

    line = {
        "metric": METRIC if args.workload == WORKLOAD else
        f"AI.{wl.function.upper()} rows/sec + prefill tok/s, {model_name(cfg)} FP8, 1 MI355X; "
        f"% FP8 MFMA peak",
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
        "data": f"synthetic (seeded random-init {model_name(cfg)} weights, uniform token ids)",
        "config": {
            "workload": describe(wl, cfg, args.attention),
            "documents": docs, "fresh_tokens": fresh, "packs": stats[0]["chunks"],
            "borrowed_tokens": stats[0]["borrowed_tokens"], "attention_pairs": pairs,
            "parallelism": "none (1 GPU)", "v_pages": args.v_dtype,
        },
        "prefill_tok_s": round(tok_s, 1),
        "e2e_roofline_frac": round(e2e_frac, 4),
        "e2e_roofline_basis": "issued work: the last layer's attention, o_proj and MLP on "
                              "final rows only, as the engine runs it",
        "e2e_roofline_frac_model_work": round(e2e_model, 4),
        "roofline": {
            "bound": "mfma",
            "kernel": f"FP8 block-scaled GEMM, all four {model_name(cfg)} projections: "
                      "qx_gemm_fp8_blockscaled (qkv, o_proj, down) and "
                      "qx_gemm_fp8_swiglu_quant (gate_up with the SiLU-quant epilogue)",
            "achieved": round(gemm_tflops, 2),
            "peak": PEAK_FP8 / 1e12,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops * 1e12 / PEAK_FP8, 4),
            "traffic": traffic and round(traffic["total"]),
            "traffic_source": traffic and str(TRAFFIC_FILE.relative_to(ROOT)),
            "algorithmic_bytes_per_launch": round(gemm_bytes / max(launches, 1)),
            "launches": all_launches,
            "timed_launches": launches,
            "avg_launch_us": round(gemm_ms * 1e3 / max(launches, 1), 2),
            "gemm_time_share": round(gemm_ms / max(launches, 1) * all_launches * 1e-3 / elapsed,
                                     4),
            "per_shape_tflops": {s: round(v[0] / (v[1] * 1e-3) / 1e12, 1)
                                 for s, v in per_shape.items()},
        },
        "gemm_alone": alone,
        "cpu_baseline": cpu,
        "setup_s": round(t_build, 1),
    }
    print(json.dumps(line, default=lambda o: o.item() if hasattr(o, "item") else str(o)))


if __name__ == "__main__":
    main()
