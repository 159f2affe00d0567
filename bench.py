"""Benchmark of the DenseGPA core on one MI355X (backend="hip").

Workload (one step): forward + backward of a Qwen3-0.6B-shaped GPA attention
layer, B=1, T=8192, heads=16, key_dim=value_dim=128, slots=(128,128,128,256),
chunk_size=64; q,k,v ~ N(0,1) in bf16 with K L2-normalised per head; fp32
master parameters; loss = mean(out.float()^2).  Inputs are resident in HBM
before the timed region.

    python bench.py [--gpus 1] [--steps 5] [--warmup 2] [--no-cpu] [--no-decode] [--no-lm]

Prints ONE JSON line.  `value` is tokens/s of the whole job over the timed
steps (independent scans overlap on side streams).  `roofline` is the dominant
kernel's achieved rate against the bf16 MFMA peak: algorithmic FLOP per launch
/ average launch time, timed with HIP events on the launch stream during one
extra step in which the schedule runs on one stream (no kernel overlaps
another, so the interval is the kernel's own run time and agrees with a rocprof
kernel trace of that step).  `step_roofline` is the whole step's algorithmic
FLOP over the timed step time; `decode` is the batched one-token decode rate (B=64 streams of the same layer, 2048-token
prefill, 256 graph-replayed steps) with its HBM roofline from the state bytes a
token step must move; `lm` is the all-GPA Qwen3-0.6B-architecture LM (a T=8192
training step with AdamW, a 4096-token prefill and 512 graphed greedy tokens);
`cpu_baseline` times the CPU oracle (the reference's per-token torch algorithm)
on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "GPA attn fwd+bwd tokens/s @T=8192 bf16; decode tok/s; % of roofline"
SHAPE = dict(heads=16, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=64)
BATCH, TOKENS = 1, 8192


def f_scan(k: int, v: int, c: int) -> float:
    """Algorithmic FLOP per token of one chunked GDN scan forward: inter-chunk
    Q S, W S, S += K^T V' (6KV) plus intra-chunk QK^T, KK^T, W, U, P V'
    (2C(3K+2V)) and the triangular solve (C^2/3)."""
    return 6 * k * v + 2 * c * (3 * k + 2 * v) + c * c / 3


def f_forward_per_token_head(dk: int, dv: int, slots, c: int) -> float:
    """Inner + outer + relation scans + level/route glue per token per head."""
    total = 0.0
    for m in slots:
        total += f_scan(dk, m, c) + f_scan(m, dv, c)
        total += 8 * dk * m + 2 * m * dv + 10 * m * m + 8 * dk
    for i, mi in enumerate(slots):
        for j, mj in enumerate(slots):
            if i != j:
                total += f_scan(mi, mj, c)
    return total


DECODE_BATCH = 64


def decode_state_bytes(dk: int, dv: int, slots) -> int:
    """HBM bytes one stream (b, h) must move per decoded token: every fp32
    state read and written once (A_j [Dk,M_j] and B_j [M_j,Dv], R_ij [M_i,M_j],
    counts [M_j]) and the block-start snapshots of A_j, B_j read once."""
    s = sum(slots)
    rel = sum(mi * mj for i, mi in enumerate(slots) for j, mj in enumerate(slots) if i != j)
    return 4 * (3 * (dk * s + s * dv) + 2 * rel + 2 * s)


def decode_rate(model, steps: int = 256, warmup: int = 64, prefill: int = 2048) -> dict:
    """Batched one-token decode through the model's cache (chunk mode, T=1 per
    call), B=64 streams of the same layer, bf16, under no_grad, on the path
    that serves it: the schedule's T=1 segments (one-token steps that read
    and write each state once), replayed from one HIP graph per block
    position (`DecodeGraph`).  The cache is first prefilled over `prefill`
    tokens of N(0,1) q, k (k normalised), v, in 512-token calls (chunk mode
    carries the cache exactly across calls that end on block boundaries);
    after one untimed cycle of replays (`warmup`) the timed steps span whole
    blocks, so the once-per-block state copy of the graph cycle is included.
    The eager rate of 64 steps from the same cache is reported beside it."""
    import torch

    from gpa_amd import DecodeGraph, params
    cfg = model.config
    dev = next(model.parameters()).device
    h, dk, dv = cfg.heads, cfg.key_dim, cfg.value_dim
    gen = torch.Generator(device=dev).manual_seed(1)

    def tokens(t):
        q = torch.randn(DECODE_BATCH, t, h, dk, device=dev, generator=gen).bfloat16()
        k = torch.nn.functional.normalize(torch.randn(DECODE_BATCH, t, h, dk, device=dev, generator=gen), dim=-1)
        v = torch.randn(DECODE_BATCH, t, h, dv, device=dev, generator=gen).bfloat16()
        return q, k.bfloat16(), v

    _progress(f"decode: {prefill}-token prefill at B={DECODE_BATCH}")
    # Inference leaves the parameters unchanged, so parameter-derived tensors
    # (packed weight layouts, gate constants) are computed once (params.frozen).
    with torch.no_grad(), params.frozen():
        state = model.initial_state(DECODE_BATCH, device=dev, dtype=torch.bfloat16)
        for _ in range(prefill // 512):
            _, state = model(*tokens(512), state)
        torch.cuda.synchronize()
        toks = [tokens(1) for _ in range(warmup + steps)]

        def timed(run, n_warm, n_timed):
            for i in range(n_warm):
                run(toks[i])
            torch.cuda.synchronize()
            start = time.perf_counter()
            for i in range(n_warm, n_warm + n_timed):
                run(toks[i])
            torch.cuda.synchronize()
            return (time.perf_counter() - start) / n_timed

        box = [state]

        def eager(x):
            _, box[0] = model(*x, box[0])
        _progress("decode: eager token steps")
        eager_s = timed(eager, 8, 64)
        del box
        _progress("decode: graph capture and replays")
        graphed = DecodeGraph(model, state, *toks[0])
        seconds = timed(lambda x: graphed.step(*x), warmup, steps)
        del graphed
    moved = decode_state_bytes(dk, dv, cfg.slots) * DECODE_BATCH * h
    gbs = moved / seconds / 1e9
    return {"value": DECODE_BATCH / seconds, "unit": "tokens/s", "batch": DECODE_BATCH,
            "ms_per_token_step": seconds * 1e3, "eager_ms_per_token_step": eager_s * 1e3,
            "prefill_tokens": prefill, "warmup_steps": warmup, "steps": steps,
            "path": "schedule T=1 segments (one-token scan steps gdn_token_step, register-resident block-snapshot "
                    "level kernel, each 128-slot level's inner step and level write in one launch, one-launch "
                    "gate/logit/mix glue, cached parameter layouts) replayed from one HIP graph per block position; "
                    "the fused one-kernel step is switched off",
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "state_bytes_per_token_step": moved}}


LM_SLOTS = (128, 128, 128, 256)


def lm_native_flop_per_token(cfg) -> float:
    """Forward FLOP per token of the LM's native (non-GPA) products: the q, k,
    v, o projections and the SwiGLU MLP of every layer, and the LM head."""
    hid, inter, heads, kv, d = (cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads,
                                cfg.num_key_value_heads, cfg.head_dim)
    per_layer = 2 * hid * (heads * d + 2 * kv * d) + 2 * heads * d * hid + 2 * 3 * hid * inter
    return cfg.num_hidden_layers * per_layer + 2 * hid * cfg.vocab_size


def lm_rate(train_steps: int = 2, prefill: int = 4096, decode_tokens: int = 512) -> dict:
    """The Qwen3-0.6B-architecture all-GPA LM (28 layers, hidden 1024, 16 query
    / 8 KV heads of width 128, SwiGLU 3072, vocab 151936, tied embeddings; GPA
    slots (128,128,128,256) with the LM wrapper's flag set), random init, fp32
    master weights under bf16 autocast: a B=1, T=8192 training step (forward,
    per-layer checkpointed backward, AdamW) on uniform random token ids; then
    a `prefill`-token prefill and `decode_tokens` greedy tokens, the decode
    replayed from one HIP graph per block position (LMDecodeGraph, greedy
    choice inside the graph)."""
    import torch

    from gpa_amd import params
    from gpa_amd.lm import GPALMConfig, GPALMForCausalLM, LMDecodeGraph
    dev = torch.device("cuda:0")
    torch.cuda.set_per_process_memory_fraction(0.85)
    torch.manual_seed(0)
    cfg = GPALMConfig(gpa=dict(slots=LM_SLOTS))
    model = GPALMForCausalLM(cfg).to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)
    model.gradient_checkpointing_enable()
    model.train()
    gen = torch.Generator(device=dev).manual_seed(2)
    ids = torch.randint(0, cfg.vocab_size, (1, TOKENS), device=dev, generator=gen)

    def train_step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(ids, labels=ids).loss
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
        return loss

    _progress("LM: training step warm-up and timed steps")
    train_step()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(train_steps):
        loss = train_step()
    torch.cuda.synchronize()
    train_s = (time.perf_counter() - start) / train_steps
    peak_gb = torch.cuda.max_memory_allocated() / 2 ** 30
    del opt
    model.eval()
    prompt = torch.randint(0, cfg.vocab_size, (1, prefill), device=dev, generator=gen)
    _progress("LM: prefill and graphed greedy decode")
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16), params.frozen():
        model(prompt[:, :64], logits_to_keep=1)
        torch.cuda.synchronize()
        start = time.perf_counter()
        out = model(prompt, logits_to_keep=1)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - start
        first = out.logits[:, -1].argmax(-1, keepdim=True)
        graph = LMDecodeGraph(model, out.past_key_values, first)
        del out
        for _ in range(graph.chunk):  # one untimed block of replays
            graph.step()
        torch.cuda.synchronize()
        start = time.perf_counter()
        graph.generate(decode_tokens + 1)  # feeds decode_tokens tokens: whole blocks
        torch.cuda.synchronize()
        decode_s = (time.perf_counter() - start) / decode_tokens
        del graph
    torch.cuda.set_per_process_memory_fraction(1.0)
    gpa_flop = f_forward_per_token_head(cfg.head_dim, cfg.head_dim, LM_SLOTS, 64) * cfg.num_attention_heads
    flop_step = 3 * (cfg.num_hidden_layers * gpa_flop + lm_native_flop_per_token(cfg)) * TOKENS
    tf = flop_step / train_s / 1e12
    return {"workload": "Qwen3-0.6B-architecture all-GPA LM (28 layers, hidden 1024, heads 16/8, head_dim 128, "
                        "MLP 3072, vocab 151936), GPA slots (128,128,128,256), random init, bf16 autocast",
            "train": {"value": TOKENS / train_s, "unit": "tokens/s", "ms_per_step": train_s * 1e3,
                      "batch": 1, "seq_len": TOKENS, "loss": loss.item(), "peak_gib": peak_gb,
                      "optimizer": "AdamW (fused)", "checkpointing": "per layer",
                      "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                   "frac": tf / PEAK_BF16_TFLOPS, "flop_per_step": flop_step,
                                   "note": "algorithmic FLOP (no recompute) of the GPA layers and native products"}},
            "prefill": {"value": prefill / prefill_s, "unit": "tokens/s", "tokens": prefill,
                        "ms": prefill_s * 1e3},
            "decode": {"value": 1 / decode_s, "unit": "tokens/s", "ms_per_token": decode_s * 1e3,
                       "tokens": decode_tokens, "batch": 1,
                       "path": "LMDecodeGraph: one HIP graph per block position, greedy choice in the graph"}}


def _progress(what: str) -> None:
    print(f"bench: {what}", file=sys.stderr, flush=True)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


C1 = dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), positional_mode="gated", chunk_size=1)
C2 = dict(heads=4, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=64)


def cpu_baseline() -> dict:
    """The oracle (per-token reference algorithm, fp32) timed on this host with
    the reference benchmark's protocol (scripts/benchmark.py:44-54: warm-ups,
    then timed runs with perf_counter), per workload:
      * the training workload's layer (B=1, H=16, Dk=Dv=128, slots
        (128,128,128,256), C=64): fwd+bwd, 2 warm-ups then 3 timed runs each at
        T=128 and T=256 (`value` = T=256; full T=8192 autograd would hold
        ~240 GB of per-token states), and forward only (no_grad) at T=1024,
        1 warm-up then 2 timed runs;
      * config 1 in full (tokenwise, B=2, T=16, H=4, Dk=32, Dv=48, slots
        (64,64,64,128)): fwd+bwd of out.square().mean() and a one-token
        continuation, 2 warm-ups then 3 timed runs;
      * config 2 (the same widths, C=64, B=8): fwd+bwd at T=128, one 16-token
        warm-up then 2 timed runs (the full T=1024 takes about a minute a run
        on 16 cores; the per-token cost does not depend on T, which the two
        lengths of the training layer check);
      * batched decode of the training layer at B=64 after a one-block
        (64-token) prefill, 8 timed one-token steps (the step cost does not
        depend on the prefill length: the cache is fixed-size)."""
    import torch

    import oracle
    from gpa_amd import DenseGPA, GPAConfig
    cores = len(os.sched_getaffinity(0))
    old = torch.get_num_threads()
    torch.set_num_threads(cores)

    def inputs(shape, b, t, normalize=True):
        q = torch.randn(b, t, shape["heads"], shape["key_dim"])
        k = torch.randn_like(q)
        if normalize:
            k = torch.nn.functional.normalize(k, dim=-1)
        return q, k, torch.randn(b, t, shape["heads"], shape["value_dim"])

    def train_rate(run, model, shape, b, t, warm_t, warmups, reps, normalize=True):
        def once(tt):
            xs = [x.requires_grad_() for x in inputs(shape, b, tt, normalize)]
            model.zero_grad(set_to_none=True)
            start = time.perf_counter()
            out, state = run(*xs)
            out.float().square().mean().backward()
            return time.perf_counter() - start, state
        for _ in range(warmups):
            once(warm_t)
        secs = [once(t)[0] for _ in range(reps)]
        return b * t * len(secs) / sum(secs)

    try:
        torch.manual_seed(0)
        model = DenseGPA(GPAConfig(**SHAPE))
        run = oracle.OracleRun(model)
        rates = {t: train_rate(run, model, SHAPE, BATCH, t, 32, 2, 3) for t in (128, 256)}
        with torch.no_grad():
            run(*inputs(SHAPE, BATCH, 32))
            secs = []
            for _ in range(2):
                xs = inputs(SHAPE, BATCH, 1024)
                start = time.perf_counter()
                run(*xs)
                secs.append(time.perf_counter() - start)
            fwd_rate = BATCH * 1024 * len(secs) / sum(secs)
            _, state = run(*inputs(SHAPE, DECODE_BATCH, 64))
            toks = [inputs(SHAPE, DECODE_BATCH, 1) for _ in range(10)]
            for x in toks[:2]:
                _, state = run(*x, state)
            start = time.perf_counter()
            for x in toks[2:]:
                _, state = run(*x, state)
            step_s = (time.perf_counter() - start) / (len(toks) - 2)
        # config 1: tokenwise, fwd+bwd, then a one-token continuation from the returned state
        torch.manual_seed(0)
        m1 = DenseGPA(GPAConfig(**C1))
        r1 = oracle.OracleRun(m1)
        c1_rate = train_rate(r1, m1, C1, 2, 16, 16, 2, 3, normalize=False)
        with torch.no_grad():
            _, s1 = r1(*inputs(C1, 2, 16, False))
            start = time.perf_counter()
            r1(*inputs(C1, 2, 1, False), s1)
            c1_cont_ms = (time.perf_counter() - start) * 1e3
        # config 2 in full
        torch.manual_seed(0)
        m2 = DenseGPA(GPAConfig(**C2))
        c2_rate = train_rate(oracle.OracleRun(m2), m2, C2, 8, 128, 16, 1, 2, normalize=False)
    finally:
        torch.set_num_threads(old)
    return {"value": rates[256], "unit": "tokens/s", "cores": cores, "kind": "port",
            "tokens_per_s_T128": rates[128], "tokens_per_s_T256": rates[256],
            "forward_T1024": {"value": fwd_rate, "unit": "tokens/s"},
            "decode": {"value": DECODE_BATCH / step_s, "unit": "tokens/s", "ms_per_token_step": step_s * 1e3,
                       "batch": DECODE_BATCH},
            "config1": {"value": c1_rate, "unit": "tokens/s", "continuation_ms": c1_cont_ms,
                        "workload": "B=2 T=16 H=4 Dk=32 Dv=48 slots (64,64,64,128) C=1, fwd+bwd"},
            "config2": {"value": c2_rate, "unit": "tokens/s",
                        "workload": "B=8 H=4 Dk=32 Dv=48 slots (64,64,64,128) C=64, fwd+bwd, timed at T=128"},
            "sample": f"oracle, fp32, on {_cpu_model()} with {cores} threads: the training layer (B=1) fwd+bwd with "
                      f"2 warm-ups (T=32) and 3 timed runs at T=128 and at T=256 (value = T=256), forward only at "
                      f"T=1024 (2 timed runs); config 1 in full (3 timed fwd+bwd runs and a one-token "
                      f"continuation); config 2 at B=8, T=128 (2 timed fwd+bwd runs); decode B=64 after a 64-token "
                      f"prefill, 8 timed steps"}


def _measured_traffic(kernel: str) -> float | None:
    """HBM bytes per launch of `kernel` from the committed PMC summary
    (FETCH_SIZE x its copy-calibrated factor + WRITE_SIZE, KiB per dispatch),
    or None when the summary has no row for it."""
    path = os.path.join(ROOT, "profiles", "dense_gpa_layer_T8192_pmc_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 6 and cells[0].strip("`") == kernel:
                    return (float(cells[4].replace(",", "")) + float(cells[5].replace(",", ""))) * 1e6
    except OSError:
        pass
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-decode", action="store_true", help="skip the batched decode measurement")
    ap.add_argument("--no-lm", action="store_true", help="skip the all-GPA LM (config 5) measurement")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build", file=sys.stderr)
        return 2

    import torch

    from gpa_amd import DenseGPA, GPAConfig, profiling, schedule

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = DenseGPA(GPAConfig(**SHAPE)).to(dev)
    h, dk, dv = SHAPE["heads"], SHAPE["key_dim"], SHAPE["value_dim"]
    q = torch.randn(BATCH, TOKENS, h, dk, device=dev).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(BATCH, TOKENS, h, dk, device=dev), dim=-1).bfloat16()
    v = torch.randn(BATCH, TOKENS, h, dv, device=dev).bfloat16()
    xs = [x.requires_grad_() for x in (q, k, v)]

    def step():
        model.zero_grad(set_to_none=True)
        for x in xs:
            x.grad = None
        out, _ = model(*xs)
        out.float().square().mean().backward()

    _progress("training step: warm-up and timed steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    time.sleep(0.3)  # an idle gap that marks the timed steps in a kernel trace
    start = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    ms = elapsed / args.steps * 1e3
    tokens_per_s = BATCH * TOKENS * args.steps / elapsed

    # Kernel roofline: one more step with the schedule on one stream, so that
    # each kernel's HIP-event interval is its own run time (with side streams a
    # big-grid kernel also waits for CUs held by its neighbours).  The idle gap
    # before it marks the step in a rocprof kernel trace
    # (`python -m gpa_amd.profiling trace <kernel_trace.csv>` summarises it).
    _progress("training step: one-stream step with kernel timers")
    time.sleep(0.3)
    with schedule.one_stream(), profiling.kernel_timer() as timer:
        serial_start = time.perf_counter()
        step()
        torch.cuda.synchronize()
        serial_ms = (time.perf_counter() - serial_start) * 1e3

    flop_step = 3 * f_forward_per_token_head(dk, dv, SHAPE["slots"], SHAPE["chunk_size"]) * BATCH * TOKENS * h
    step_tflops = flop_step / (ms * 1e-3) / 1e12
    dominant = timer.dominant()
    roofline = None
    if dominant is not None:
        chain = "_state_" in dominant["name"]
        roofline = {"bound": "mfma", "kernel": dominant["name"], "achieved": dominant["tflops"],
                    "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": dominant["tflops"] / PEAK_BF16_TFLOPS,
                    "traffic": _measured_traffic(dominant["name"]),
                    "limited_by": ("latency of the sequential chunk chain (one state step per 64 tokens)"
                                   if chain else "issue latency at one workgroup per CU"),
                    "avg_launch_us": dominant["avg_us"], "launches": dominant["launches"],
                    "share_of_step": dominant["total_ms"] / serial_ms,
                    "timed_in": f"one extra step on one stream ({serial_ms:.1f} ms)"}
    # The sequential state recurrences: every state launch of the step together
    # (packed launches advance several scan groups at once), algorithmic FLOP
    # over their summed launch time.
    state_rows = [r for r in timer.table() if "_state_" in r["name"]]
    state_roofline = None
    if state_rows:
        st_ms = sum(r["total_ms"] for r in state_rows)
        st_flop = sum(r["tflops"] * r["total_ms"] * 1e-3 * 1e12 for r in state_rows)
        st_tf = st_flop / (st_ms * 1e-3) / 1e12
        state_roofline = {"bound": "latency", "achieved": st_tf, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                          "frac": st_tf / PEAK_BF16_TFLOPS, "launches": sum(r["launches"] for r in state_rows),
                          "total_ms": st_ms, "share_of_step": st_ms / serial_ms,
                          "limited_by": "one dependent chunk step after another (128 per launch at T=8192)"}
    kernels = [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()} for r in timer.table()[:12]]
    result = {
        "metric": METRIC, "value": tokens_per_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic N(0,1) q,k,v; random-init fp32 params",
        "config": {"workload": "DenseGPA layer fwd+bwd, B=1 T=8192 H=16 Dk=Dv=128 slots=(128,128,128,256) "
                               "C=64, bf16 activations", "global_batch": BATCH, "seq_len": TOKENS,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "state_roofline": state_roofline,
        "kernels_one_stream_step": kernels,
        "step_roofline": {"bound": "mfma", "achieved": step_tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                          "frac": step_tflops / PEAK_BF16_TFLOPS, "flop_per_step": flop_step},
    }
    if not args.no_decode:
        result["decode"] = decode_rate(model)
    if not args.no_lm:
        del model, xs, q, k, v
        torch.cuda.empty_cache()
        result["lm"] = lm_rate()
    if not args.no_cpu:
        _progress("CPU baseline")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
