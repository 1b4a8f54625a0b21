#!/usr/bin/env python3
"""Decode throughput of the batched SwarmLoRA step on one MI355X.

Workload: a 32-layer Llama-3.1-8B-shaped decode step for
28 workers, one token each, every worker with its own rank-16 LoRA adapter on
all seven projections (scale 2.0), a paged bf16 KV cache per worker (page 16,
8 kv heads of 128) holding U{128..2048} tokens of ~N(0,1) context, RMSNorm
weights 1, RoPE theta 500000, embedding / LM head / projections ~N(0,0.02),
greedy sampling.  One step = embed + 32 x (QKV, O, Gate+Up, Down rounds with
attention and the worker-side elementwise work) + LM head = 130 rounds, one
token per worker.  Synthetic random-init weights (seeded), no checkpoint.

`value` is tokens/s over the timed replays of the captured step (inputs and
weights resident in HBM).  `roofline` is the decode projection's base
kernel (split_kernel, the 128 projection rounds of a step; the LM head is a
whole-K round of its own): algorithmic bytes per launch over its mean
duration, both from HIP events recorded around each launch on its stream
during eager steps of the same workload (HIP events inside a replayed graph
carry no timestamps on ROCm).  `cpu_baseline` times
the CPU oracle's decode_step (torch-CPU bf16, the reference's op order) on a
bounded sample: the LM head and one layer, scaled to 32 layers, on every
core the process may use (CPU model and bf16-relevant flags reported).

`config.per_config` holds BASELINE configs 1, 2, 3 and 5 measured after the
headline: µs per round (config 1) or per layer of four rounds (configs 2, 3,
5) from HIP-graph replays (config 3: HIP events around eager rounds), the
algorithmic bytes (FLOPs for config 3), the achieved rate, its fraction of
the roofline and the floor; configs 1 and 2 also on the host's CPU cores.

`config.drop_in` is the drop-in (multi-process) path: a spawned aggregator
process and --ipc-workers worker processes over the shared-memory ring and
IPC slot buffers, 32 layers (130 rounds per token), in three modes by
default: the reference's host-synchronised protocol with the worker-side
LoRA, the same with the worker's input copies ordered on the GPU, and
host-synchronised with adapters pooled in the aggregator's rounds
(--ipc-modes adds the others).  The modes run in turn, twice (a run's level varies more between
runs than within one); per mode tokens/s and µs per round of the median of
its 6 windows (3 per run, timed once every slot is active), each pass's
median, and the mean [LAYER_PROFILE] stage split (gather / round wait /
scatter / LoRA / norms and attention) of stage-synchronised tokens.
"""

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
# Published decode throughput of the reference at 28 adapter workers, 8B
# model (one NVIDIA L40S, real Llama-3.1-8B-Instruct weights): README.md:69-70
# of the reference repository.
REFERENCE_TOK_S = 314.0
# HBM bytes per launch of the decode projection's base kernel, measured with
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on this workload and scaled by a
# copy kernel of known size (the summary file gives the commands and factors)
PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
TRAFFIC_FILE = os.path.join(PROFILES, "split_kernel_decode_config4_pmc.md")


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=10, help="untimed decode steps before timing")
    ap.add_argument("--workers", type=int, default=28)
    ap.add_argument("--timer-steps", type=int, default=3, help="eager steps with per-launch HIP events")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after timing, copy a buffer of this many MiB (a kernel of known HBM traffic for "
                         "calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--weights", choices=("packed", "row-major"), default="packed",
                    help="decode: projection weights in fragment tiles (default) or row-major")
    ap.add_argument("--whole-k", choices=("lm", "none"), default="lm",
                    help="decode: the LM head as a whole-K round (one launch, no K-slice partials; default) or "
                         "K-sliced like the projection rounds")
    ap.add_argument("--workload", choices=("decode", "prefill", "ipc", "configs"), default="decode",
                    help="decode: BASELINE config 4 (the headline line); prefill: config 3's ragged one-layer "
                         "rounds on the MFMA path; ipc: the multi-process serving path (worker processes, "
                         "shared-memory ring, IPC slots) in the modes of --ipc-modes; configs: the per-config "
                         "figures of configs 1, 2, 3 and 5. The last three print lines of their own")
    ap.add_argument("--ipc-workers", type=int, default=8,
                    help="drop-in leg of the decode line: worker processes (at most 8; with the aggregator's "
                         "process and this one at most 10 processes use the GPU)")
    ap.add_argument("--no-ipc", action="store_true", help="decode: skip the drop-in (multi-process) leg")
    ap.add_argument("--no-per-config", action="store_true",
                    help="decode: skip the per-config figures (BASELINE configs 1, 2, 3 and 5)")
    ap.add_argument("--ipc-layers", type=int, default=32, help="drop-in leg: 8B-shaped layers")
    ap.add_argument("--ipc-tokens", type=int, default=6, help="drop-in leg: decode tokens per timed window")
    ap.add_argument("--ipc-reps", type=int, default=3, help="drop-in leg: timed windows per run")
    ap.add_argument("--ipc-passes", type=int, default=2,
                    help="drop-in leg: passes over the modes in turn (the median window of all is reported)")
    ap.add_argument("--ipc-modes", default="host_sync,gpu_ordered_inputs,host_sync_pooled",
                    help="drop-in leg: comma list of " + ", ".join(IPC_MODES) + " (the decode line's default: the "
                         "reference's protocol with the worker's own LoRA, host-synchronised, then with its input "
                         "copies ordered on the GPU, then host-synchronised with adapters pooled in the "
                         "aggregator's rounds; gpu_ordered, which also orders the output reads on the GPU, "
                         "measured level with or slower than host_sync and is left to this flag)")
    return ap.parse_args()


def copy_calibration(args, dev):
    """--copy-calibration MIB: one copy of a buffer of that size (reads and
    writes MIB each), the reference dispatch that scales rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters to bytes."""
    if args.copy_calibration <= 0:
        return
    import torch
    n = args.copy_calibration * (1 << 20) // 2
    src = torch.ones(n, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def read_traffic():
    """hbm_bytes_per_launch of the dominant kernel (split_kernel) from the
    committed counter summary, or None."""
    path = TRAFFIC_FILE
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    return None


def host_cpu_info():
    """CPU model, the x86 flags that matter for bf16 matrix work on the host,
    and the number of cores this process may use: the affinity mask, capped
    by a cgroup-v2 CPU quota when one is set (the job's CPU share)."""
    info = {"model": None, "flags": [], "os_cpu_count": os.cpu_count()}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and info["model"] is None:
                    info["model"] = line.split(":", 1)[1].strip()
                elif line.startswith("flags"):
                    fl = set(line.split(":", 1)[1].split())
                    info["flags"] = sorted(fl & {"avx2", "avx512f", "avx512_bf16", "amx_bf16", "amx_tile",
                                                 "avx512_vnni", "avx_vnni"})
                    break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    info["affinity_cpus"] = usable
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            info["cgroup_cpus"] = int(quota) / int(period)
            usable = max(1, min(usable, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    info["usable_cpus"] = usable
    return info


def cpu_baseline(workers, budget_s):
    """The CPU oracle's batched decode_step (torch-CPU, bf16) at config-4
    shapes on this host's cores (every core the process may use): the LM head
    alone (layers=0) and with one layer, repeated within the budget; per
    step = t0 + 32 * (t1 - t0)."""
    import torch
    from oracle import reference_path as ref
    from swarmlora_amd.decode import DecodeShape
    host = host_cpu_info()
    threads = host["usable_cpus"]
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    s = DecodeShape()
    g = torch.Generator().manual_seed(0)

    def rn(*shape, std=0.02):
        return torch.randn(*shape, generator=g, dtype=torch.bfloat16).mul_(std)

    layer = {p: rn(o, i) for p, (i, o) in s.proj_dims().items()}
    layer["input_norm"] = torch.ones(s.hidden, dtype=torch.bfloat16)
    layer["post_norm"] = torch.ones(s.hidden, dtype=torch.bfloat16)
    weights = {"layers": [layer], "embed": rn(s.vocab, s.hidden), "lm_head": rn(s.vocab, s.hidden),
               "final_norm": torch.ones(s.hidden, dtype=torch.bfloat16)}
    adapters = [{0: {p: (rn(s.rank, i), rn(o, s.rank)) for p, (i, o) in s.proj_dims().items()}}
                for _ in range(workers)]
    ctx = torch.randint(128, 2049, (workers,), generator=torch.Generator().manual_seed(3))
    mb = (2048 + 16 + s.block_size - 1) // s.block_size
    kc = [rn(workers * mb, s.block_size, s.kv_heads, s.head_dim, std=1.0)]
    vc = [rn(workers * mb, s.block_size, s.kv_heads, s.head_dim, std=1.0)]
    bt = torch.arange(workers * mb, dtype=torch.int32).reshape(workers, mb)
    cs = ref.cos_sin_cache(ref.rope_inv_freq(s.head_dim, s.theta), mb * s.block_size)
    ids = torch.randint(0, s.vocab, (workers,), generator=torch.Generator().manual_seed(4))
    seq = ctx.to(torch.int32)
    times = {0: [], 1: []}
    t_start = time.perf_counter()
    while True:
        for L in (0, 1):
            t0 = time.perf_counter()
            ref.decode_step(s, weights, adapters, [kc[0].clone()], [vc[0].clone()], bt, seq, ids, cs, layers=L)
            times[L].append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times[1]) >= 2:
            break
    torch.set_num_threads(prev_threads)
    t0 = statistics.median(times[0])
    t1 = statistics.median(times[1])
    step_s = t0 + s.layers * max(t1 - t0, 0.0)
    return {"value": workers / step_s, "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": host["model"], "cpu_flags": host["flags"], "os_cpu_count": host["os_cpu_count"],
            "affinity_cpus": host["affinity_cpus"], "cgroup_cpus": host.get("cgroup_cpus"),
            "sample": (f"oracle decode_step (torch-CPU bf16) at config-4 shapes, {workers} workers: LM head alone "
                       f"{t0 * 1e3:.0f} ms and with one layer {t1 * 1e3:.0f} ms (medians of {len(times[1])}); "
                       f"step = LM head + 32 x layer = {step_s * 1e3:.0f} ms; includes the per-step page clone; "
                       f"CPU-seeded weights of the same shapes")}


def prefill_measure(steps):
    """one 8B-shaped layer's four rounds (QKV, O,
    Gate+Up, Down) over 16 slots, half of them one token, the rest
    U{32..512} tokens (seeded), each slot with its own adapter of rank drawn
    from {8, 16, 32, 64}; > 64 token rows, so the rounds take the prefill
    path (LoRA shrink, then the 256 x 256 MFMA GEMM reading the slot rows in
    place, the delta as extra MFMA k-steps, rows written to their slots).
    Returns per-round ms and TFLOP/s of the base GEMM flops (2*T*N*K) over
    the measured time of each round (HIP events around `steps` eager calls)."""
    import torch
    from swarmlora_amd import ops
    dev = torch.device("cuda:0")
    H, KV, HD, I = 4096, 8, 128, 14336
    g = torch.Generator().manual_seed(3)
    rows = [1] * 8 + torch.randint(32, 513, (8,), generator=g).tolist()
    ranks = [[8, 16, 32, 64][int(i)] for i in torch.randint(0, 4, (16,), generator=g)]
    T = sum(rows)
    gd = torch.Generator(device=dev).manual_seed(0)

    def rn(*shape, std=0.02):
        return torch.randn(*shape, generator=gd, device=dev, dtype=torch.bfloat16) * std

    rounds = [("qkv", H, [H, KV * HD, KV * HD]), ("o", H, [H]), ("gate_up", H, [I, I]), ("down", I, [H])]
    plan = []
    for nm, k, dims in rounds:
        n = sum(dims)
        table = ops.LoraTable(dev)
        for i, r in enumerate(ranks):
            table.add(rn(r * len(dims), k).contiguous(), [rn(d, r).contiguous() for d in dims], r, 2.0)
        xs = [rn(t, k, std=1.0) for t in rows]
        ys = [torch.empty(t, n, dtype=torch.bfloat16, device=dev) for t in rows]
        plan.append((nm, n, k, dims, rn(n, k), table, xs, ys))

    def run(p):
        nm, n, k, dims, w, table, xs, ys = p
        ops.round_fused(xs, ys, rows, w, None, seg_lora=list(range(len(rows))), table=table, blk_cols=dims)

    for p in plan:
        for _ in range(3):
            run(p)
    torch.cuda.synchronize()
    per = {}
    flops = 0
    tot_ms = 0.0
    for p in plan:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            run(p)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        f = 2.0 * T * p[1] * p[2]
        per[p[0]] = {"ms": round(ms, 4), "TFLOPs": round(f / (ms * 1e-3) / 1e12, 1)}
        flops += f
        tot_ms += ms
    del plan
    torch.cuda.empty_cache()
    return {"T": T, "rows": rows, "ranks": ranks, "rounds": per, "flops": flops, "ms": tot_ms,
            "tflops": round(flops / (tot_ms * 1e-3) / 1e12, 1)}


def prefill(args):
    """--workload prefill: config 3's line on its own; `roofline` is bf16
    MFMA."""
    import torch
    pf = prefill_measure(args.steps)
    copy_calibration(args, torch.device("cuda:0"))
    tflops = pf["tflops"]
    line = {
        "metric": "prefill-shape round TFLOP/s (BASELINE config 3)",
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": 3,
        "ms_per_step": round(pf["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random-init weights, adapters and activations)",
        "config": {"workload": "config3: one 8B-shaped layer's QKV, O, Gate+Up and Down rounds over 16 ragged "
                               "slots (8 x 1 token, 8 x U{32..512}), per-slot adapter rank in {8,16,32,64}",
                   "token_rows": pf["T"], "slot_rows": pf["rows"], "ranks": pf["ranks"], "rounds": pf["rounds"]},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4), "traffic": None,
                     "kernel": "prefill round (LoRA shrink + gemm256_kernel), base-GEMM flops"},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def _graph_us(fn, iters=20, reps=5):
    """Mean µs of one fn() call: `iters` calls captured in one HIP graph after
    3 eager calls (which size the library's scratch and upload adapter
    tables), the graph replayed `reps` times between HIP events; the kernel
    boundaries inside the graph are counted, the host's launch time is not."""
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(iters):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * iters)
    del g
    return us


def _cpu_us(fn, budget_s=3.0, min_reps=20):
    """Median µs of fn() on the host's cores (3 warm-up calls)."""
    for _ in range(3):
        fn()
    ts = []
    t_start = time.perf_counter()
    while len(ts) < min_reps or (time.perf_counter() - t_start < budget_s and len(ts) < 200):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts) * 1e6


def _copies_for(nbytes, total=512 << 20):
    """Copies of a weight of nbytes that together pass `total` bytes."""
    return max(1, -(-total // nbytes))


def _decode_layer_case(dev, n_slots, adapter_of_slot, n_pool, seed):
    """One 8B-shaped layer's four projection rounds (fused QKV, O, Gate+Up,
    Down) over n_slots one-token slots, every weight and adapter bf16
    ~N(0, 0.02), activations ~N(0, 1); n_pool rank-16 adapters (scale 2.0)
    on all seven projections, slot i using adapter adapter_of_slot[i].
    Weights and stacked lora_A in fragment tiles (the decode step's layout).
    Each round keeps enough copies of its weight (at least 512 MB, twice the
    last-level cache) and every call takes the next one, so replays stream
    the weight from HBM as the decode step's layers do instead of finding it
    in the cache.  Returns the round closures and their algorithmic bytes."""
    import torch
    from swarmlora_amd import ops
    H, KV, I, r = 4096, 1024, 14336, 16
    gd = torch.Generator(device=dev).manual_seed(seed)

    def rn(*shape, std=0.02):
        return (torch.randn(*shape, generator=gd, device=dev) * std).to(torch.bfloat16)

    rounds = [("qkv", H, [H, KV, KV]), ("o", H, [H]), ("gate_up", H, [I, I]), ("down", I, [H])]
    used = sorted(set(adapter_of_slot))
    out = []
    for nm, k, dims in rounds:
        n = sum(dims)
        w_rm = rn(n, k)
        ws = [ops.pack_weight(w_rm) for _ in range(_copies_for(2 * n * k))]
        del w_rm
        table = ops.LoraTable(dev)
        for _ in range(n_pool):
            table.add(ops.pack_weight(rn(r * len(dims), k)), [rn(d, r) for d in dims], r, 2.0)
        xs = [rn(1, k, std=1.0) for _ in range(n_slots)]
        ys = [torch.empty(1, n, dtype=torch.bfloat16, device=dev) for _ in range(n_slots)]
        ids = list(adapter_of_slot)
        fz = ops.round_fusion(w_layout=1, a_layout=1)

        def run(xs=xs, ys=ys, ws=ws, table=table, ids=ids, dims=dims, fz=fz, turn=[0]):
            w = ws[turn[0] % len(ws)]
            turn[0] += 1
            ops.round_ex(xs, ys, [1] * len(xs), w, None, seg_lora=ids, table=table, blk_cols=dims, fusion=fz)

        nbytes = 2 * (n * k + n_slots * (k + n) + len(used) * r * len(dims) * k + len(used) * r * n)
        out.append((nm, run, nbytes, n, k))
    return out


def per_config_measure(args):
    """BASELINE configs 1, 2, 3 and 5 on this GPU: µs per round (per layer for
    the four-round configs) from HIP-graph replays, algorithmic bytes (or
    FLOPs for config 3) per unit, the achieved rate and its fraction of the
    roofline, and the BASELINE.md floor; configs 1 and 2 also on the host's
    CPU cores (the reference's torch path: oracle.execute_round plus the LoRA
    delta and add, bf16)."""
    import torch
    dev = torch.device("cuda:0")
    res = {}
    # config 1: fused QKV round, 4 one-token slots, one rank-16 adapter per
    # slot on the fused output (A [16, 4096], B [6144, 16]), scale 2.0
    from swarmlora_amd import ops
    H, QKV, r = 4096, 6144, 16
    gd = torch.Generator(device=dev).manual_seed(0)

    def rn(*shape, std=0.02):
        return (torch.randn(*shape, generator=gd, device=dev) * std).to(torch.bfloat16)

    w1 = rn(QKV, H)
    xs1 = [rn(1, H, std=1.0) for _ in range(4)]
    ad1 = [(rn(r, H), rn(QKV, r)) for _ in range(4)]
    wp1 = [ops.pack_weight(w1) for _ in range(_copies_for(2 * QKV * H))]  # streamed from HBM (see above)
    tab1 = ops.LoraTable(dev)
    ids1 = [tab1.add(ops.pack_weight(a), [b], r, 2.0) for a, b in ad1]
    ys1 = [torch.empty(1, QKV, dtype=torch.bfloat16, device=dev) for _ in range(4)]
    fz1 = ops.round_fusion(w_layout=1, a_layout=1)
    turn1 = [0]

    def run1():
        w = wp1[turn1[0] % len(wp1)]
        turn1[0] += 1
        ops.round_ex(xs1, ys1, [1] * 4, w, None, seg_lora=ids1, table=tab1, blk_cols=[QKV], fusion=fz1)

    us1 = _graph_us(run1, iters=50)
    b1 = 2 * (QKV * H + 4 * (H + QKV) + 4 * r * (H + QKV))
    # the CPU torch path on the same shapes (gather, x @ W.T, (x @ A.T) @ B.T * s, add, scatter)
    from oracle import reference_path as ref
    host = host_cpu_info()
    prev = torch.get_num_threads()
    torch.set_num_threads(host["usable_cpus"])
    w1c, xs1c, ad1c = w1.cpu(), [x.cpu() for x in xs1], [(a.cpu(), b.cpu()) for a, b in ad1]

    def cpu1():
        base = ref.execute_round(xs1c, [1] * 4, w1c)
        return [base[i] + ref.remote_lora_delta(xs1c[i], a, b, 2.0) for i, (a, b) in enumerate(ad1c)]

    cpu_us1 = _cpu_us(cpu1)
    res["config1"] = {"unit": "round", "us": round(us1, 2), "algorithmic_MB": round(b1 / 1e6, 2),
                      "GBps": round(b1 / us1 / 1e3, 1), "frac_hbm": round(b1 / us1 / 1e3 / HBM_PEAK_GBS, 4),
                      "floor_us": round(b1 / HBM_PEAK_GBS / 1e3, 2),
                      "cpu_baseline": {"us": round(cpu_us1, 1), "cores": host["usable_cpus"], "kind": "port",
                                       "sample": "oracle execute_round + remote_lora_delta per slot, torch-CPU bf16, "
                                                 "median of >= 20"}}
    del w1, wp1, tab1, xs1, ys1
    # configs 2 and 5: one layer's four rounds
    for name, n_slots, n_pool, ids in (
            ("config2", 28, 28, list(range(28))),
            ("config5", 64, 500, None)):
        if ids is None:
            g = torch.Generator().manual_seed(3)
            p = torch.tensor([(i + 1) ** -1.1 for i in range(n_pool)])
            ids = torch.multinomial(p / p.sum(), n_slots, replacement=True, generator=g).tolist()
        case = _decode_layer_case(dev, n_slots, ids, n_pool, seed=0)
        rounds = {}
        tot_us = tot_b = 0.0
        for nm, run, nb, n, k in case:
            u = _graph_us(run, iters=20)
            rounds[nm] = {"us": round(u, 2), "algorithmic_MB": round(nb / 1e6, 2),
                          "frac_hbm": round(nb / u / 1e3 / HBM_PEAK_GBS, 4)}
            tot_us += u
            tot_b += nb
        res[name] = {"unit": "layer (4 rounds)", "us": round(tot_us, 2), "algorithmic_MB": round(tot_b / 1e6, 2),
                     "GBps": round(tot_b / tot_us / 1e3, 1), "frac_hbm": round(tot_b / tot_us / 1e3 / HBM_PEAK_GBS, 4),
                     "floor_us": round(tot_b / HBM_PEAK_GBS / 1e3, 2), "slots": n_slots,
                     "distinct_adapters": len(set(ids)), "pool": n_pool, "rounds": rounds}
        del case
        torch.cuda.empty_cache()
    # config 2 on the CPU: one layer's four rounds at 28 slots (torch-CPU bf16)
    gc = torch.Generator().manual_seed(0)

    def rc(*shape, std=0.02):
        return (torch.randn(*shape, generator=gc) * std).to(torch.bfloat16)

    cpu_rounds = []
    for k, dims in ((4096, [4096, 1024, 1024]), (4096, [4096]), (4096, [14336, 14336]), (14336, [4096])):
        n = sum(dims)
        cpu_rounds.append((rc(n, k), [rc(1, k, std=1.0) for _ in range(28)],
                           [(rc(r, k), rc(n, r)) for _ in range(28)]))

    def cpu2():
        for w, xs, ad in cpu_rounds:
            base = ref.execute_round(xs, [1] * 28, w)
            [base[i] + ref.remote_lora_delta(xs[i], a, b, 2.0) for i, (a, b) in enumerate(ad)]

    cpu_us2 = _cpu_us(cpu2, budget_s=4.0, min_reps=5)
    torch.set_num_threads(prev)
    res["config2"]["cpu_baseline"] = {"us": round(cpu_us2, 1), "cores": host["usable_cpus"], "kind": "port",
                                      "sample": "oracle execute_round + per-slot LoRA delta for the four rounds, "
                                                "torch-CPU bf16, median of >= 5"}
    del cpu_rounds
    # config 3: the prefill rounds (MFMA bound)
    pf = prefill_measure(steps=20)  # 5 calls per round under-measure: the first after a sync starts slow
    res["config3"] = {"unit": "layer (4 rounds)", "us": round(pf["ms"] * 1e3, 1), "TFLOPs": pf["tflops"],
                      "frac_mfma": round(pf["tflops"] / 2500.0, 4), "token_rows": pf["T"],
                      "floor_us": round(pf["flops"] / 2.5e15 * 1e6, 1),
                      "rounds": pf["rounds"]}
    return res


IPC_WARM, IPC_COOL = 2, 2


def _ipc_worker(shm_name, claim, wid, all_sids, start, layers, n_tok, reps, gpu_ordered, pooled, out):
    """One worker process of the drop-in path: 8B-shaped layer modules with a
    rank-16 adapter (on the worker, or pooled in the aggregator), decoding
    through the aggregator.  All workers join together (barrier `start`), run
    untimed tokens until every slot of the run is active, then IPC_WARM
    tokens, `reps` timed windows of n_tok tokens, IPC_COOL tokens and two
    stage-timed tokens, so that no timed window overlaps another worker's
    joining, warm-up or stage-synchronised tokens (the rounds run in lock
    step: one slow worker slows every round)."""
    try:
        from types import SimpleNamespace
        import torch
        from swarmlora_amd import ext_ipc_queue as extq
        from swarmlora_amd import ext_unified_barrier as ub
        from swarmlora_amd.decode import DecodeShape, synthetic_adapter
        from swarmlora_amd.worker.batched_ops import BatchedAggregatorOps, SlotState
        from swarmlora_amd.worker.engine import LayerModules, StageTimer, WorkerEngine
        from swarmlora_amd.worker.model_builder import (FastLoRAModule, FusedLoRA, SyncFusedGateUp, SyncFusedQKV,
                                                        SyncRemoteLinear, SyncRemoteLoRALinear)
        from swarmlora_amd.worker.paged_attention import PagedKVCache, RotaryInvFreq, build_vllm_cos_sin_cache
        dev = torch.device("cuda:0")
        torch.cuda.set_device(0)
        s = DecodeShape(layers=layers)
        kvd = s.kv_heads * s.head_dim
        extq.open_queue(shm_name, 1024, 1024)
        ub.init_worker_slot_manager(wid, 0, 0, s.hidden, s.inter, s.qkv)
        sid = claim["slot_id"]
        ub.open_slot(sid, claim["input_handle"], claim["output_handle"], claim["input_buffer_size"],
                     claim["output_buffer_size"])
        ones = torch.ones(s.hidden, dtype=torch.bfloat16, device=dev)
        mods = []
        if pooled:
            # the aggregator adds the delta in its rounds: plain remote modules
            for li in range(layers):
                mods.append(LayerModules(ones, ones, SyncFusedQKV(li, [s.hidden, kvd, kvd], None),
                                         SyncRemoteLinear(3, li, s.hidden), SyncFusedGateUp(li, [s.inter, s.inter], None),
                                         SyncRemoteLinear(6, li, s.hidden)))
        else:
            ad = synthetic_adapter(s, dev, seed=1000 + wid)
            for li in range(layers):
                m = {p: FastLoRAModule(a.contiguous(), b.contiguous(), s.scale) for p, (a, b) in ad[li].items()}
                mods.append(LayerModules(ones, ones,
                                         SyncFusedQKV(li, [s.hidden, kvd, kvd], FusedLoRA([m["q"], m["k"], m["v"]],
                                                                                          [s.hidden, kvd, kvd], dev,
                                                                                          torch.bfloat16)),
                                         SyncRemoteLoRALinear(3, li, s.hidden, m["o"]),
                                         SyncFusedGateUp(li, [s.inter, s.inter], FusedLoRA([m["gate"], m["up"]],
                                                                                           [s.inter, s.inter], dev,
                                                                                           torch.bfloat16)),
                                         SyncRemoteLoRALinear(6, li, s.hidden, m["down"])))
        max_tok = 64 + IPC_WARM + reps * n_tok + IPC_COOL + 2
        kv = PagedKVCache(layers, s.kv_heads, s.head_dim, s.block_size, 1, max_tok, dev, torch.bfloat16)
        cs = build_vllm_cos_sin_cache(RotaryInvFreq(s.head_dim, s.theta), max_tok, dev, torch.bfloat16)
        bops = BatchedAggregatorOps(SimpleNamespace(base_client=SimpleNamespace(hidden_dim=s.hidden)), wid, 15,
                                    pooled_adapter=wid if pooled else None, gpu_ordered=gpu_ordered)
        eng = WorkerEngine(mods, ones, s.eps, s.heads, s.kv_heads, s.head_dim, kv, cs, bops)
        torch.cuda.synchronize()
        start.wait(timeout=300)
        extq.slot_signal_join(sid)
        t0 = time.time()
        while not extq.slot_is_active(sid):
            if time.time() - t0 > 120:
                raise RuntimeError("slot never became active")
            time.sleep(0.0005)
        st = SlotState(sid, torch.tensor([[1 + wid]], dtype=torch.int64, device=dev))
        slots = {sid: st}
        pre = 0
        while not all(extq.slot_is_active(x) for x in all_sids):
            eng.generate_one_token_all(slots)
            pre += 1
            if pre > 60:
                raise RuntimeError("the other workers never became active")
        for _ in range(IPC_WARM):
            eng.generate_one_token_all(slots)
        windows = []
        for _ in range(reps):
            t1 = time.perf_counter()
            for _ in range(n_tok):
                eng.generate_one_token_all(slots)  # host-synchronous: reads the sampled token
            windows.append(time.perf_counter() - t1)
        for _ in range(IPC_COOL):
            eng.generate_one_token_all(slots)
        eng.profiler = StageTimer()
        for _ in range(2):
            eng.generate_one_token_all(slots)
        prof = eng.profiler.records
        eng.profiler = None
        extq.slot_signal_leave(sid)
        ub.close_slot(sid)
        out.put((wid, (windows, prof, pre), None))
    except Exception:
        import traceback
        out.put((wid, None, traceback.format_exc()))


IPC_MODES = {  # name: (GPU-ordered rounds, adapters pooled in the aggregator)
    "host_sync": (False, False),          # the reference's protocol: worker-side LoRA, host-synchronised rounds
    "host_sync_pooled": (False, True),    # adapters in the aggregator's pool, delta added inside the round
    "gpu_ordered": (True, False),         # input copies and output reads ordered on the GPU
    "gpu_ordered_pooled": (True, True),
    "gpu_ordered_inputs": ("inputs", False),  # input copies ordered on the GPU, outputs read after the round
    "gpu_ordered_inputs_pooled": ("inputs", True),
}
IPC_MODE_TEXT = {
    "host_sync": "adapter applied on the worker, host-synchronised rounds (the reference's protocol)",
    "host_sync_pooled": "adapters pooled in the aggregator's rounds",
    "gpu_ordered": "input copies and output reads ordered on the GPU",
    "gpu_ordered_pooled": "input copies and output reads ordered on the GPU, adapters pooled",
    "gpu_ordered_inputs": "the worker's own LoRA with the input copies ordered on the GPU",
    "gpu_ordered_inputs_pooled": "input copies ordered on the GPU, adapters pooled",
}


def ipc_measure(W, L, n_tok, modes, reps=3, passes=1):
    """The multi-process serving path: this process is the aggregator (native
    main loop on a thread, 8B-shaped weights for L layers, embed and LM
    head), W worker processes decode one token per step each through the
    shared-memory ring and IPC-mapped slots, once per mode of IPC_MODES in
    each of `passes` passes over the modes (fresh worker processes per run).
    Per mode: tokens/s, step time and µs per round from the median of all
    its timed windows (`reps` windows of n_tok tokens per run, per window the
    slowest worker), each pass's median, then the mean [LAYER_PROFILE] stage
    split of two stage-timed tokens per worker and run."""
    import multiprocessing as mp
    import threading
    import torch
    from swarmlora_amd import ext_aggregator as agg
    from swarmlora_amd import ext_ipc_queue as extq
    from swarmlora_amd.decode import DecodeShape, synthetic_adapter, synthetic_weights
    dev = torch.device("cuda:0")
    s = DecodeShape(layers=L)
    wts = synthetic_weights(s, dev, seed=0)
    runs = {m: [] for m in modes}
    for mode in [m for _ in range(passes) for m in modes]:
        gpu_ordered, pooled = IPC_MODES[mode]
        q = extq.create_queue(1024, 1024)
        extq.init_batch_control(W)
        agg.init_slot_pool(W, 0, s.hidden, s.inter, s.kv_heads, s.head_dim, 1, 2)
        agg.init_aggregator_begin(L, 0)
        for li, w in enumerate(wts["layers"]):
            agg.init_aggregator_layer(li, w["q"], w["k"], w["v"], w["o"], torch.empty(0), w["gate"], w["up"],
                                      w["down"], torch.empty(0))
        agg.init_aggregator_finalize()
        agg.init_embed_lm_head_weights(wts["embed"], wts["lm_head"])
        agg.init_aggregator_queue(q["shm_name"], 1024)
        agg.clear_adapters()
        if pooled:
            for wid in range(W):
                ad = synthetic_adapter(s, dev, seed=1000 + wid)
                for li in range(L):
                    for op, projs in ((agg.OP_QKV_FUSED, ("q", "k", "v")), (agg.OP_O_PROJ, ("o",)),
                                      (agg.OP_GATE_UP_FUSED, ("gate", "up")), (agg.OP_DOWN_PROJ, ("down",))):
                        agg.register_adapter(wid, li, op, torch.cat([ad[li][p][0] for p in projs], 0).contiguous(),
                                             [ad[li][p][1].contiguous() for p in projs], s.scale)
                del ad
        claims = {wid: agg.claim_slot(wid) for wid in range(W)}
        sids = [claims[w]["slot_id"] for w in range(W)]
        loop = threading.Thread(target=agg.aggregator_main_loop_slots, args=(W, 15), daemon=True)
        loop.start()
        ctx = mp.get_context("spawn")
        out = ctx.Queue()
        start = ctx.Barrier(W)
        procs = [ctx.Process(target=_ipc_worker, args=(q["shm_name"], claims[w], w, sids, start, L, n_tok, reps,
                                                       gpu_ordered, pooled, out))
                 for w in range(W)]
        wins, profs, pre = [], [], []
        load0 = os.getloadavg()[0]
        try:
            for p in procs:
                p.start()
            for _ in procs:
                wid, r, err = out.get(timeout=600)
                if err:
                    raise RuntimeError(f"worker {wid}: {err}")
                wins.append(r[0])
                profs.extend(r[1])
                pre.append(r[2])
        finally:
            extq.set_quit(1)
            loop.join(timeout=60)
            for p in procs:
                p.join(timeout=60)
                if p.is_alive():
                    p.kill()
            for wid in range(W):
                try:
                    agg.release_slot(claims[wid]["slot_id"], wid)
                except RuntimeError:
                    pass
            agg.clear_adapters()
            agg.cleanup_slot_pool()
            extq.close_queue()
        per_win = [max(w[i] for w in wins) / n_tok for i in range(reps)]  # slowest worker per window
        runs[mode].append((per_win, profs, max(pre), load0))
    rounds = 2 + 4 * L
    res = {}
    for mode, rr in runs.items():
        wins_all = [x for r in rr for x in r[0]]
        profs = [p for r in rr for p in r[1]]
        step_s = statistics.median(wins_all)
        split = {k: round(statistics.fmean(r[k] for r in profs), 1)
                 for k in ("gather_us", "gemm_us", "scatter_us", "lora_us", "attn_us", "compute_us", "wall_us")}
        split["ipc_pct"] = round(100.0 * (split["gather_us"] + split["scatter_us"]) / split["wall_us"], 1)
        split["round_wait_us"] = round(split["gemm_us"] / rounds, 1)
        res[mode] = {"tok_s": round(W / step_s, 1), "ms_per_step": round(step_s * 1e3, 3),
                     "us_per_round": round(step_s * 1e6 / rounds, 1),
                     "us_per_round_passes": [round(statistics.median(r[0]) * 1e6 / rounds, 1) for r in rr],
                     "us_per_round_windows": [round(x * 1e6 / rounds, 1) for x in wins_all],
                     "untimed_tokens_before_all_active": max(r[2] for r in rr),
                     "host_load_1min": [round(r[3], 2) for r in rr],
                     "layer_profile": split}
    return res


def _drop_in_child(W, L, n_tok, modes, reps, passes, out):
    """ipc_measure in a process of its own (a fresh aggregator: nothing of the
    parent's GPU state, threads or memory carries over)."""
    try:
        out.put((ipc_measure(W, L, n_tok, modes, reps, passes), None))
    except Exception:
        import traceback
        out.put((None, traceback.format_exc()))


def drop_in_leg(W, L, n_tok, modes, reps=3, passes=1):
    """ipc_measure run by a freshly spawned aggregator process."""
    import multiprocessing as mp
    ctx = mp.get_context("spawn")
    out = ctx.Queue()
    p = ctx.Process(target=_drop_in_child, args=(W, L, n_tok, modes, reps, passes, out))
    p.start()
    try:
        res, err = out.get(timeout=900)
    finally:
        p.join(timeout=120)
        if p.is_alive():
            p.kill()
    if err:
        raise RuntimeError(err)
    return res


def ipc(args):
    """--workload ipc: the drop-in path's line on its own; `value` is tokens/s
    of the first mode."""
    W = min(args.workers, 8)
    L = args.ipc_layers
    modes = [m for m in args.ipc_modes.split(",") if m]
    res = drop_in_leg(W, L, args.ipc_tokens, modes, args.ipc_reps, args.ipc_passes)
    first = res[modes[0]]
    line = {
        "metric": f"multi-process decode tok/s (drop-in path, {modes[0]})",
        "value": first["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.ipc_tokens * args.ipc_reps * args.ipc_passes,
        "warmup": IPC_WARM,
        "ms_per_step": first["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random-init weights and adapters)",
        "config": {"workload": f"{W} worker processes x 1 decode token, {L} Llama-3.1-8B-shaped layers, rank-16 "
                               "adapter per worker, aggregator main loop in a spawned process",
                   "workers": W, "layers": L, "rounds_per_token": 2 + 4 * L, "modes": res},
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build runs on one GPU (one aggregator per GPU; workers and aggregator share it "
              "through same-device IPC). --gpus must be 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.workload == "prefill":
        return prefill(args)
    if args.workload == "ipc":
        return ipc(args)
    if args.workload == "configs":
        print(json.dumps({"per_config": per_config_measure(args)}), flush=True)
        return
    from swarmlora_amd import ops
    from swarmlora_amd.decode import BatchedDecoder, DecodeShape, synthetic_adapter, synthetic_weights

    dev = torch.device("cuda:0")
    W = args.workers
    s = DecodeShape()
    ctx = torch.randint(128, 2049, (W,), generator=torch.Generator().manual_seed(3)).tolist()
    first = torch.randint(0, s.vocab, (W,), generator=torch.Generator().manual_seed(4)).tolist()
    weights = synthetic_weights(s, dev, seed=0)
    adapters = [synthetic_adapter(s, dev, seed=1000 + w) for w in range(W)]
    kv_gen = torch.Generator(device=dev).manual_seed(5)

    def kv_fill(li, kc, vc, bt):
        kc.copy_(torch.randn(kc.shape, generator=kv_gen, device=dev, dtype=torch.bfloat16))
        vc.copy_(torch.randn(vc.shape, generator=kv_gen, device=dev, dtype=torch.bfloat16))

    max_new = 1 + args.warmup + args.steps + args.timer_steps + 1
    dec = BatchedDecoder(s, weights, adapters, ctx, first, dev, max_new=max_new, kv_fill=kv_fill,
                         packed=args.weights == "packed",
                         whole_k=args.whole_k == "lm")
    del weights, adapters
    torch.cuda.synchronize()

    dec.step_eager()  # sizes scratch, uploads the adapter table
    dec.capture()
    for _ in range(args.warmup):
        dec.step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        dec.step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    ms_per_step = gpu_ms / args.steps
    value = W * args.steps / (gpu_ms / 1e3)

    # per-launch HIP events on eager steps of the same workload
    n_rounds = 4 * s.layers
    ops.timer_arm(args.timer_steps * (n_rounds + 1))
    for _ in range(args.timer_steps):
        # keep the GPU busy while the host queues the step's ~450 launches,
        # so they run back to back like the graph replays
        torch.cuda.synchronize()
        torch.cuda._sleep(100_000_000)
        dec.step_eager()
    recs = ops.timer_collect()
    # the dominant kernel: the K-sliced base kernel (split_kernel) of the 128
    # projection rounds; the LM head (a whole-K round by default) is in the
    # `rounds` breakdown only
    lm_wk = bool(dec.wk.get("lm"))
    dom = [r for r in recs if not (lm_wk and r["n"] == s.vocab)]
    base_ms = [r["base_ms"] for r in dom]
    base_bytes = [r["bytes"] for r in dom]
    mean_ms = statistics.fmean(base_ms)
    mean_bytes = statistics.fmean(base_bytes)
    achieved = mean_bytes / (mean_ms * 1e-3) / 1e9
    rounds = [r for r in recs if r["n"] != s.vocab]
    us_round = statistics.fmean([(r["base_ms"] + r["epilogue_ms"]) * 1e3 for r in rounds])
    per_op = {}
    names = {(s.qkv, s.hidden): "qkv", (s.hidden, s.hidden): "o", (2 * s.inter, s.hidden): "gate_up",
             (s.hidden, s.inter): "down", (s.vocab, s.hidden): "lm_head"}
    for r in recs:
        nm = names.get((r["n"], r["k"]), f"{r['n']}x{r['k']}")
        per_op.setdefault(nm, []).append(r)
    breakdown = {nm: {"base_us": round(statistics.fmean([x["base_ms"] for x in v]) * 1e3, 2),
                      "epilogue_us": round(statistics.fmean([x["epilogue_ms"] for x in v]) * 1e3, 2),
                      "base_GBps": round(statistics.fmean([x["bytes"] for x in v]) /
                                         (statistics.fmean([x["base_ms"] for x in v]) * 1e-3) / 1e9, 1)}
                 for nm, v in per_op.items()}
    traffic = read_traffic()
    copy_calibration(args, dev)

    step_bytes = s.step_bytes(ctx, W)
    dec.close()
    del dec
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    drop_in = None
    if not args.no_ipc:
        # the drop-in path: a freshly spawned aggregator process, real worker
        # processes, the shared-memory ring and IPC slot buffers, 8B widths
        W_ipc = max(1, min(args.ipc_workers, 8))
        modes = [m for m in args.ipc_modes.split(",") if m]
        try:
            res = drop_in_leg(W_ipc, args.ipc_layers, args.ipc_tokens, modes, args.ipc_reps, args.ipc_passes)
            drop_in = {
                "workload": f"{W_ipc} worker processes + a spawned aggregator process, {args.ipc_layers} 8B-shaped "
                            f"layers ({2 + 4 * args.ipc_layers} rounds per token), rank-16 adapter per worker; "
                            + "".join(f"{m}: {IPC_MODE_TEXT[m]}; " for m in modes)
                            + f"{args.ipc_passes} passes over the "
                            f"modes in turn, {args.ipc_reps} windows of {args.ipc_tokens} tokens per run once "
                            "every slot is active, median window of all passes",
                "workers": W_ipc, "layers": args.ipc_layers, "rounds_per_token": 2 + 4 * args.ipc_layers, **res}
        except Exception as e:  # the headline line is still printed
            drop_in = {"error": f"{type(e).__name__}: {e}"[:2000]}
    per_config = None
    if not args.no_per_config:
        try:
            per_config = per_config_measure(args)
        except Exception as e:  # the headline line is still printed
            per_config = {"error": f"{type(e).__name__}: {e}"[:2000]}
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(W, args.cpu_seconds)

    line = {
        "metric": "tok/s at 28 workers, 8B-shape decode; µs per gather-GEMM-scatter round",
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / REFERENCE_TOK_S, 2),
        "dtype": "bf16",
        "data": "synthetic (seeded random-init weights, adapters, KV pages and token ids)",
        "config": {"workload": "config4: 32-layer Llama-3.1-8B-shaped batched decode step, 28 workers x 1 token, "
                               "rank-16 adapter per worker on q/k/v/o/gate/up/down, paged KV ctx U{128..2048}, "
                               "130 rounds per token, greedy sampling, captured as one HIP graph",
                   "workers": W, "layers": s.layers, "rounds_per_token": 2 + n_rounds,
                   "weight_layout": args.weights,
                   "us_per_round": round(us_round, 2),
                   "us_per_round_of_step": round(ms_per_step * 1e3 / (2 + n_rounds), 2),
                   "step_algorithmic_GB": round(step_bytes / 1e9, 3),
                   "step_GBps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                   "wall_s": round(wall, 3),
                   "rounds": breakdown},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": ("split_kernel (K-sliced decode projection base kernel; the LM head is "
                                + ("a whole-K round)" if lm_wk else "K-sliced too)")),
                     "launches": len(dom),
                     "mean_launch_us": round(mean_ms * 1e3, 3), "bytes_per_launch": int(mean_bytes)},
        "cpu_baseline": cpu,
    }
    if per_config is not None:
        line["config"]["per_config"] = per_config
    if drop_in is not None:
        line["config"]["drop_in"] = drop_in
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
