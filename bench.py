"""MoE decode throughput at batch 1 on a Qwen3-30B-A3B-shaped Q4_K stack, all experts cached.

Workload (one "step" = one decode token through the whole MoE stack):
  48 layers, hidden 2048, 128 experts, top-8, expert intermediate 768, gate/up/down
  Q4_K from N(0, 0.02), router f32 N(0, 0.02) [128, 2048], activations N(0, 1) bf16,
  every expert resident in its layer's slot bank.  Each step starts from its own
  synthetic token and runs x <- bf16(x + MoE_l(x)) for l = 0..47 with routing on
  the device (naiwa_stack_decode, fused persistent kernel).

Prints one JSON line: tok/s, the dominant kernel's achieved HBM GB/s against the
8 TB/s MI355X peak (algorithmic bytes of the experts actually routed, the router
weights and the activations), and a CPU baseline: the CPU oracle's restatement of
the reference's CPU expert path (plus router) timed on a bounded sample of the
same layers and tokens on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "naiwa-rs_amd"))

METRIC = "MoE decode tok/s @bs1 (Qwen3-30B-A3B shape, Q4_K); HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0
Q4K_BLOCK, Q4K_BYTES = 256, 144


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "stack_kernel_qwen3_bs1_traffic.txt")
PREFILL_TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "prefill_deepseek_v2_lite_traffic.txt")


def profile_traffic(path: str):
    """The traffic_bytes_per_launch line of a committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (scaled by a device copy of known size), or None."""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    return None


def measured_traffic(rows: int, layers: int, fused: bool):
    """HBM bytes per launch of the fused kernel on this exact workload (bs1, 48
    layers); None for any other workload."""
    if not (fused and rows == 1 and layers == 48):
        return None
    return profile_traffic(TRAFFIC_PROFILE)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def activation_health(buf, n: int) -> dict:
    """Largest |value| and count of non-finite values of n bf16 activations on the device
    (a chained residual stream whose values overflow routes on NaN and measures nothing)."""
    v = (buf.download(np.uint16)[:n].astype(np.uint32) << 16).view(np.float32)
    finite = np.isfinite(v)
    return {"absmax": float(np.abs(v[finite]).max()) if finite.any() else None,
            "nonfinite": int((~finite).sum())}


# Std of the synthetic down projections of the chained prefill and Mixtral stacks.
# With N(0, 0.02) down weights one layer's output is as large as its unit-scale input
# and grows with its square, so the residual chain overflows within a few layers; at
# these values a layer adds about a tenth of the input's scale and the chain stays
# finite (checked by activation_health on every run).
DOWN_STD_DEEPSEEK = 0.004
DOWN_STD_MIXTRAL = 0.0015


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--rows", type=int, default=1, help="decode batch (tokens per step)")
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--path", choices=["auto", "fused", "layered"], default="auto",
                    help="auto: the fused persistent kernel up to 4 rows, per-layer launches (matrix-core "
                         "expert GEMMs) from 5 rows on (measured: fused 1,548 vs 1,486 tok/s at 4 rows, "
                         "1,518 vs 1,765 at 5)")
    ap.add_argument("--blocks-per-cu", type=int, default=2)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="budget of the CPU-baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run one device-to-device copy of MIB MiB before timing (a known-size "
                         "reference for HBM traffic counters)")
    ap.add_argument("--trace", action="store_true",
                    help="print per-phase times of one fused step (diagnostic, untimed)")
    ap.add_argument("--lookahead-swaps", type=int, default=-1, metavar="N",
                    help="cache25: predict each next layer's experts from this layer's activation and load them "
                         "(at most N LRU swaps per row, the reference's --lookahead-swaps); -1 = off")
    ap.add_argument("--depth", type=int, default=0, metavar="N",
                    help="prefill-stream: layer buffers (default: the memory plan's stride)")
    ap.add_argument("--budget-gb", type=float, default=0.0, metavar="GB",
                    help="prefill-stream: device memory the plan may assume free (default: what is free)")
    ap.add_argument("--cache-layers", type=int, default=32, metavar="N",
                    help="mixtral: layers of the 4-of-8 cached decode (each pins 0.8 GB of host stacks)")
    ap.add_argument("--db-iters", type=int, default=20000, help="doorbell: round trips timed")
    ap.add_argument("--upload-sync", choices=["event", "poll"], default="poll",
                    help="cache25: staged uploads complete into the expert pass through an event the compute "
                         "stream waits for, or a device flag one wave polls")
    ap.add_argument("--upload-path", choices=["kernel", "dma"], default="kernel",
                    help="cache25: staged uploads as one copy kernel reading the mapped host stacks (the expert "
                         "pass after it), or hipMemcpyAsync on the copy stream (the cache pairs during it)")
    ap.add_argument("--pcie-frac", type=float, default=1.0,
                    help="cache25: share of each step's missed experts staged over PCIe; the rest run on the "
                         "CPU (the reference's default is 0)")
    ap.add_argument("--workload", choices=["resident", "cache25", "prefill", "prefill-stream", "mixtral", "doorbell"],
                    default="resident",
                    help="resident: every expert in HBM (the headline); cache25: 32 of 128 experts "
                         "cached per layer, Zipf(1.1) routing, misses streamed over PCIe; prefill: "
                         "DeepSeek-V2-Lite-shaped 2048-token prefill in 512-token chunks (MFMA)")
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.workload in ("cache25", "prefill", "prefill-stream", "mixtral", "doorbell"):
        if args.gpus != 1:
            print("bench.py measures one GPU", file=sys.stderr)
            return 2
        if args.workload == "prefill-stream":
            return run_prefill_stream(args)
        if args.workload == "mixtral":
            return run_mixtral(args)
        if args.workload == "doorbell":
            return run_doorbell(args)
        return run_cache25(args) if args.workload == "cache25" else run_prefill(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(the expert path runs on one GPU; how it would shard is described, not built)", file=sys.stderr)
        return 2
    import naiwa_moe as nm

    if nm.device_count() < 1:
        log("no HIP device")
        return 1
    info = nm.device_info(0)
    log(f"device {info}")
    L, H, E, K, I, rows = args.layers, 2048, 128, 8, 768, args.rows
    nm.lib().naiwa_stack_set_blocks_per_cu(args.blocks_per_cu)

    # ---- synthetic weights on the device ----
    t0 = time.time()
    stream = nm.Stream()
    layers, keep = [], []
    proj_bytes = I * (H // Q4K_BLOCK) * Q4K_BYTES  # 884,736 B per projection per expert
    for l in range(L):
        banks = nm.LayerBanks(E, H, I, (nm.Q4_K,) * 3)
        for t, bank in enumerate((banks.gate, banks.up, banks.down)):
            assert bank.stride == proj_bytes
            nm.synth(nm.Q4_K, 1000 + 8 * l + t, E * bank.n * bank.k, bank.base, 0.0, 0.02,
                     stream=stream.handle)
        router = nm.DeviceBuffer(E * H * 4)
        nm.synth(nm.F32, 1000 + 8 * l + 3, E * H, router, 0.0, 0.02, stream=stream.handle)
        layers.append(nm.layer_desc(router, banks))
        keep += [banks, router]
    steps_total = args.warmup + args.steps
    xs = nm.DeviceBuffer(steps_total * rows * H * 2)
    nm.synth(nm.BF16, 999, steps_total * rows * H, xs, 0.0, 1.0, stream=stream.handle)
    stream.sync()
    log(f"synthesized {L} layers ({L * 3 * E * proj_bytes / 1e9:.2f} GB Q4_K) in {time.time() - t0:.1f}s")

    import ctypes as C
    arr = (nm._lib.Layer * L)(*layers)
    x = nm.DeviceBuffer(rows * H * 2)
    ids_d = nm.DeviceBuffer(L * rows * K * 4)
    w_d = nm.DeviceBuffer(L * rows * K * 4)
    if args.path == "auto":
        args.path = "fused" if rows <= 4 else "layered"
    fused = args.path == "fused"
    lib = nm.lib()

    def step(i: int, record_routing: bool) -> None:
        lib.naiwa_memcpy_d2d(x.ptr, xs.ptr + i * rows * H * 2, rows * H * 2, stream.handle)
        nm.stack_decode(arr, x, rows, H, E, K, ids_out=ids_d if record_routing else None,
                        w_out=w_d if record_routing else None, fused=fused, stream=stream.handle)

    for i in range(args.warmup):
        step(i, True)
    stream.sync()
    if fused:
        to, miss = nm.stack_status()
        if to or miss:
            log(f"fused kernel status: {to} barrier timeouts, {miss} missing experts")
            return 1
    # routing sanity and distinct experts per layer (for the algorithmic bytes)
    ids = ids_d.download(np.uint32).reshape(L, rows, K)
    ws = w_d.download(np.float32).reshape(L, rows, K)
    assert (ids < E).all() and np.allclose(ws.sum(-1), 1.0, atol=1e-4), "routing output invalid"

    if args.calibrate_copy:
        calibration_copy(nm, args.calibrate_copy, stream)

    if args.trace and fused:
        print_trace(nm, lambda: step(0, False), stream, L, info["wall_clock_khz"])

    # ---- timed region ----
    ev = [nm.Event() for _ in range(args.steps + 1)]
    k0, k1 = [nm.Event() for _ in range(args.steps)], [nm.Event() for _ in range(args.steps)]
    distinct = []
    nm.synchronize()
    start = time.perf_counter()
    ev[0].record(stream.handle)
    for s in range(args.steps):
        i = args.warmup + s
        lib.naiwa_memcpy_d2d(x.ptr, xs.ptr + i * rows * H * 2, rows * H * 2, stream.handle)
        k0[s].record(stream.handle)
        nm.stack_decode(arr, x, rows, H, E, K, ids_out=ids_d, w_out=w_d, fused=fused,
                        stream=stream.handle)
        k1[s].record(stream.handle)
        ev[s + 1].record(stream.handle)
    stream.sync()
    wall = time.perf_counter() - start
    total_ms = ev[0].elapsed_ms(ev[-1])
    kernel_ms = [k0[s].elapsed_ms(k1[s]) for s in range(args.steps)]
    # distinct experts routed per layer in the last timed step (bs1: always 8)
    ids = ids_d.download(np.uint32).reshape(L, rows, K)
    distinct = [len(np.unique(ids[l])) for l in range(L)]
    if fused:
        to, miss = nm.stack_status()
        if to or miss:
            log(f"fused kernel status after timing: {to} barrier timeouts, {miss} missing")
            return 1

    health = activation_health(x, rows * H)
    if health["nonfinite"]:
        log(f"activations overflowed: {health}")
        return 1

    ms_per_step = total_ms / args.steps
    tok_s = rows * args.steps / (total_ms / 1e3)
    kern_avg_ms = float(np.mean(kernel_ms))
    # algorithmic bytes per step: distinct routed experts x 3 projections, the router, x in/out
    expert_bytes = 3 * proj_bytes
    alg_bytes = sum(d * expert_bytes for d in distinct) + L * (E * H * 4 + rows * H * 4)
    achieved = alg_bytes / (kern_avg_ms / 1e3) / 1e9
    log(f"{args.path}: {ms_per_step * 1e3:.1f} us/step, kernel {kern_avg_ms * 1e3:.1f} us, "
        f"{tok_s:.1f} tok/s, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS * 100:.1f}% of peak), "
        f"wall {wall:.3f}s")

    cpu = None if args.no_cpu_baseline else cpu_baseline(nm, layers_host_sample(nm, keep, L, E, H, I),
                                                         xs, rows, H, E, K, I, L, args.cpu_seconds)
    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 x Q4_K (f32 accumulate)",
        "data": "synthetic (device-generated N(0,0.02) Q4_K experts, N(0,1) bf16 tokens)",
        "config": {
            "workload": f"Qwen3-30B-A3B-shaped MoE stack decode, bs{rows}, all experts cached",
            "layers": L, "hidden": H, "experts": E, "top_k": K, "intermediate": I,
            "weights": "Q4_K", "activations": "bf16", "rows": rows, "path": args.path,
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(rows, L, fused),
            "kernel": "stack_kernel<Q4_K,Q4_K>" if fused else "layered chain",
            "bytes_per_launch": alg_bytes,
            "kernel_avg_us": round(kern_avg_ms * 1e3, 2),
        },
        "activations_after_last_layer": health,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def calibration_copy(nm, mib, stream) -> None:
    """One device-to-device copy of mib MiB, so a counter profile of the same process
    can be scaled by what its counters read for bytes of known size."""
    nbytes = mib << 20
    a, b = nm.DeviceBuffer(nbytes), nm.DeviceBuffer(nbytes)
    a.zero(stream.handle)
    stream.sync()
    nm.lib().naiwa_memcpy_d2d(b.ptr, a.ptr, nbytes, stream.handle)
    stream.sync()
    log(f"calibration copy: {nbytes} bytes device to device")
    del a, b


def print_trace(nm, run, stream, L, khz):
    """One extra (untimed) fused step with every workgroup's phase timestamps, reduced to
    the critical path of each layer: logits published -> all received -> gate/up done
    (slowest producer) -> h received -> down + partials done (slowest) -> next logits."""
    import ctypes as C
    lib = nm.lib()
    lib.naiwa_stack_trace_enable(1)
    run()
    stream.sync()
    lib.naiwa_stack_trace_enable(0)
    slots = 24
    cap = 2048 * (L + 1) * slots
    buf = (C.c_uint64 * cap)()
    nl, nb = C.c_int(0), C.c_int(0)
    nm._lib.check(lib.naiwa_stack_trace_read(buf, cap, C.byref(nl), C.byref(nb)), "trace_read")
    G = nb.value
    t = np.frombuffer(buf, dtype=np.uint64)[: G * (L + 1) * slots].astype(np.float64)
    t = t.reshape(G, L + 1, slots) / (khz / 1000.0)
    nlead = min(32, G)
    names = ["recv", "rank", "route", "issue", "gate_up", "h_recv", "down", "combine", "partials", "reduce"]
    med = {n: [] for n in names[1:]}
    crit = {"logits->recv(max)": [], "recv->gate_up end(max)": [], "h hop": [], "h recv spread": [],
            "h recv->partials(max)": [], "reduce hop": []}
    late_gu, late_dn = np.zeros(8), np.zeros(8)
    pub = t[:nlead, L, 2].max()
    for l in range(L - 1):
        m = t[:, l]
        for i, n in enumerate(names[1:], start=1):
            if n in ("h_recv",):
                continue
            med[n].append(np.median(m[:, i] - m[:, i - 1]))
        gu_end = m[:, 4].max()
        crit["logits->recv(max)"].append(m[:, 0].max() - pub)
        crit["recv->gate_up end(max)"].append(gu_end - m[:, 0].max())
        crit["h hop"].append(m[:, 5].min() - gu_end)
        crit["h recv spread"].append(m[:, 5].max() - m[:, 5].min())
        crit["h recv->partials(max)"].append(m[:, 8].max() - m[:, 5].max())
        nxt = m[:nlead, 9].max()
        crit["reduce hop"].append(nxt - m[:, 8].max())
        pub = nxt
        for w in np.argsort(m[:, 4])[-16:]:
            late_gu[w % 8] += 1
        for w in np.argsort(m[:, 8])[-16:]:
            late_dn[w % 8] += 1
    log("trace: median per-workgroup phase us/layer: " +
        ", ".join(f"{n} {np.mean(v):.2f}" for n, v in med.items() if v))
    log("trace: critical path us/layer: " + ", ".join(f"{n} {np.mean(v):.2f}" for n, v in crit.items()) +
        f" | sum {sum(np.mean(v) for n, v in crit.items() if n != 'h recv spread'):.2f}")
    land = t[:, : L - 1, 21] - t[:, : L - 1, 3]
    # (at one token, marks 21 follow the first of the two landing groups, rows r of each item)
    log(f"trace: gate/up rows (r) landed, last wave after wave 0: median {np.median(land):.2f} us; "
        f"last wave's compute (and rows r + 1 landing) {np.median(t[:, : L - 1, 16] - t[:, : L - 1, 21]):.2f}; "
        f"top-k ready {np.median(t[:, : L - 1, 22] - t[:, : L - 1, 1]):.2f} after the ranks, pairs grouped "
        f"{np.median(t[:, : L - 1, 12] - t[:, : L - 1, 22]):.2f} later")
    cyc = np.frombuffer(buf, dtype=np.uint64)[: G * (L + 1) * slots].reshape(G, L + 1, slots)[:, :L, 23]
    dc = np.diff(cyc.astype(np.float64), axis=1)
    dt_us = np.diff(t[:, :L, 2], axis=1)
    log(f"trace: shader clock over the layers: median {np.median(dc / dt_us):.0f} MHz "
        f"(min {np.min(dc / dt_us):.0f}, max {np.max(dc / dt_us):.0f})")
    gu = t[:, : L - 1, 4] - t[:, : L - 1, 3]
    log(f"trace: gate_up (issue->done) us: median {np.median(gu):.2f} p90 {np.percentile(gu, 90):.2f} "
        f"max {gu.max():.2f}; recv spread {np.mean(t[:, :L-1, 0].max(0) - t[:, :L-1, 0].min(0)):.2f}")
    sub = {"logits seen": [], "x staged (wave 1)": [], "keys+barrier": [], "weights": [], "pairs": []}
    pub = t[:nlead, L, 2].max()
    for l in range(L - 1):
        m = t[:, l]
        if m[:, 10].min() > 0:
            sub["logits seen"].append(np.median(m[:, 10]) - pub)
            sub["x staged (wave 1)"].append(np.median(m[:, 13]) - pub)
            sub["keys+barrier"].append(np.median(m[:, 0] - m[:, 10]))
            sub["weights"].append(np.median(m[:, 11] - m[:, 2]))
            sub["pairs"].append(np.median(m[:, 12] - m[:, 1]))
        pub = m[:nlead, 9].max()
    if sub["weights"]:
        log("trace: one-token routing, median us after the last logits publish: " +
            ", ".join(f"{n} {np.mean(v):.2f}" for n, v in sub.items()))
    log("trace: XCD of the 16 latest gate/up finishers " + str(late_gu.astype(int).tolist()) +
        ", of the 16 latest partials " + str(late_dn.astype(int).tolist()))
    # per-XCD medians (workgroup b runs on XCD b % 8), us after the last logits publish
    rows = []
    pubs = np.concatenate([[t[:nlead, L, 2].max()], t[:nlead, : L - 2, 9].max(0)])
    rel = t[:, : L - 1, :] - pubs[None, :, None]
    for x in range(8):
        m = rel[x::8]
        rows.append(f"xcd{x}: recv {np.median(m[:, :, 0]):.2f} dma {np.median(m[:, :, 3] - m[:, :, 2]):.2f} "
                    f"gu_end {np.median(m[:, :, 4]):.2f} h_recv {np.median(m[:, :, 5]):.2f} "
                    f"gu_last_wave {np.median(m[:, :, 16]):.2f} max {np.median(m[:, :, 16].max(0)):.2f} "
                    f"ind {np.median(m[:, :, 14]):.2f} h_loads {np.median(m[:, :, 17]):.2f} "
                    f"polls {np.median(t[x::8, : L - 1, 18] * (khz / 1000.0)):.0f} h_read {np.median(m[:, :, 15]):.2f} "
                    f"down {np.median(m[:, :, 6] - m[:, :, 5]):.2f} part_end {np.median(m[:, :, 8]):.2f}")
    log("trace: per XCD, median us after the logits publish:\n  " + "\n  ".join(rows))
    lead = rel[:nlead]
    log(f"trace: leaders: part_end(own) {np.median(lead[:, :, 8]):.2f} partials seen {np.median(lead[:, :, 19]):.2f} "
        f"(polls {np.median(t[:nlead, : L - 1, 20] * (khz / 1000.0)):.0f}) published {np.median(lead[:, :, 9]):.2f}; "
        f"all part_end max {np.median(rel[:, :, 8].max(0)):.2f}")
    log(f"trace: kernel span {t[:, L - 1, 9].max() - t[:, L, 0].min():.1f} us over {G} workgroups")


def layers_host_sample(nm, keep, L, E, H, I, n_layers: int = 4):
    """Host copies of a few layers (router + every expert's bytes) for the CPU baseline."""
    picks = sorted(set(int(round(v)) for v in np.linspace(0, L - 1, n_layers)))
    out = []
    for l in picks:
        banks, router = keep[2 * l], keep[2 * l + 1]
        get = lambda b: b.buffer.download(np.uint8).reshape(E, b.n, -1)
        out.append((router.download(np.float32).reshape(E, H), (get(banks.gate), get(banks.up),
                                                                get(banks.down))))
    return out


# Host threads for the CPU baseline: every physical core of the host, at most the GPU's
# share of the host's cores (16 per GPU).
CPU_BASELINE_MAX_THREADS = 16


def cpu_threads():
    """(threads used, physical cores from lscpu or None, logical cores)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cpu_baseline as CB

    phys = CB.physical_cores()
    logical = os.cpu_count() or 1
    return max(1, min(CPU_BASELINE_MAX_THREADS, phys or logical)), phys, logical


def cpu_baseline(nm, sample, xs, rows, H, E, K, I, L, budget_s: float, repeats: int = 3, dtypes=None):
    """The reference's CPU expert path (two passes, int8 activations, AVX2 integer dots;
    oracle/cpu_baseline.c) plus the router and top-k, on the sampled layers, one token at a
    time, on a persistent pool of every physical core (at most 16).  The sample (tokens x
    layers) is sized so one pass takes about budget_s / repeats; it runs `repeats` times
    and the median per-token time, scaled to the full stack depth, is reported."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cpu_baseline as CB
    import oracle as O

    threads, phys, logical = cpu_threads()
    pool = CB.Pool(threads)
    dts = dtypes or (O.Q4_K,) * 3
    layers = [(r, (O.stack(g, dts[0], I, H), O.stack(u, dts[1], I, H), O.stack(d, dts[2], H, I)))
              for r, (g, u, d) in sample]
    x_all = xs.download(np.uint16).reshape(-1, rows, H)

    def one_token(i):
        x = O.from_bf16(x_all[i % x_all.shape[0]])
        for r, st in layers:
            ids, w = O.topk(O.router_logits(x, r), K, O.ROUTE_SOFTMAX_TOPK_RENORM)
            y = pool.fused_moe_decode(*st, x, ids, w)
            x = O.from_bf16(O.to_bf16(x + y))

    # size the sample: tokens whose pass takes about budget_s / repeats
    t0 = time.perf_counter()
    one_token(0)
    per_tok = max(time.perf_counter() - t0, 1e-4)
    tokens = int(max(3, min(200, budget_s / repeats / per_tok)))
    runs = []
    for rep in range(repeats):
        t0 = time.perf_counter()
        for i in range(tokens):
            one_token(i)
        runs.append((time.perf_counter() - t0) / tokens)
    pool.close()
    med = float(np.median(runs))
    tok_s = rows / (med / len(layers) * L)
    log(f"cpu baseline: {tokens} tokens x {len(layers)} layers, {repeats} runs "
        f"{', '.join(f'{r * 1e3:.2f}' for r in runs)} ms/token -> median {tok_s:.3f} tok/s at {L} layers "
        f"({threads} threads; lscpu physical cores {phys}, logical {logical})")
    return {"value": round(tok_s, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "physical_cores": phys, "logical_cores": logical,
            "sample": f"{tokens} tokens x {len(layers)} of {L} layers (bs{rows}; router, top-{K} and the "
                      f"two-pass expert path with int8 activations and AVX2 integer dots), median of "
                      f"{repeats} runs, scaled to {L} layers"}


def run_cache25(args) -> int:
    """Qwen3-30B-A3B-shaped 48-layer decode, bs1, with 32 of 128 experts cached per layer.

    Routing adds a Zipf(1.1) bias b_e = ln p_e (p_e ~ rank(e)^-1.1 over a fixed random
    rank permutation per layer) to the router logits.  Each layer runs the partial-cache
    step (include/naiwa_cached.h): device routing, top-k read-back, the host policy's
    hit/miss split, misses streamed from pinned host stacks into the 16-slot staging ring
    (pcie_frac 1), the expert kernel over cache + ring slots, one promotion per layer per
    step (min 4 sightings).  Caches start with each layer's 32 most popular experts, seeded from an
    expert profile (include/naiwa_policy.h) written from the bias ranks."""
    import naiwa_moe as nm

    if nm.device_count() < 1:
        log("no HIP device")
        return 1
    L, H, E, K, I, rows, usable = args.layers, 2048, 128, 8, 768, 1, 32
    steps = args.steps if args.steps != 50 else 256
    warmup = args.warmup if args.warmup != 5 else 8
    dt = (nm.Q4_K,) * 3
    t0 = time.time()
    compute, copy = nm.Stream(), nm.Stream()
    ring = nm.policy.StagingRing()
    proj = I * (H // Q4K_BLOCK) * Q4K_BYTES
    tmp = nm.DeviceBuffer(E * proj)
    layers, keep, ranking = [], [], []
    for l in range(L):
        # each expert's gate | up | down adjacent in host memory and in its slot: one range per upload
        stacks = nm.HostExpertStacks(E, H, I, dt, interleaved=True)
        for t in range(3):
            nm.synth(nm.Q4_K, 1000 + 8 * l + t, E * proj * 256 // Q4K_BYTES, tmp, 0.0, 0.02, stream=compute.handle)
            nm._lib.check(nm.lib().naiwa_memcpy_2d(stacks.ptrs[t], stacks.stride, tmp.ptr, proj, proj, E,
                                                   compute.handle), "memcpy_2d")
            compute.sync()
        router = nm.DeviceBuffer(E * H * 4)
        nm.synth(nm.F32, 1000 + 8 * l + 3, E * H, router, 0.0, 0.02, stream=compute.handle)
        ranks = np.random.default_rng(5000 + l).permutation(E) + 1
        p = ranks.astype(np.float64) ** -1.1
        bias = np.log(p / p.sum()).astype(np.float32)
        bias_d = nm.DeviceBuffer.from_array(bias)
        banks = nm.LayerBanks(usable + ring.length, H, I, dt, contiguous=True)
        layer = nm.policy.CachedLayer(router, banks, stacks, E, K, usable, ring, copy.handle,
                                      mode=nm.ROUTE_SOFTMAX_TOPK_RENORM, router_bias=bias_d)
        layer.set_upload_sync(nm.policy.UPLOAD_SYNC_POLL if args.upload_sync == "poll"
                              else nm.policy.UPLOAD_SYNC_EVENT)
        layer.set_upload_path(nm.policy.UPLOAD_PATH_DMA if args.upload_path == "dma"
                              else nm.policy.UPLOAD_PATH_KERNEL)
        ranking += [(l, int(e)) for e in np.argsort(ranks)]
        layers.append(layer)
        keep += [stacks, router, bias_d, banks]
    del tmp
    # the caches start hot from an expert profile: each layer's experts by popularity
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "profile.bin")
        nm.policy.write_profile(path, ranking, L, E, slots=L * usable)
        profile = nm.policy.ExpertProfile(path, L, E)
    seeded = sum(layer.seed(profile.layer(l)) for l, layer in enumerate(layers))
    log(f"cache25: {L} layers, {usable}/{E} cached + {ring.length} ring slots, pinned host stacks "
        f"{L * 3 * E * proj / 1e9:.1f} GB, {seeded} slots seeded from {profile.source}, set-up {time.time() - t0:.1f}s")
    xs = nm.DeviceBuffer((warmup + steps) * rows * H * 2)
    nm.synth(nm.BF16, 999, (warmup + steps) * rows * H, xs, 0.0, 1.0, stream=compute.handle)
    x = nm.DeviceBuffer(rows * H * 2)
    y = nm.DeviceBuffer(rows * H * 4)
    lib = nm.lib()

    swaps = args.lookahead_swaps
    ahead_tot = {"loads": 0, "swaps": 0, "predicted": 0, "resident": 0}

    def step(i: int) -> dict:
        lib.naiwa_memcpy_d2d(x.ptr, xs.ptr + i * rows * H * 2, rows * H * 2, compute.handle)
        # every layer's partial-cache step and residual in order (with swaps >= 0 each layer
        # also predicts the next layer's experts from its activation and loads them)
        info, ahead = nm.policy.CachedLayer.stack_forward(layers, x, rows, y, pcie_frac=args.pcie_frac,
                                                          promote_cap=1, min_hits=4, lookahead_swaps=swaps,
                                                          stream=compute.handle)
        for k_ in ahead_tot:
            ahead_tot[k_] += ahead[k_]
        return {k_: info[k_] for k_ in ("hits", "staged", "staged_experts", "promoted", "pcie_bytes", "cpu")}

    for i in range(warmup):
        step(i)
    compute.sync()
    copy.sync()
    nm.policy.stats(reset=True)
    for k_ in ahead_tot:
        ahead_tot[k_] = 0
    tot = {"hits": 0, "staged": 0, "staged_experts": 0, "promoted": 0, "pcie_bytes": 0, "cpu": 0}
    e0, e1 = nm.Event(), nm.Event()
    e0.record(compute.handle)
    start = time.perf_counter()
    for s in range(steps):
        r = step(warmup + s)
        for k_ in tot:
            tot[k_] += r[k_]
    e1.record(compute.handle)
    compute.sync()
    wall = time.perf_counter() - start
    ms = e0.elapsed_ms(e1)
    tok_s = rows * steps / (ms / 1e3)
    pairs = tot["hits"] + tot["staged"] + tot["cpu"]
    pcie_gbs = tot["pcie_bytes"] / (ms / 1e3) / 1e9
    log(f"cache25 ({args.upload_sync}, {args.upload_path} uploads, pcie_frac {args.pcie_frac}): {ms / steps * 1e3:.1f} us/step, "
        f"{tok_s:.1f} tok/s, hit rate {tot['hits'] / pairs:.3f}, "
        f"{tot['staged_experts'] / (steps * L):.2f} staged experts/layer/token, "
        f"{tot['cpu'] / (steps * L):.2f} CPU pairs/layer/token, {tot['promoted']} promotions, "
        f"PCIe {pcie_gbs:.1f} GB/s, wall {wall:.2f}s")
    if swaps >= 0:
        log(f"cache25 lookahead (swaps {swaps}/row): {ahead_tot['loads']} loads, {ahead_tot['swaps']} swaps, "
            f"{ahead_tot['resident'] / max(ahead_tot['predicted'], 1):.3f} of predictions already resident")
    result = {
        "metric": "MoE decode tok/s, 25% expert cache, Zipf(1.1) routing (Qwen3-30B-A3B shape, Q4_K)",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms / steps, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 x Q4_K (f32 accumulate)", "data": "synthetic (device-generated N(0,0.02) Q4_K experts in pinned host stacks)",
        "config": {"workload": "Qwen3-30B-A3B-shaped MoE stack decode, bs1, 32/128 experts cached per layer, "
                               "Zipf(1.1) routing bias, the pcie_frac share of misses staged over PCIe "
                               "(16-slot ring), the rest on the CPU",
                   "layers": L, "hidden": H, "experts": E, "top_k": K, "intermediate": I, "cached": usable,
                   "ring": ring.length, "pcie_frac": args.pcie_frac, "upload_sync": args.upload_sync, "upload_path": args.upload_path,
                   "promote_cap": 1,
                   "lookahead_swaps": swaps if swaps >= 0 else None, "parallelism": "none (1 GPU)"},
        "cache": {"hit_rate": round(tot["hits"] / pairs, 4),
                  "cpu_pairs_per_layer_token": round(tot["cpu"] / (steps * L), 3),
                  "staged_experts_per_layer_token": round(tot["staged_experts"] / (steps * L), 3),
                  "promotions": tot["promoted"], "pcie_bytes": tot["pcie_bytes"],
                  "lookahead": dict(ahead_tot) if swaps >= 0 else None,
                  "stats": nm.policy.stats()},
        "roofline": {"bound": "pcie", "achieved": round(pcie_gbs, 2), "peak": 64.0, "unit": "GB/s",
                     "frac": round(pcie_gbs / 64.0, 4), "traffic": None},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def run_prefill_stream(args) -> int:
    """The DeepSeek-V2-Lite-shaped prefill of --workload prefill with every expert (64 routed
    + 2 shared per layer) in pinned host memory: each layer's stacks are uploaded into a ring
    of device layer buffers (include/naiwa_prefill.h) while the previous layer computes.  The
    memory plan picks the chunk (up to the 2048 prompt tokens) and the depth from the free
    device memory (or --budget-gb).  One step = the 2048-token prefill through the 26 layers."""
    import naiwa_moe as nm
    from naiwa_moe import prefill as P

    if nm.device_count() < 1:
        log("no HIP device")
        return 1
    L = 26 if args.layers == 48 else args.layers
    H, E, S_, K, I, tokens = 2048, 64, 2, 6, 1408, 2048
    steps = args.steps if args.steps != 50 else 3
    warmup = args.warmup if args.warmup != 5 else 1
    dt = (nm.Q4_K, nm.Q4_K, nm.Q8_0)
    compute, copy = nm.Stream(), nm.Stream()
    t0 = time.time()
    stacks, routers = [], []
    scratch = nm.DeviceBuffer(max((E + S_) * nm.row_bytes(d, k) * n for d, n, k in ((dt[0], I, H), (dt[2], H, I))))
    for l in range(L):
        hs = nm.HostExpertStacks(E + S_, H, I, dt)
        for t, (n, k) in enumerate(((I, H), (I, H), (H, I))):
            nbytes = hs.expert_bytes[t] * (E + S_)
            for e in range(E + S_):
                nm.synth(dt[t], 3000 + 8 * l + t, n * k, scratch.ptr + e * hs.expert_bytes[t], 0.0,
                         DOWN_STD_DEEPSEEK if t == 2 else 0.02, offset=e * n * k, stream=compute.handle)
            nm.lib().naiwa_memcpy_d2h(hs.buffers[t].ptr, scratch.ptr, nbytes, compute.handle)
            compute.sync()
        router = nm.DeviceBuffer(E * H * 4)
        nm.synth(nm.F32, 3000 + 8 * l + 3, E * H, router, 0.0, 0.02, stream=compute.handle)
        stacks.append(hs)
        routers.append(router)
    del scratch
    layer_bytes = (E + S_) * sum(stacks[0].expert_bytes)
    free, total = nm.mem_info()
    budget = int(args.budget_gb * (1 << 30)) if args.budget_gb > 0 else free
    planned = P.plan_with_lend_depth(budget, layer_bytes, tokens, False, 0, 0, P.MAX_DEPTH)
    if planned is None:
        log(f"prefill-stream: nothing fits in {budget / 2**30:.1f} GiB")
        return 1
    stride, chunk = planned
    depth = args.depth if args.depth > 0 else stride
    ps = P.PrefillStream(stacks, H, I, dt, depth, copy.handle)
    log(f"prefill-stream: {L} layers x {E}+{S_} experts in pinned host memory "
        f"({L * layer_bytes / 1e9:.1f} GB, {layer_bytes / 2**20:.0f} MiB a layer), plan on "
        f"{budget / 2**30:.1f} GiB: chunk {chunk}, stride {stride}; running depth {depth}; set-up {time.time() - t0:.1f}s")
    chunk = min(chunk, tokens)
    xs = nm.DeviceBuffer(tokens * H * 2)
    nm.synth(nm.BF16, 998, tokens * H, xs, 0.0, 1.0, stream=compute.handle)
    x = nm.DeviceBuffer(tokens * H * 2)
    ids, w = nm.DeviceBuffer(chunk * K * 4), nm.DeviceBuffer(chunk * K * 4)
    sid = nm.DeviceBuffer.from_array(np.tile(np.array([E, E + 1], dtype=np.uint32), (chunk, 1)))
    sw = nm.DeviceBuffer.from_array(np.ones((chunk, S_), dtype=np.float32))
    y = nm.DeviceBuffer(chunk * H * 4)
    compute.sync()
    lib = nm.lib()

    def step() -> None:
        lib.naiwa_memcpy_d2d(x.ptr, xs.ptr, tokens * H * 2, compute.handle)
        for c0 in range(0, tokens, chunk):
            T = min(chunk, tokens - c0)
            xc = x.ptr + c0 * H * 2
            for l in range(L):
                nm.router_topk(xc, nm.BF16, routers[l], T, H, E, K, ids, w, mode=nm.ROUTE_SOFTMAX_TOPK,
                               stream=compute.handle)
                ps.forward(l, xc, ids, w, T, K, y, stream=compute.handle)
                ps.forward(l, xc, sid, sw, T, S_, y, accumulate=True, stream=compute.handle)
                nm._lib.check(lib.naiwa_residual_add_bf16(xc, y.ptr, T * H, compute.handle), "residual")

    for _ in range(warmup):
        step()
    compute.sync()
    before = ps.stats()
    e0, e1 = nm.Event(), nm.Event()
    e0.record(compute.handle)
    for _ in range(steps):
        step()
    e1.record(compute.handle)
    compute.sync()
    ms = e0.elapsed_ms(e1) / steps
    health = activation_health(x, tokens * H)
    if health["nonfinite"]:
        log(f"activations overflowed: {health}")
        return 1
    after = ps.stats()
    moved = (after["upload_bytes"] - before["upload_bytes"]) / steps
    tok_s = tokens / (ms / 1e3)
    pcie = moved / (ms / 1e3) / 1e9
    log(f"prefill-stream: {ms:.2f} ms per {tokens}-token prefill, {tok_s:.0f} tok/s, {moved / 1e9:.2f} GB uploaded "
        f"a step, {pcie:.1f} GB/s ({pcie / 64.0 * 100:.0f}% of 64 GB/s PCIe 5.0 x16)")
    result = {
        "metric": "MoE prefill tok/s with host-resident experts (DeepSeek-V2-Lite shape, layer stream)",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 x Q4_K/Q8_0 (f32 accumulate)",
        "data": "synthetic (device-generated Q4_K/Q8_0 experts in pinned host stacks: gate/up N(0,0.02), "
                f"down N(0,{DOWN_STD_DEEPSEEK}); N(0,1) bf16 tokens)",
        "config": {"workload": "DeepSeek-V2-Lite-shaped MoE prefill, 26 layers, 64 routed top-6 + 2 shared experts "
                               "streamed from pinned host memory per layer, 2048 tokens",
                   "layers": L, "chunk": chunk, "depth": depth, "plan_stride": stride,
                   "plan_budget_gib": round(budget / 2**30, 1), "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "pcie", "achieved": round(pcie, 2), "peak": 64.0, "unit": "GB/s",
                     "frac": round(pcie / 64.0, 4), "traffic": None},
        "activations_after_last_layer": health,
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def run_mixtral(args) -> int:
    """Mixtral-8x7B-shaped MoE (32 layers, H 4096, 8 experts top-2, I 14336, Q4_K, uniform-random
    router): decode steps at batch 1, 16 and 64 with every expert resident (router, expert decode and
    residual per layer, layered launches), the 4096-token prefill in one chunk (grouped MFMA GEMMs), and
    batch-1 decode with 4 of 8 experts cached per layer (misses staged from pinned host stacks).  The
    JSON line's value is the batch-1 resident decode; the other parts are reported beside it."""
    import naiwa_moe as nm

    if nm.device_count() < 1:
        log("no HIP device")
        return 1
    L = 32 if args.layers == 48 else args.layers
    H, E, K, I = 4096, 8, 2, 14336
    dt = (nm.Q4_K,) * 3
    stream = nm.Stream()
    t0 = time.time()
    layers, keep = [], []
    proj = I * (H // Q4K_BLOCK) * Q4K_BYTES
    expert_bytes = 3 * proj
    for l in range(L):
        banks = nm.LayerBanks(E, H, I, dt)
        for t, bank in enumerate((banks.gate, banks.up, banks.down)):
            nm.synth(nm.Q4_K, 6000 + 8 * l + t, E * bank.n * bank.k, bank.base, 0.0,
                     DOWN_STD_MIXTRAL if t == 2 else 0.02, stream=stream.handle)
        router = nm.DeviceBuffer(E * H * 4)
        nm.synth(nm.F32, 6000 + 8 * l + 3, E * H, router, 0.0, 0.02, stream=stream.handle)
        layers.append(nm.layer_desc(router, banks))
        keep.append((banks, router))
    arr = (nm._lib.Layer * L)(*layers)
    max_rows = 4096
    xs = nm.DeviceBuffer(max_rows * H * 2)
    nm.synth(nm.BF16, 998, max_rows * H, xs, 0.0, 1.0, stream=stream.handle)
    stream.sync()
    log(f"mixtral: {L} layers x {E} experts ({L * E * expert_bytes / 1e9:.1f} GB Q4_K) in {time.time() - t0:.1f}s")
    lib = nm.lib()
    out = {}

    # ---- resident decode at batch 1 / 16 / 64 ----
    for rows in (1, 16, 64):
        x = nm.DeviceBuffer(rows * H * 2)
        ids_d, w_d = nm.DeviceBuffer(L * rows * K * 4), nm.DeviceBuffer(L * rows * K * 4)
        steps = max(3, min(args.steps, 20))

        def step(i):
            lib.naiwa_memcpy_d2d(x.ptr, xs.ptr + (i * rows % (max_rows - rows + 1)) * H * 2, rows * H * 2,
                                 stream.handle)
            nm.stack_decode(arr, x, rows, H, E, K, mode=nm.ROUTE_TOPK_SOFTMAX, ids_out=ids_d, w_out=w_d,
                            fused=False, stream=stream.handle)
        for i in range(2):
            step(i)
        stream.sync()
        e0, e1 = nm.Event(), nm.Event()
        e0.record(stream.handle)
        for i in range(steps):
            step(2 + i)
        e1.record(stream.handle)
        stream.sync()
        ms = e0.elapsed_ms(e1) / steps
        health = activation_health(x, rows * H)
        if health["nonfinite"]:
            log(f"mixtral decode bs{rows}: activations overflowed: {health}")
            return 1
        ids = ids_d.download(np.uint32).reshape(L, rows, K)
        distinct = sum(len(np.unique(ids[l])) for l in range(L))
        alg = distinct * expert_bytes + L * (E * H * 4 + rows * H * 4)
        gbs = alg / (ms / 1e3) / 1e9
        out[f"decode_bs{rows}"] = {"tok_s": round(rows / (ms / 1e3), 2), "ms_per_step": round(ms, 3),
                                   "distinct_experts_per_layer": round(distinct / L, 2),
                                   "activation_absmax": health["absmax"],
                                   "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"mixtral decode bs{rows}: {ms:.3f} ms/step, {rows / (ms / 1e3):.1f} tok/s, {distinct / L:.2f} "
            f"experts/layer, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM peak)")

    # ---- the 4096-token prefill, one chunk per layer ----
    T = 4096
    x = nm.DeviceBuffer(T * H * 2)
    ids, w = nm.DeviceBuffer(T * K * 4), nm.DeviceBuffer(T * K * 4)
    y = nm.DeviceBuffer(T * H * 4)

    def prefill():
        lib.naiwa_memcpy_d2d(x.ptr, xs.ptr, T * H * 2, stream.handle)
        for banks, router in keep:
            nm.router_topk(x, nm.BF16, router, T, H, E, K, ids, w, mode=nm.ROUTE_TOPK_SOFTMAX, stream=stream.handle)
            nm.moe_prefill(banks, x, ids, w, T, K, y, stream=stream.handle, residual=True)
    prefill()
    stream.sync()
    e0, e1 = nm.Event(), nm.Event()
    e0.record(stream.handle)
    reps = 2
    for _ in range(reps):
        prefill()
    e1.record(stream.handle)
    stream.sync()
    ms = e0.elapsed_ms(e1) / reps
    health = activation_health(x, T * H)
    if health["nonfinite"]:
        log(f"mixtral prefill: activations overflowed: {health}")
        return 1
    flop = 6.0 * H * I * K * T * L
    tflops = flop / (ms / 1e3) / 1e12
    out["prefill_4096"] = {"tok_s": round(T / (ms / 1e3), 1), "ms": round(ms, 2), "tflops": round(tflops, 1),
                           "mfma_frac": round(tflops / 2500.0, 4), "flop": flop,
                           "activation_absmax": health["absmax"]}
    log(f"mixtral prefill {T} tokens: {ms:.1f} ms, {T / (ms / 1e3):.0f} tok/s, {tflops:.0f} TFLOP/s "
        f"({tflops / 2500 * 100:.1f}% of 2.5 PFLOP/s dense)")
    del x, ids, w, y

    # ---- batch-1 decode with 4 of 8 experts cached per layer ----
    usable = 4
    copy = nm.Stream()
    ring = nm.policy.StagingRing()
    cached, ckeep = [], []
    for l, (banks, router) in enumerate(keep[: min(L, args.cache_layers)]):
        hs = nm.HostExpertStacks(E, H, I, dt, interleaved=True)
        for t, bank in enumerate((banks.gate, banks.up, banks.down)):
            nm._lib.check(lib.naiwa_memcpy_2d(hs.ptrs[t], hs.stride, bank.base, bank.stride, proj, E, stream.handle),
                          "memcpy_2d")
        stream.sync()
        cb = nm.LayerBanks(usable + ring.length, H, I, dt, contiguous=True)
        layer = nm.policy.CachedLayer(router, cb, hs, E, K, usable, ring, copy.handle, mode=nm.ROUTE_TOPK_SOFTMAX)
        layer.seed(list(range(usable)))
        cached.append(layer)
        ckeep += [hs, cb]
    Lc = len(cached)
    xc = nm.DeviceBuffer(H * 2)
    yc = nm.DeviceBuffer(H * 4)
    tot = {"hits": 0, "staged": 0, "staged_experts": 0, "pcie_bytes": 0}

    def cstep(i):
        lib.naiwa_memcpy_d2d(xc.ptr, xs.ptr + i * H * 2, H * 2, stream.handle)
        for layer in cached:
            info = layer.forward(xc, 1, yc, pcie_frac=1.0, promote_cap=1, min_hits=4, stream=stream.handle)
            nm._lib.check(lib.naiwa_residual_add_bf16(xc.ptr, yc.ptr, H, stream.handle), "residual")
            for k_ in tot:
                tot[k_] += info[k_]
    cstep(0)
    stream.sync()
    for k_ in tot:
        tot[k_] = 0
    csteps = 4
    e0, e1 = nm.Event(), nm.Event()
    e0.record(stream.handle)
    for i in range(csteps):
        cstep(1 + i)
    e1.record(stream.handle)
    stream.sync()
    ms = e0.elapsed_ms(e1) / csteps
    health = activation_health(xc, H)
    if health["nonfinite"]:
        log(f"mixtral 4-of-8 cache: activations overflowed: {health}")
        return 1
    pcie = tot["pcie_bytes"] / csteps / (ms / 1e3) / 1e9
    out["cache_4of8_bs1"] = {"layers": Lc, "ms_per_token": round(ms, 2), "tok_s_at_32_layers": round(1e3 / (ms * 32 / Lc), 3),
                             "hit_rate": round(tot["hits"] / max(1, tot["hits"] + tot["staged"]), 3),
                             "staged_experts_per_layer_token": round(tot["staged_experts"] / (csteps * Lc), 3),
                             "pcie_gbs": round(pcie, 2), "pcie_frac": round(pcie / 64.0, 4)}
    log(f"mixtral 4-of-8 cache, bs1, {Lc} layers: {ms:.2f} ms/token, hit rate "
        f"{out['cache_4of8_bs1']['hit_rate']:.3f}, PCIe {pcie:.1f} GB/s ({pcie / 64 * 100:.0f}% of 64 GB/s)")
    del cached, ckeep

    cpu = None
    if not args.no_cpu_baseline:
        sample = []
        for banks, router in keep[:1]:
            get = lambda b: b.buffer.download(np.uint8).reshape(E, b.n, -1)
            sample.append((router.download(np.float32).reshape(E, H), (get(banks.gate), get(banks.up),
                                                                     get(banks.down))))
        cpu = cpu_baseline(nm, sample, xs, 1, H, E, K, I, L, args.cpu_seconds)
    d1 = out["decode_bs1"]
    result = {
        "metric": "MoE decode tok/s @bs1 (Mixtral-8x7B shape, Q4_K, all experts resident)",
        "value": d1["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": max(3, min(args.steps, 20)), "warmup": 2,
        "ms_per_step": d1["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 x Q4_K (f32 accumulate)",
        "data": f"synthetic (device-generated Q4_K experts: gate/up N(0,0.02), down N(0,{DOWN_STD_MIXTRAL}); "
                "N(0,1) bf16 tokens)",
        "config": {"workload": "Mixtral-8x7B-shaped MoE stack: decode bs 1/16/64 (all resident), 4096-token "
                               "prefill, bs1 decode with 4 of 8 experts cached", "layers": L, "hidden": H,
                   "experts": E, "top_k": K, "intermediate": I, "weights": "Q4_K", "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": d1["hbm_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": d1["hbm_frac"], "traffic": None, "kernel": "layered decode step (bs1)"},
        "parts": out,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def run_doorbell(args) -> int:
    """Doorbell round trip: the host release-stores seq = i into mapped memory, one
    persistent device wave (doorbell_poll_serve) observes it and release-stores ack = i,
    the host observes the ack.  Median and p99 over --db-iters rings (the reference's
    harness reports 31.7 us per iteration with a stream sync each, docs/worklogs/m0.md:43)."""
    import ctypes as C

    import naiwa_moe as nm

    if nm.device_count() < 1:
        log("no HIP device")
        return 1
    lib = nm.lib()
    n = args.db_iters
    host = C.c_void_p()
    nm._lib.check(lib.doorbell_alloc_mapped(C.byref(host), 256), "doorbell_alloc_mapped")
    dev = C.c_void_p()
    lib.doorbell_get_device_ptr(host, C.byref(dev))
    if not dev.value:
        log("no device view of the mapped doorbell")
        return 1
    seq_h, ack_h = host.value, host.value + 128
    seq_d, ack_d = dev.value, dev.value + 128
    stream = nm.Stream()
    before = C.c_uint32()
    lib.naiwa_doorbell_timeouts(C.byref(before))
    nm._lib.check(lib.doorbell_poll_serve(seq_d, ack_d, 1, n, stream.handle), "doorbell_poll_serve")
    lat = np.zeros(n)
    for i in range(1, n + 1):
        t0 = time.perf_counter_ns()
        lib.naiwa_host_store_release_u32(seq_h, i)
        if lib.naiwa_host_wait_ge(ack_h, i, 2_000_000, 50) != 0:
            log(f"doorbell: ack {i} not seen within 2 s")
            lib.naiwa_host_store_release_u32(seq_h, n)  # let the wave finish its rings
            stream.sync()
            return 1
        lat[i - 1] = (time.perf_counter_ns() - t0) / 1e3
    stream.sync()
    after = C.c_uint32()
    lib.naiwa_doorbell_timeouts(C.byref(after))
    # the reference's style: one launch and a stream sync per round trip
    m = 200
    sync_lat = np.zeros(m)
    for i in range(m):
        t0 = time.perf_counter_ns()
        nm._lib.check(lib.doorbell_poll_serve(seq_d, ack_d, n, 1, stream.handle), "doorbell_poll_serve")
        stream.sync()
        sync_lat[i] = (time.perf_counter_ns() - t0) / 1e3
    lib.doorbell_free_host(host)
    med, p99 = float(np.median(lat)), float(np.percentile(lat, 99))
    log(f"doorbell round trip over {n} rings: median {med:.2f} us, p99 {p99:.2f} us, max {lat.max():.1f} us; "
        f"launch + stream sync per trip: median {np.median(sync_lat):.1f} us; timeouts {after.value - before.value}")
    result = {
        "metric": "doorbell round-trip latency (host ring -> persistent device wave -> host), median",
        "value": round(med, 3), "unit": "us", "n_gpus": 1, "steps": n, "warmup": 0,
        "ms_per_step": round(med / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "u32", "data": "synthetic",
        "config": {"workload": "doorbell_poll_serve round trips over fine-grained mapped host memory",
                   "iterations": n},
        "p99_us": round(p99, 3), "max_us": round(float(lat.max()), 2),
        "launch_and_sync_us_median": round(float(np.median(sync_lat)), 2),
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def run_prefill(args) -> int:
    """DeepSeek-V2-Lite-shaped MoE prefill: 26 MoE layers, H 2048, 64 routed experts top-6
    (softmax without renormalisation) + 2 shared experts, I 1408, gate/up Q4_K, down Q8_0.
    2048 tokens in 4 chunks of 512; per layer and chunk: device routing, the routed experts
    and the shared experts (weight 1, after each token's routed pairs) in one grouped MFMA
    call, residual.  One
    step = the whole 2048-token prefill through the MoE layers."""
    import naiwa_moe as nm

    if nm.device_count() < 1:
        log("no HIP device")
        return 1
    L = 26 if args.layers == 48 else args.layers
    H, E, S_, K, I, T, chunks = 2048, 64, 2, 6, 1408, 512, 4
    steps = args.steps if args.steps != 50 else 3
    warmup = args.warmup if args.warmup != 5 else 1
    dt = (nm.Q4_K, nm.Q4_K, nm.Q8_0)
    stream = nm.Stream()
    t0 = time.time()
    layers, keep = [], []
    for l in range(L):
        banks = nm.LayerBanks(E + S_, H, I, dt)
        for t, bank in enumerate((banks.gate, banks.up, banks.down)):
            for e in range(E + S_):
                nm.synth(dt[t], 3000 + 8 * l + t, bank.n * bank.k, bank.base + e * bank.stride, 0.0,
                         DOWN_STD_DEEPSEEK if t == 2 else 0.02, offset=e * bank.n * bank.k, stream=stream.handle)
        router = nm.DeviceBuffer(E * H * 4)
        nm.synth(nm.F32, 3000 + 8 * l + 3, E * H, router, 0.0, 0.02, stream=stream.handle)
        layers.append((banks, router))
        keep.append((banks, router))
    tokens = chunks * T
    xs = nm.DeviceBuffer(tokens * H * 2)
    nm.synth(nm.BF16, 998, tokens * H, xs, 0.0, 1.0, stream=stream.handle)
    x = nm.DeviceBuffer(tokens * H * 2)
    # one grouped call per layer: each token's K routed pairs, then its S_ shared experts
    # (slots E.., weight 1), so the shared GEMM tiles run in the routed launch and the
    # ordered combine adds them after the routed pairs, as a second accumulating call would
    KA = K + S_
    ids_all = nm.DeviceBuffer.from_array(np.tile(np.concatenate([np.zeros(K), np.arange(E, E + S_)]).astype(np.uint32),
                                                 (T, 1)))
    w_all = nm.DeviceBuffer.from_array(np.tile(np.concatenate([np.zeros(K), np.ones(S_)]).astype(np.float32), (T, 1)))
    y = nm.DeviceBuffer(T * H * 4)
    stream.sync()
    log(f"prefill: {L} layers x {E}+{S_} experts synthesized in {time.time() - t0:.1f}s")
    lib = nm.lib()

    def step() -> None:
        lib.naiwa_memcpy_d2d(x.ptr, xs.ptr, tokens * H * 2, stream.handle)
        for c in range(chunks):
            xc = x.ptr + c * T * H * 2
            for banks, router in layers:
                # the routed experts straight into columns 0..K-1 of the (routed | shared) table
                nm.router_topk(xc, nm.BF16, router, T, H, E, K, ids_all, w_all, mode=nm.ROUTE_SOFTMAX_TOPK,
                               stream=stream.handle, ld=KA)
                nm.moe_prefill(banks, xc, ids_all, w_all, T, KA, y, stream=stream.handle, residual=True)

    for _ in range(warmup):
        step()
    stream.sync()
    if args.calibrate_copy:
        calibration_copy(nm, args.calibrate_copy, stream)
    e0, e1 = nm.Event(), nm.Event()
    e0.record(stream.handle)
    for _ in range(steps):
        step()
    e1.record(stream.handle)
    stream.sync()
    ms = e0.elapsed_ms(e1) / steps
    health = activation_health(x, tokens * H)
    if health["nonfinite"]:
        log(f"prefill: activations overflowed: {health}")
        return 1
    flop = 6.0 * H * I * (K + S_) * tokens * L   # 2 flop/MAC x (gate + up + down)
    tflops = flop / (ms / 1e3) / 1e12
    tok_s = tokens / (ms / 1e3)
    log(f"prefill: {ms:.2f} ms per {tokens}-token prefill, {tok_s:.0f} tok/s, {tflops:.1f} TFLOP/s "
        f"({tflops / 2500 * 100:.1f}% of 2.5 PFLOP/s bf16 dense)")
    # The grouped call's roofline: a 512-token chunk's 3072 routed + 1024 shared pairs touch
    # every expert of the layer (66 x 6,307,840 B of weights) for 70.9 GFLOP, 170 flop/B,
    # below the ridge of 2.5 PFLOP/s / 8 TB/s = 312 flop/B: the call is HBM-bound.  Each
    # layer-chunk's naiwa_moe_prefill is timed with events on its stream (one more pass).
    per_expert = (2 * I * nm.row_bytes(dt[0], H) + H * nm.row_bytes(dt[2], I))
    ev = [(nm.Event(), nm.Event()) for _ in range(chunks * L)]
    lib.naiwa_memcpy_d2d(x.ptr, xs.ptr, tokens * H * 2, stream.handle)
    distinct = []
    for c in range(chunks):
        xc = x.ptr + c * T * H * 2
        for li, (banks, router) in enumerate(layers):
            nm.router_topk(xc, nm.BF16, router, T, H, E, K, ids_all, w_all, mode=nm.ROUTE_SOFTMAX_TOPK,
                           stream=stream.handle, ld=KA)
            a, b = ev[c * L + li]
            a.record(stream.handle)
            nm.moe_prefill(banks, xc, ids_all, w_all, T, KA, y, stream=stream.handle, residual=True)
            b.record(stream.handle)
            if li == 0 and c == 0:
                stream.sync()
                distinct.append(len(np.unique(ids_all.download(np.uint32).reshape(T, KA)[:, :K])))
    stream.sync()
    call_ms = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
    n_exp = (distinct[0] if distinct else E) + S_
    call_bytes = n_exp * per_expert + T * H * 2 + T * KA * 8 + T * H * 4
    hbm = call_bytes / (call_ms / 1e3) / 1e9
    call_flop = 6.0 * H * I * KA * T
    log(f"prefill call (one layer-chunk): {call_ms * 1e3:.1f} us, {call_bytes / 1e6:.1f} MB ({n_exp} experts), "
        f"{hbm:.0f} GB/s = {hbm / HBM_PEAK_GBS * 100:.1f}% of HBM peak; {call_flop / (call_ms / 1e3) / 1e12:.0f} TFLOP/s")
    result = {
        "metric": "MoE prefill tok/s (DeepSeek-V2-Lite shape, 2048 tokens in 512-token chunks)",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 x Q4_K/Q8_0 (f32 accumulate)",
        "data": f"synthetic (device-generated Q4_K/Q8_0 experts: gate/up N(0,0.02), down N(0,{DOWN_STD_DEEPSEEK}); "
                "N(0,1) bf16 tokens)",
        "config": {"workload": "DeepSeek-V2-Lite-shaped MoE prefill, 26 layers, 64 routed top-6 + 2 shared "
                               "experts, I 1408, gate/up Q4_K, down Q8_0, 2048 tokens in 512-token chunks",
                   "layers": L, "hidden": H, "experts": E, "shared": S_, "top_k": K, "intermediate": I,
                   "chunk": T, "tokens": tokens, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(hbm, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(hbm / HBM_PEAK_GBS, 4), "traffic": profile_traffic(PREFILL_TRAFFIC_PROFILE),
                     "kernel": "naiwa_moe_prefill (one 512-token layer-chunk: gather, tiles, GEMMs, combine)",
                     "bytes_per_launch": call_bytes, "call_avg_us": round(call_ms * 1e3, 2),
                     "mfma_tflops": round(call_flop / (call_ms / 1e3) / 1e12, 2),
                     "mfma_frac": round(call_flop / (call_ms / 1e3) / 1e12 / 2500.0, 4)},
        "activations_after_last_layer": health,
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
