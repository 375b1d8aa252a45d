#!/usr/bin/env python3
"""Benchmark of the GGUF quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): Q4_K batch-1 decode GEMV weight
GB/s at Llama-3-8B layer shapes.  One step = QMatMul::forward (activation Q8_K
quantisation + fused dequant/integer-dot GEMV) for the 7 projections of one
Llama-3-8B layer (q, k, v, o 4096/1024 x 4096; gate, up 14336 x 4096;
down 4096 x 14336), all Q4_K, x ~ N(0, 1) f32 [1, K].  Weights ~ N(0, 0.02)
quantised on the device; 8 distinct layer copies (982 MB) rotate so the
256 MB Infinity Cache cannot hold the working set.  Launches are replayed
from HIP graphs so the host's issue rate does not limit the measurement.

roofline: the step's kernel (the fused quantise + GEMV, one launch per
projection), algorithmic bytes (weights + x + y) per launch over its average
launch time; traffic: HBM bytes per launch from the committed rocprofv3
FETCH_SIZE/WRITE_SIZE summary (profiles/traffic_q4k_gemv.json), when present.

Also reported (extra keys): the dot kernel alone, per-shape kernel times, the
batched MFMA path at M = 512 in TFLOP/s against dense bf16 peak,
the 32-layer Q4_K_M stack in tokens/s at batch 1 and 32, and the
oracle (C restatement of the reference CPU QMatMul) on a bounded sample on the
host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "Q4_K GEMV weight GB/s (% of HBM peak); 8B linear-stack tokens/s at batch 1"

LAYER = [("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096), ("o_proj", 4096, 4096),
         ("gate_proj", 14336, 4096), ("up_proj", 14336, 4096), ("down_proj", 4096, 14336)]
VOCAB = 128256


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=800)
    p.add_argument("--warmup", type=int, default=80)
    p.add_argument("--copies", type=int, default=8, help="distinct weight copies rotated per step")
    p.add_argument("--no-stack", action="store_true", help="skip the 32-layer stack measurement")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-gemm", action="store_true", help="skip the M = 512 MFMA measurement")
    p.add_argument("--no-configs", action="store_true",
                   help="skip configs 1, 3 and 4 (Q8_0 GEMV, Q6_K head / Q5_K batch 1-8, M crossover)")
    p.add_argument("--prefill-profile", action="store_true",
                   help="only run QMatMul::forward for Q4_K gate_proj 14336x4096 and down_proj 4096x14336 at "
                        "the --prefill-ms batch sizes (a short, fixed workload for rocprofv3 counter runs of "
                        "the batched kernels)")
    p.add_argument("--prefill-library", action="store_true",
                   help="with --prefill-profile: also run the library fp16 GEMM (torch.matmul, hipBLASLt) "
                        "on the same shapes and batch sizes, operands already fp16, for counter runs of it")
    p.add_argument("--prefill-ms", default="16,64,512",
                   help="batch sizes M of --prefill-profile, comma-separated (configs[3]: 16,64,512,2048)")
    p.add_argument("--copy-probe", action="store_true",
                   help="first run a 256 MiB device copy 4 times (reference kernel of known size for "
                        "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    p.add_argument("--read-probe", action="store_true",
                   help="only the headline step and the read-only stream over the same bytes (read_floor), "
                        "a short fixed workload for rocprofv3 counter runs of both")
    return p.parse_args()


def copy_probe(torch, dev):
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy probe: 4 x {src.numel() * 4} B copies")
    del src, dst


def read_floor(torch, copies, stream, reps):
    """The same weight bytes as the headline step, read by a plain read-only stream
    (liblbq_probe.so: every wave a contiguous range, four 1 KiB steps in flight) at
    2, 4 and 8 four-wave workgroups per CU, the fastest of the three kept (per launch
    and per step): one launch per projection, the 7 launches of a step and the same
    copies rotated, HIP-graph replay.  The floor the decode kernels are compared with."""
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "lightbulb_amd" / "liblbq_probe.so"))
    lib.lbq_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.lbq_probe_read.restype = ctypes.c_int
    out = torch.zeros(16, dtype=torch.int32, device=stream.device)
    cus = torch.cuda.get_device_properties(stream.device).multi_processor_count

    def read(qm, grid):
        d = qm.qtensor().data
        st = ctypes.c_void_p(torch.cuda.current_stream(d.device).cuda_stream)  # the capturing stream in capture
        if lib.lbq_probe_read(d.data_ptr(), d.numel(), out.data_ptr(), grid, st) != 0:
            raise RuntimeError("lbq_probe_read failed")

    best_step, per, grids = None, {}, {}
    for grid in (2 * cus, 4 * cus, 8 * cus):
        def step(layer, grid=grid):
            for qm in layer:
                read(qm, grid)
        g = StepGraphs(torch, step, copies)
        g.run(len(copies))
        us = g.time(reps * len(copies), stream) * 1e3
        del g
        if best_step is None or us < best_step[0]:
            best_step = (us, grid)
        for i, (name, n, k) in enumerate(LAYER):
            if name in ("k_proj", "up_proj", "o_proj"):
                continue  # same shape as v_proj / gate_proj / q_proj
            gi = capture(torch, lambda i=i: [read(layer[i], grid) for layer in copies])
            timed_graph(torch, gi, 2, stream)
            t = timed_graph(torch, gi, reps, stream) / len(copies) * 1e3
            key = f"{name}_{n}x{k}"
            if key not in per or t < per[key]:
                per[key], grids[key] = round(t, 3), grid
            del gi
    return {"us_per_step": round(best_step[0], 3), "us_per_launch": per, "grid": best_step[1], "grid_per_launch": grids,
            "kernel": "k_probe_read (liblbq_probe.so): loads only, per-wave contiguous 1 KiB steps, 4 in flight; "
                      "fastest of 2, 4 and 8 four-wave workgroups per CU"}


def load_traffic():
    """HBM bytes per launch of the headline kernel, from the committed PMC summary."""
    f = ROOT / "profiles" / "traffic_q4k_gemv.json"
    try:
        return json.loads(f.read_text())
    except (OSError, ValueError):
        return None


def make_weights(torch, qz, dtype, n, k, gen, dev):
    w = torch.randn(n, k, generator=gen, device=dev, dtype=torch.float32).mul_(0.02)
    qt = qz.QTensor.quantize(w, dtype)
    del w
    return qz.QMatMul.from_qtensor(qt)


def timed_graph(torch, graph, reps, stream):
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record(stream)
    for _ in range(reps):
        graph.replay()
    e.record(stream)
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps  # ms per replay


def timed_graph_median(torch, graph, reps, stream):
    """Median over `reps` replays, each bracketed by its own events (ms per replay)."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    for s, e in evs:
        s.record(stream)
        graph.replay()
        e.record(stream)
    torch.cuda.synchronize()
    t = sorted(s.elapsed_time(e) for s, e in evs)
    return t[len(t) // 2]


class StepGraphs:
    """Exactly n steps of a per-copy step function: a graph over all C copies
    (C steps per replay) replayed n // C times, then a graph over the first n % C
    copies once."""

    def __init__(self, torch, step_fn, copies):
        self.torch, self.copies = torch, copies
        self.step_fn = step_fn
        self.full = capture(torch, lambda: [step_fn(c) for c in copies])
        self.part = {}

    def _part(self, r):
        if r not in self.part:
            self.part[r] = capture(self.torch, lambda: [self.step_fn(c) for c in self.copies[:r]])
        return self.part[r]

    def run(self, n):
        q, r = divmod(n, len(self.copies))
        g = self._part(r) if r else None
        for _ in range(q):
            self.full.replay()
        if g is not None:
            g.replay()

    def time(self, n, stream):
        """ms per step over exactly n steps."""
        q, r = divmod(n, len(self.copies))
        if r:
            self._part(r)  # captured outside the timed region
        s = self.torch.cuda.Event(enable_timing=True)
        e = self.torch.cuda.Event(enable_timing=True)
        self.torch.cuda.synchronize()
        s.record(stream)
        self.run(n)
        e.record(stream)
        self.torch.cuda.synchronize()
        return s.elapsed_time(e) / n


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    fn()  # eager pass: sizes scratch and warms the allocator outside capture
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def _cpu_layer_rate(oracle, layer_blocks, xs, budget_s, nthreads, native):
    total_bytes = sum(b.size for b in layer_blocks)
    reps = 0
    t0 = time.perf_counter()
    while True:
        for (name, n, k), blk, x in zip(LAYER, layer_blocks, xs):
            oracle.qmatmul(oracle.Q4_K, blk, n, k, x, nthreads=nthreads, native=native)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 200:
            break
    return total_bytes, reps, el


def cpu_baseline(layer_blocks, xs, budget_s):
    """Oracle (C restatement of the reference CPU QMatMul) on one layer, all host cores: the
    scalar-faithful build (candle's default x86-64 target runs the generic vec_dot), and the same
    source built with -march=native on this host (an upper bound for the CPU path)."""
    import oracle
    nthreads = oracle.nproc()
    total_bytes, reps, el = _cpu_layer_rate(oracle, layer_blocks, xs, budget_s, nthreads, False)
    per = el / reps
    out = {"value": round(total_bytes / per / 1e9, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
           "sample": f"oracle qmatmul (Q8_K activation quant + integer vec_dot, rows split over {nthreads} "
                     f"threads) on the 7 Q4_K projections of one layer at batch 1 ({total_bytes / 1e6:.1f} MB "
                     f"of blocks), {reps} passes in {el:.1f} s; {per * 1e3:.2f} ms per layer; scalar-faithful "
                     f"build (-O3, generic x86-64)",
           "ms_per_step": round(per * 1e3, 3),
           "cpu_model": _cpu_model()}
    try:
        tb, r2, el2 = _cpu_layer_rate(oracle, layer_blocks, xs, budget_s / 2, nthreads, "host")
        out["native"] = {"value": round(tb / (el2 / r2) / 1e9, 3), "unit": "GB/s", "cores": nthreads,
                         "ms_per_step": round(el2 / r2 * 1e3, 3),
                         "sample": f"same oracle built with -O3 -march=native on this host, {r2} passes in {el2:.1f} s"}
    except Exception as e:  # no compiler on the host
        out["native"] = {"value": None, "sample": f"unavailable: {e}"}
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    from lightbulb_amd import _lib
    if not _lib.LIB_PATH.exists():
        from lightbulb_amd import build
        build.build()
    from lightbulb_amd import quantized as qz

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_probe:
        copy_probe(torch, dev)
    if args.prefill_profile:
        prefill_profile(torch, qz, dev, [int(v) for v in args.prefill_ms.split(",")], args.prefill_library)
        return
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x1B1)
    Q4K, Q6K = qz.GgmlDType.Q4K, qz.GgmlDType.Q6K

    # ---------------------------------------------------------------- config 2 weights
    t0 = time.perf_counter()
    copies = [[make_weights(torch, qz, Q4K, n, k, gen, dev) for (_, n, k) in LAYER] for _ in range(args.copies)]
    xs = [torch.randn(1, k, generator=gen, device=dev) for (_, n, k) in LAYER]
    ys = [torch.empty(1, n, device=dev) for (_, n, k) in LAYER]
    layer_bytes = sum(q.qtensor().storage_size_in_bytes() for q in copies[0])
    io_bytes = sum(4 * (n + k) for (_, n, k) in LAYER)
    log(f"weights ready: {args.copies} x {layer_bytes / 1e6:.1f} MB in {time.perf_counter() - t0:.1f} s")

    def full_step(layer):
        for qm, x in zip(layer, xs):
            qm.forward(x)

    # the same step through the grouped entry point (q|k|v and gate|up as the
    # reference's call sites feed them one x): 4 launches instead of 7
    def grouped_step(layer):
        qz.qmatmul_group(layer[0:3], xs[0])
        layer[3].forward(xs[3])
        qz.qmatmul_group(layer[4:6], xs[4])
        layer[6].forward(xs[6])

    # the layer as its call sites would run it: input RMS norm + q|k|v in one
    # launch, o, then post-attention RMS norm + gate/up + SiLU product in one
    # launch feeding down_proj
    norm_w = [1.0 + 0.1 * torch.randn(4096, generator=gen, device=dev) for _ in range(2)]

    def fused_step(layer):
        qz.rmsnorm_qmatmul_group(layer[0:3], xs[0], norm_w[0], 1e-5)
        layer[3].forward(xs[3])
        h = qz.rmsnorm_gate_up_silu(layer[4], layer[5], xs[4], norm_w[1], 1e-5)
        layer[6].forward(h)

    # activation handles for the dot-only graph
    acts = {k: qz.QActivation(qz.GgmlDType.Q8K, 1, k, dev) for k in (4096, 14336)}
    for (_, n, k), x in zip(LAYER, xs):
        acts[k].quantize(x)

    def dot_step(layer):
        for qm, (_, n, k), y in zip(layer, LAYER, ys):
            qm.forward_quantized(acts[k], y)

    # the step as a caller holding x and y in host memory runs it (a shim over host
    # tensors): per projection x host -> device, forward, y device -> host, through
    # pinned buffers on the same stream -- the PCIe-inclusive rate, never `value`
    hxs = [torch.randn(1, k, generator=gen, device=dev).cpu().pin_memory() for (_, n, k) in LAYER]
    hys = [torch.empty(1, n, pin_memory=True) for (_, n, k) in LAYER]
    dxs = [torch.empty(1, k, device=dev) for (_, n, k) in LAYER]

    def host_step(layer):
        for qm, hx, hy, dx in zip(layer, hxs, hys, dxs):
            dx.copy_(hx, non_blocking=True)
            hy.copy_(qm.forward(dx), non_blocking=True)

    stream = torch.cuda.current_stream(dev)
    for fn in (full_step, dot_step, grouped_step, fused_step, host_step):
        fn(copies[0])  # eager pass: sizes scratch outside capture
    torch.cuda.synchronize()
    g_full = StepGraphs(torch, full_step, copies)
    g_dot = StepGraphs(torch, dot_step, copies)
    g_grp = StepGraphs(torch, grouped_step, copies)
    g_fus = StepGraphs(torch, fused_step, copies)
    g_host = StepGraphs(torch, host_step, copies)
    steps, warmup = args.steps, args.warmup
    # the headline: exactly `warmup` untimed steps, then exactly `steps` timed ones
    if warmup:
        g_full.run(warmup)
    ms_full = g_full.time(steps, stream)
    floor = read_floor(torch, copies, stream, max(20, (steps + args.copies - 1) // args.copies))
    log(f"read-only stream of the same bytes: {floor['us_per_step']:.2f} us per step; per launch {floor['us_per_launch']}")
    if args.read_probe:
        print(json.dumps({"us_per_step": round(ms_full * 1e3, 3), "read_floor": floor}), flush=True)
        return
    reps = max(1, (steps + args.copies - 1) // args.copies)
    wreps = max(1, (warmup + args.copies - 1) // args.copies)
    side = max(args.copies, min(steps, 8 * args.copies))  # steps timed for the side measurements
    ms = {}
    for name, g in (("dot", g_dot), ("grp", g_grp), ("fus", g_fus), ("host", g_host)):
        g.run(args.copies)
        ms[name] = g.time(side, stream)
    ms_dot, ms_grp, ms_fus, ms_host = ms["dot"], ms["grp"], ms["fus"], ms["host"]
    value = layer_bytes / (ms_full * 1e-3) / 1e9
    full_gbs = (layer_bytes + io_bytes) / (ms_full * 1e-3) / 1e9
    dot_gbs = (layer_bytes + io_bytes) / (ms_dot * 1e-3) / 1e9
    log(f"step (7 x QMatMul::forward): {ms_full * 1e3:.2f} us -> {value:.0f} GB/s; "
        f"dot kernels alone {ms_dot * 1e3:.2f} us -> {dot_gbs:.0f} GB/s; "
        f"grouped (4 launches) {ms_grp * 1e3:.2f} us -> {layer_bytes / (ms_grp * 1e-3) / 1e9:.0f} GB/s; "
        f"call-site fused (norm+q|k|v, o, norm+gate|up+SiLU, down) {ms_fus * 1e3:.2f} us; "
        f"host-staged x/y {ms_host * 1e3:.2f} us")

    # per-shape dot kernel times (same graphs, one shape at a time)
    kernels = {}
    for i, (name, n, k) in enumerate(LAYER):
        if name in ("k_proj", "up_proj", "o_proj"):
            continue  # same shape as v_proj / gate_proj / q_proj
        def one_shape(i=i, k=k):
            for layer in copies:
                layer[i].forward_quantized(acts[k], ys[i])
        g = capture(torch, one_shape)
        timed_graph(torch, g, wreps, stream)
        ms = timed_graph(torch, g, reps, stream) / args.copies
        b = copies[0][i].qtensor().storage_size_in_bytes() + 4 * (n + k)
        kernels[f"{name}_{n}x{k}"] = {"us": round(ms * 1e3, 3), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                                      "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del g

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_full, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "Q4_K batch-1 decode GEMV at Llama-3-8B layer shapes (configs[1]): one step = "
                        "QMatMul::forward for q,k,v,o,gate,up,down of one layer, x f32 [1,K] ~ N(0,1), "
                        f"weights N(0,0.02) -> Q4_K, {args.copies} layer copies rotated "
                        f"({args.copies * layer_bytes / 1e6:.0f} MB working set), HIP-graph replay",
            "weight_bytes_per_step": layer_bytes,
            "arithmetic": "Q8_K activation codes x Q4_K codes in int8 sdot4, int32 sub-block sums, f32 combine",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(full_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(full_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "k_gemv1<Q4_K, fused> (quantise x + dequant/int-dot GEMV, one launch per projection, "
                      "four lanes per block, static group schedule: q/o 4 and k/v 1 row per wave in four-wave "
                      "workgroups, gate/up 7 and down 2 in eight-wave workgroups); algorithmic bytes per launch = "
                      "N*K/256*144 + 4K + 4N, averaged over the 7 launches",
            "us_per_launch": round(ms_full * 1e3 / len(LAYER), 3),
            "algorithmic_bytes_per_launch": round((layer_bytes + io_bytes) / len(LAYER)),
        },
        "dot_only": {"us_per_step": round(ms_dot * 1e3, 3), "GB/s": round(dot_gbs, 1),
                     "kernel": "k_gemv1<Q4_K> on pre-quantised activations (forward_quantized)"},
        "grouped": {"us_per_step": round(ms_grp * 1e3, 3),
                    "GB/s": round(layer_bytes / (ms_grp * 1e-3) / 1e9, 1),
                    "frac_hbm": round(layer_bytes / (ms_grp * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "launches": 4,
                    "path": "lbq_qmatmul_group_f32 for q|k|v and gate|up (one fused launch each), "
                            "lbq_qmatmul_f32 for o and down; outputs bit-identical to the 7 separate calls"},
        "call_site_fused": {"us_per_step": round(ms_fus * 1e3, 3),
                            "GB/s": round(layer_bytes / (ms_fus * 1e-3) / 1e9, 1),
                            "launches": 4,
                            "path": "lbq_rmsnorm_qmatmul_group_f32 (input RMS norm + q|k|v, the norm in the GEMV "
                                    "prologue), lbq_qmatmul_f32 (o), lbq_rmsnorm_gate_up_silu_f32 (post-attention "
                                    "norm + gate|up, silu(gate)*up in the epilogue), lbq_qmatmul_f32 (down on that "
                                    "product): the reference's layer data flow, its two RMS norms included"},
        "host_staged": {"us_per_step": round(ms_host * 1e3, 3),
                        "GB/s": round(layer_bytes / (ms_host * 1e-3) / 1e9, 1),
                        "pcie_bytes_per_step": io_bytes,
                        "path": "per projection: x copied from pinned host memory, lbq_qmatmul_f32, y copied "
                                "back to pinned host memory, on one stream (a caller whose tensors live on "
                                "the host); PCIe-inclusive, not the headline"},
        "kernels": kernels,
        "read_floor": floor,
    }
    del g_full, g_dot, g_grp, g_fus, g_host
    tr = load_traffic()
    if tr and "bytes_per_launch" in tr:
        result["roofline"]["traffic"] = tr["bytes_per_launch"]
        result["roofline"]["traffic_source"] = "profiles/traffic_q4k_gemv.json (" + tr.get("method", "") + ")"

    # ---------------------------------------------------------------- CPU baseline (bounded sample)
    if not args.no_cpu:
        try:
            blocks = [q.qtensor().data.cpu().numpy() for q in copies[0]]
            xh = [x.cpu().numpy() for x in xs]
            result["cpu_baseline"] = cpu_baseline(blocks, xh, args.cpu_seconds)
            log(f"cpu baseline: {result['cpu_baseline']['value']} GB/s")
        except Exception as e:  # the oracle is optional on a box without a compiler
            result["cpu_baseline"] = {"value": None, "unit": "GB/s", "cores": 0, "kind": "port",
                                      "sample": f"unavailable: {e}"}
    del copies, acts
    torch.cuda.empty_cache()

    # ---------------------------------------------------------------- config 4: M = 512 MFMA path
    if not args.no_gemm:
        result["prefill_gemm"] = gemm_bench(torch, qz, gen, dev, stream)

    # ---------------------------------------------------------------- configs 1, 3, 4: other shapes
    if not args.no_configs:
        result["configs"] = configs_bench(torch, qz, gen, dev, stream, result.get("prefill_gemm"))

    # ---------------------------------------------------------------- config 5: 32-layer stack
    if not args.no_stack:
        result["stack"] = stack_bench(torch, qz, gen, dev, stream)

    print(json.dumps(result), flush=True)


def prefill_profile(torch, qz, dev, ms, library=False):
    """configs[3]'s batched calls: Q4_K gate_proj 14336x4096 and down_proj 4096x14336 forward at
    each M of ms -- by default 16 (integer matrix cores), 64 (gate: k-sliced fp16 GEMM; down:
    matrix cores, two row halves) and 512 (wide fp16 tiles); 2048 takes the tall fp16 tiles --
    the weights rotated over >= 512 MB of copies, 5 graph replays each, for counter collection."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x1B4)
    stream = torch.cuda.current_stream(dev)
    out = {}
    for name, n, k in (("gate_proj", 14336, 4096), ("down_proj", 4096, 14336)):
        qms = [make_weights(torch, qz, qz.GgmlDType.Q4K, n, k, gen, dev) for _ in range(n_copies(n * k // 256 * 144))]
        for M in ms:
            x = torch.randn(M, k, generator=gen, device=dev)
            out[f"q4_k_{name}_{n}x{k}_m{M}"] = round(time_forwards(torch, qms, x, stream, reps=5, warm=1), 2)
        del qms
        torch.cuda.empty_cache()
        if library:
            # the library's fp16 GEMM on the same shape (LDS-staged operand tiles, no
            # dequantisation): fp16 weight copies rotated over the same >= 512 MB
            w16s = [torch.randn(k, n, generator=gen, device=dev).to(torch.float16)
                    for _ in range(n_copies(n * k * 2))]
            for M in ms:
                a16 = torch.randn(M, k, generator=gen, device=dev).to(torch.float16)
                g = capture(torch, lambda: [torch.matmul(a16, w) for w in w16s])
                timed_graph(torch, g, 1, stream)
                us = timed_graph_median(torch, g, 5, stream) / len(w16s) * 1e3
                out[f"fp16_library_{name}_{n}x{k}_m{M}"] = round(us, 2)
                del g, a16
            del w16s
            torch.cuda.empty_cache()
    print(json.dumps({"prefill_profile_us": out}), flush=True)


def load_prefill_traffic():
    """HBM bytes per M = 512 forward (gate and down), from the committed PMC summary."""
    f = ROOT / "profiles" / "traffic_q4k_prefill_m512.json"
    try:
        return json.loads(f.read_text())
    except (OSError, ValueError):
        return None


ROTATE_BYTES = 512e6  # every leg rotates at least this many distinct weight bytes (MALL: 256 MB)


def n_copies(nbytes: int) -> int:
    """Weight copies whose bytes together exceed ROTATE_BYTES (at least 2)."""
    return max(2, -(-int(ROTATE_BYTES) // int(nbytes)) + (1 if int(ROTATE_BYTES) % int(nbytes) == 0 else 0))


def ws_mb(qms) -> float:
    """Working set of a rotation: the distinct weight bytes one replay streams (MB)."""
    return round(sum(q.qtensor().storage_size_in_bytes() for q in qms) / 1e6, 1)


def time_forwards(torch, qms, x, stream, reps=25, warm=3):
    """us per QMatMul::forward: one graph replay runs forward over every weight copy in qms
    (rotating copies keeps the working set out of the MALL); median over `reps` replays."""
    g = capture(torch, lambda: [qm.forward(x) for qm in qms])
    timed_graph(torch, g, warm, stream)
    us = timed_graph_median(torch, g, reps, stream) / len(qms) * 1e3
    del g
    return us


def gemm_bench(torch, qz, gen, dev, stream):
    """Q4_K gate_proj / down_proj at M = 512: QMatMul::forward (quantise + operand
    pre-pass + MFMA GEMM) and the dot half alone (forward_quantized: pre-pass from Q8_K codes +
    GEMM), 2*M*N*K flops over the median of 25 graph replays, against dense bf16/fp16 peak."""
    out = {}
    M = 512
    for name, n, k in (("gate_proj", 14336, 4096), ("down_proj", 4096, 14336)):
        nc = n_copies(n * k // 256 * 144)
        qms = [make_weights(torch, qz, qz.GgmlDType.Q4K, n, k, gen, dev) for _ in range(nc)]
        x = torch.randn(M, k, generator=gen, device=dev)
        y = torch.empty(M, n, device=dev)
        act = qz.QActivation.for_weight(qms[0], M).quantize(x)
        us_f = time_forwards(torch, qms, x, stream)
        g_d = capture(torch, lambda: [qm.forward_quantized(act, y) for qm in qms])
        timed_graph(torch, g_d, 3, stream)
        us_d = timed_graph_median(torch, g_d, 25, stream) / len(qms) * 1e3
        fl = 2.0 * M * n * k
        nbytes = qms[0].qtensor().storage_size_in_bytes()
        out[f"{name}_{n}x{k}_m{M}"] = {
            "us_forward": round(us_f, 2), "us_dot": round(us_d, 2),
            "TFLOP/s_forward": round(fl / us_f / 1e6, 1), "TFLOP/s_dot": round(fl / us_d / 1e6, 1),
            "frac_bf16_peak_forward": round(fl / us_f / 1e6 / BF16_PEAK_TFLOPS, 4),
            "frac_bf16_peak_dot": round(fl / us_d / 1e6 / BF16_PEAK_TFLOPS, 4),
            "weight_GB/s_forward": round(nbytes / us_f / 1e3, 1), "working_set_MB": ws_mb(qms)}
        # yardstick: the library's plain fp16 GEMM (torch.matmul -> hipBLASLt) on the same
        # shape, operands already fp16 (no quantisation, no dequantisation)
        a16 = x.to(torch.float16)
        w16 = torch.randn(k, n, generator=gen, device=dev).to(torch.float16)
        g_l = capture(torch, lambda: torch.matmul(a16, w16))
        timed_graph(torch, g_l, 3, stream)
        us_l = timed_graph_median(torch, g_l, 25, stream) * 1e3
        out[f"{name}_{n}x{k}_m{M}"]["fp16_library_gemm"] = {
            "us": round(us_l, 2), "TFLOP/s": round(fl / us_l / 1e6, 1),
            "what": "torch.matmul of fp16 [M, K] x [K, N] (hipBLASLt), no dequantisation: a yardstick, not this path"}
        log(f"gemm {name} M={M}: forward {us_f:.1f} us, dot {us_d:.1f} us ({fl / us_d / 1e6:.0f} TFLOP/s); "
            f"library fp16 GEMM {us_l:.1f} us")
        del g_d, g_l, qms, x, y, act, a16, w16
    torch.cuda.empty_cache()
    g, d = out["gate_proj_14336x4096_m512"], out["down_proj_4096x14336_m512"]
    fl = 2.0 * 512 * 14336 * 4096
    us = (g["us_forward"] + d["us_forward"]) / 2
    out["roofline"] = {
        "bound": "mfma", "achieved": round(fl / us / 1e6, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
        "frac": round(fl / us / 1e6 / BF16_PEAK_TFLOPS, 4), "traffic": None,
        "kernel": "QMatMul::forward at M = 512 (Q8_K quantise + fp16 operand pre-pass, then k_gemm_w: eight-wave "
                  "128 x 256 tiles, v_mfma_f32_32x32x16_f16), mean of gate 14336x4096 and down 4096x14336",
        "us_per_forward": round(us, 2), "flops_per_forward": fl}
    tr = load_prefill_traffic()
    if tr:
        out["roofline"]["traffic"] = tr["bytes_per_forward"]
        out["roofline"]["traffic_source"] = "profiles/traffic_q4k_prefill_m512.json (" + tr.get("method", "") + ")"
    return out


def configs_bench(torch, qz, gen, dev, stream, prefill=None):
    """BASELINE configs[0] (Q8_0 4096x4096 GEMV, m = 1), configs[2] (Q6_K LM head 128256x4096 and
    Q5_K gate/up 14336x4096 at batch 1, 4, 8; x ~ N(0, 1) with 1 % of entries x20) and configs[3]
    (Q4_K gate 14336x4096 / down 4096x14336 at M = 16, 64, 512, 2048): QMatMul::forward per launch,
    HIP-graph replay, enough weight copies rotated that the working set exceeds the 256 MB MALL."""
    out = {}

    def timed_rot(qms, x, reps):
        return time_forwards(torch, qms, x, stream, reps=max(20, reps))

    def x_outliers(b, k):
        x = torch.randn(b, k, generator=gen, device=dev)
        mask = torch.rand(b, k, generator=gen, device=dev) < 0.01
        return torch.where(mask, x * 20.0, x)

    # Q8_0 GEMV (17.8 MB per copy, 29 copies)
    q8 = [make_weights(torch, qz, qz.GgmlDType.Q8_0, 4096, 4096, gen, dev) for _ in range(n_copies(4096 * 128 * 34))]
    wb = q8[0].qtensor().storage_size_in_bytes()
    us = timed_rot(q8, torch.randn(1, 4096, generator=gen, device=dev), 20)
    out["q8_0_4096x4096_m1"] = {"us": round(us, 2), "weight_GB/s": round(wb / us / 1e3, 1),
                                "frac_hbm": round(wb / us / 1e3 / HBM_PEAK_GBS, 4), "working_set_MB": ws_mb(q8)}
    # dense F16 weights (candle's dense QMatMul variant: an f32 matmul), 4096 x 4096
    f16 = []
    for _ in range(n_copies(4096 * 4096 * 2)):
        w = (torch.randn(4096, 4096, generator=gen, device=dev) * 0.02).to(torch.float16)
        f16.append(qz.QMatMul.from_qtensor(qz.QTensor(w.view(torch.uint8).reshape(-1), qz.GgmlDType.F16, (4096, 4096))))
    fb = 4096 * 4096 * 2
    for M in (1, 512):
        x = torch.randn(M, 4096, generator=gen, device=dev)
        us = timed_rot(f16, x, 20)
        fl = 2.0 * M * 4096 * 4096
        out[f"f16_dense_4096x4096_m{M}"] = {"us": round(us, 2), "weight_GB/s": round(fb / us / 1e3, 1),
                                           "working_set_MB": ws_mb(f16),
                                           "frac_hbm": round(fb / us / 1e3 / HBM_PEAK_GBS, 4),
                                           "TFLOP/s": round(fl / us / 1e6, 1),
                                           "path": "f32 GEMV (m <= 8) / v_mfma_f32_32x32x2_f32 GEMM (fp32 peak 157.3 TFLOP/s)"}
        log(f"dense F16 M={M}: {us:.1f} us")
    del f16
    # Q8_0 batched (prefill of the same weight): M = 16 and 64 on the integer matrix
    # cores (Q8_0 activations, v_mfma_i32_32x32x32_i8; 64 as two 32-row halves), 512 on
    # the fp16 MFMA GEMM
    for M in (16, 64, 512):
        x = torch.randn(M, 4096, generator=gen, device=dev)
        us = timed_rot(q8, x, 20)
        fl = 2.0 * M * 4096 * 4096
        out[f"q8_0_4096x4096_m{M}"] = {"us": round(us, 2), "TFLOP/s": round(fl / us / 1e6, 1),
                                       "working_set_MB": ws_mb(q8),
                                       "frac_bf16_peak": round(fl / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                                       "weight_GB/s": round(wb / us / 1e3, 1),
                                       "frac_hbm": round(wb / us / 1e3 / HBM_PEAK_GBS, 4),
                                       "path": ("Q8_0 quantisation, then the integer matrix-core kernel (v_mfma_i32_32x32x32_i8, "
                                                "the reference's integer block sums)" if M <= 64 else
                                                "MFMA (fp16 operands of the Q8_0 activation and d*q weight values)")}
        log(f"configs[0] Q8_0 M={M}: {us:.1f} us")
    del q8
    torch.cuda.empty_cache()
    # the 32-value legacy types (not BASELINE configs: the GGUF files the reference's own
    # tests serve, e.g. a Q4_0 TinyLlama): M = 16 on the integer matrix cores, 512 on the
    # fp16 MFMA GEMM
    for t, tname in ((qz.GgmlDType.Q4_0, "q4_0"), (qz.GgmlDType.Q4_1, "q4_1"), (qz.GgmlDType.Q5_0, "q5_0"),
                     (qz.GgmlDType.Q5_1, "q5_1")):
        bpb = {qz.GgmlDType.Q4_0: 18, qz.GgmlDType.Q4_1: 20, qz.GgmlDType.Q5_0: 22, qz.GgmlDType.Q5_1: 24}[t]
        qms = [make_weights(torch, qz, t, 4096, 4096, gen, dev) for _ in range(n_copies(4096 * 128 * bpb))]
        lb = qms[0].qtensor().storage_size_in_bytes()
        for M in (16, 512):
            x = torch.randn(M, 4096, generator=gen, device=dev)
            us = timed_rot(qms, x, 20)
            fl = 2.0 * M * 4096 * 4096
            out[f"{tname}_4096x4096_m{M}"] = {"us": round(us, 2), "TFLOP/s": round(fl / us / 1e6, 1),
                                              "working_set_MB": ws_mb(qms),
                                              "frac_bf16_peak": round(fl / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                                              "weight_GB/s": round(lb / us / 1e3, 1),
                                              "frac_hbm": round(lb / us / 1e3 / HBM_PEAK_GBS, 4),
                                              "path": ("activation quantisation, then the integer matrix-core kernel "
                                                       "(v_mfma_i32_32x32x32_i8, the reference's integer block sums)"
                                                       if M <= 16 else "MFMA (fp16 operands)")}
        log(f"{tname}: M=16 {out[f'{tname}_4096x4096_m16']['us']} us, M=512 {out[f'{tname}_4096x4096_m512']['us']} us")
        del qms
    torch.cuda.empty_cache()

    # Q6_K LM head (431 MB, two copies) and Q5_K gate/up (13 copies of 40 MB)
    head = [make_weights(torch, qz, qz.GgmlDType.Q6K, VOCAB, 4096, gen, dev) for _ in range(n_copies(VOCAB * 16 * 210))]
    q5 = [make_weights(torch, qz, qz.GgmlDType.Q5K, 14336, 4096, gen, dev) for _ in range(n_copies(14336 * 16 * 176))]
    hb, q5b = head[0].qtensor().storage_size_in_bytes(), q5[0].qtensor().storage_size_in_bytes()
    for B in (1, 4, 8):
        x = x_outliers(B, 4096)
        for name, qms, nbytes in (("q6_k_head_128256x4096", head, hb), ("q5_k_gate_up_14336x4096", q5, q5b)):
            us = timed_rot(qms, x, 10 if qms is head else 20)
            if B <= 4:
                path = "decode GEMV quantising the rows of x in its prologue (one launch)"
            elif qms is head:
                path = "Q8_K quantisation, then the multi-row decode GEMV (Q6_K)"
            else:
                path = "Q8_K quantisation, then the integer matrix-core kernel (v_mfma_i32_32x32x32_i8)"
            out[f"{name}_b{B}"] = {"us": round(us, 2), "weight_GB/s": round(nbytes / us / 1e3, 1),
                                   "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "path": path,
                                   "working_set_MB": ws_mb(qms)}
        log(f"configs[2] batch {B}: head {out[f'q6_k_head_128256x4096_b{B}']['us']} us, "
            f"q5_k {out[f'q5_k_gate_up_14336x4096_b{B}']['us']} us")
    del head, q5
    torch.cuda.empty_cache()

    # Q4_K gate / down at M = 16, 64, 512, 2048 (16 copies of each: 528 MB)
    for name, n, k in (("gate_proj", 14336, 4096), ("down_proj", 4096, 14336)):
        qms = [make_weights(torch, qz, qz.GgmlDType.Q4K, n, k, gen, dev) for _ in range(n_copies(n * k // 256 * 144))]
        nbytes = qms[0].qtensor().storage_size_in_bytes()
        for M in (16, 64, 512, 2048):
            key = f"{name}_{n}x{k}_m{M}"
            if M == 512 and prefill and key in prefill:  # the same measurement as prefill_gemm
                us = prefill[key]["us_forward"]
            else:
                x = torch.randn(M, k, generator=gen, device=dev)
                us = timed_rot(qms, x, 20)
            fl = 2.0 * M * n * k
            out[f"q4_k_{name}_{n}x{k}_m{M}"] = {
                "us": round(us, 2), "TFLOP/s": round(fl / us / 1e6, 1), "working_set_MB": ws_mb(qms),
                "frac_bf16_peak": round(fl / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                "weight_GB/s": round(nbytes / us / 1e3, 1), "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                "bound": "hbm" if M <= 64 else "mfma",
                "path": ("Q8_K quantisation, then the integer matrix-core kernel (v_mfma_i32_32x32x32_i8, "
                         "the reference's integer sums)" if M <= 32 else
                         "fp16 operand pre-pass, then the fp16 MFMA GEMM (v_mfma_f32_32x32x16_f16)")}
            log(f"configs[3] {name} M={M}: {us:.1f} us")
        del qms
        torch.cuda.empty_cache()
    return out


def stack_bench(torch, qz, gen, dev, stream):
    """Random-init Llama-3-8B linear stack, Q4_K_M mix: attn_v and even-layer ffn_down Q6_K,
    the rest Q4_K, Q6_K output head; all 7 projections per layer plus the head per token."""
    Q4K, Q6K = qz.GgmlDType.Q4K, qz.GgmlDType.Q6K
    t0 = time.perf_counter()
    layers = []
    for li in range(32):
        mats = []
        for name, n, k in LAYER:
            t = Q6K if name == "v_proj" or (name == "down_proj" and li % 2 == 0) else Q4K
            mats.append(make_weights(torch, qz, t, n, k, gen, dev))
        layers.append(mats)
    head = make_weights(torch, qz, Q6K, VOCAB, 4096, gen, dev)
    total = sum(q.qtensor().storage_size_in_bytes() for l in layers for q in l) + head.qtensor().storage_size_in_bytes()
    log(f"stack ready: {total / 1e9:.3f} GB in {time.perf_counter() - t0:.1f} s")
    out = {"weight_bytes": total}
    for B in (1, 32):
        xs = {k: torch.randn(B, k, generator=gen, device=dev) for k in (4096, 14336)}
        ys = {n: torch.empty(B, n, device=dev) for n in (1024, 4096, 14336, VOCAB)}

        def token_step():
            for mats in layers:
                for qm, (_, n, k) in zip(mats, LAYER):
                    qm.forward(xs[k])
            head.forward(xs[4096])

        def token_step_grouped():  # q|k|v grouped where the types agree; gate|up+SiLU fused into down
            for mats in layers:
                q, kp, v, o, gate, up, down = mats
                if v.qtensor().dtype() == q.qtensor().dtype():
                    qz.qmatmul_group([q, kp, v], xs[4096])
                else:
                    qz.qmatmul_group([q, kp], xs[4096])
                    v.forward(xs[4096])
                o.forward(xs[4096])
                down.forward(qz.gate_up_silu(gate, up, xs[4096]))
            head.forward(xs[4096])

        reps = 20 if B == 1 else 5
        for tag, fn in ((f"b{B}", token_step), (f"b{B}_call_site_fused", token_step_grouped)):
            g = capture(torch, fn)
            timed_graph(torch, g, 2, stream)
            ms = timed_graph(torch, g, reps, stream)
            out[tag] = {"ms_per_token_step": round(ms, 4), "tokens_per_s": round(B / (ms * 1e-3), 1),
                        "weight_GB/s": round(total / (ms * 1e-3) / 1e9, 1)}
            log(f"stack {tag}: {ms:.3f} ms/step -> {B / (ms * 1e-3):.0f} tok/s")
            del g
        del xs, ys
    return out


if __name__ == "__main__":
    main()
