#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X.

A step is one forward of one sparse-MoE layer (router -> permute -> Q4_0
SwiGLU experts -> weighted combine) over one batch of synthetic tokens.  Steps
rotate over --layers distinct layer instances (distinct weights and inputs,
about 5.4 GB at 16 Qwen3-shaped instances) so weight traffic comes from HBM,
not from the 256 MB last-level cache.  Everything the timed region touches is
resident in HBM before it starts.

Default run (no --workload): the headline is the batch-1 Qwen3-30B-A3B-shaped
decode layer (H=2048, I=768, E=128, top-8 softmax, T=1), which runs as one
kernel; sub-records carry the 4096-token Qwen3 prefill (MFMA roofline), the
32-token Zipf-skewed Qwen3 decode batch, and the router alone at the
reference's own benchmark shape (H=4096, E=16, top-2, one fp32 token).  Each
record is timed from its own HIP graph replay of the K steps, after an eager
pass with per-stage events (stage times, the roofline of the dominant kernel).
--workload W runs one workload alone.

Output: one JSON line with the whole-job tokens/s, the roofline of the
dominant kernel (bracketed by two HIP events on its stream), and the CPU
baseline (the reference's CPU MoE path, restated in oracle/ref_cpu_path.py,
timed on this host on a bounded sample).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--workload W]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "solution-is-all-you-need_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
# Stage events of phantom_moe_set_profile_events (include/phantom_moe.h): before
# the router, gate/up, down and combine, and after the combine.
STAGES = ("route", "gate_up", "down", "combine")
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # a record needs no system-scope release
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PREFILL_T = 1024  # from this batch on, a workload is priced against the MFMA roofline
# The metric of the benchmark this line reports.
METRIC = "MoE-layer decode tok/s + % of HBM peak; prefill grouped-GEMM % of MFMA peak"
HEADLINE = "qwen3_decode_t1"
# Every other workload of the benchmark, each its own sub-record.
SUB_WORKLOADS = ("qwen3_prefill_t4096", "qwen3_decode_t32_zipf", "mixtral_decode_t1", "mixtral_decode_t16",
                 "dsv3_decode_t1", "dsv3_decode_t8", "dsv3_decode_t64", "dsv3_prefill_t2048")
# Spin cycles queued ahead of each timed graph replay (torch.cuda._sleep), so
# the start event fires once the host has queued the whole replay: the
# interval between the events is the GPU's time for the K steps, without the
# host's cost of submitting the graph.
PRE_REPLAY_SPIN_CYCLES = 400_000
# The reference's router benchmark: PhantomTopKRouter at hidden 4096, 16
# experts, top-2, one fp32 token (tests/test_moe_routing.py:199-203); its
# published latency is 54.51 us on an RTX 4050 laptop GPU
# (docs/testing/test_03_qwen3_30b_a3b.md:50).
ROUTER_REF = dict(H=4096, E=16, k=2, T=1)
ROUTER_REF_PUBLISHED_US = 54.51


def pmc_summary(kernel: str, workload: str) -> str:
    return os.path.join(ROOT, "profiles", f"{kernel}_{workload}_pmc.json")


def metric_name(cfg) -> str:
    shape = {2048: "Qwen3-30B-A3B-shaped", 4096: "Mixtral-8x7B-shaped", 7168: "DeepSeek-V3-style"}.get(
        cfg.H, f"H={cfg.H}")
    regime = "prefill" if cfg.T >= PREFILL_T else "decode"
    extra = ", Zipf-skewed routing" if cfg.zipf else ""
    return f"MoE-layer {regime} tokens/s ({shape} layer, batch {cfg.T}{extra})"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--layers", type=int, default=None,
                   help="distinct layer instances to rotate over (default: 16 Qwen3-shaped, else enough for "
                        "4.5 GB of weights, at least 3)")
    p.add_argument("--replays", type=int, default=5,
                   help="timed HIP graph replays of K steps each (the median is reported)")
    p.add_argument("--workload", default=None,
                   help="one workload alone (default: the batch-1 Qwen3 headline plus the sub-records)")
    p.add_argument("--no-subs", action="store_true", help="the headline alone, without the sub-records")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-stage-events", action="store_true", help="time without the per-stage events")
    p.add_argument("--no-graph", action="store_true",
                   help="time eager launches instead of a HIP graph replay of the K steps")
    p.add_argument("--copy-bytes", type=int, default=0,
                   help="after the timed region, one plain device copy of this many bytes (the calibration "
                        "dispatch for FETCH_SIZE / WRITE_SIZE counter runs)")
    return p.parse_args()


class HipEvents:
    """Raw hipEvent_t handles from the HIP runtime torch loaded."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n):
        out = []
        for _ in range(n):
            ev = ctypes.c_void_p()
            rc = self.hip.hipEventCreateWithFlags(ctypes.byref(ev), HIP_EVENT_DISABLE_SYSTEM_FENCE)
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            out.append(ev.value)
        return out

    def elapsed_ms(self, a, b) -> float:
        ms = ctypes.c_float()
        rc = self.hip.hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(a), ctypes.c_void_p(b))
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)

    def destroy(self, evs):
        for e in evs:
            self.hip.hipEventDestroy(ctypes.c_void_p(e))


def default_layers(cfg) -> int:
    """Layer instances to rotate over: enough that the weights the steps
    touch between two visits of one instance (L - 1 steps of active experts)
    exceed the 256 MB last-level cache; 16 for the Qwen3-shaped layers."""
    if cfg.H == 2048:
        return 16
    per_layer = (cfg.E + (1 if cfg.shared else 0)) * 3 * cfg.H * cfg.I * 18 // 32
    return max(3, -(-int(4.5e9) // per_layer))


def gate_up_bytes(cfg, U: int) -> int:
    """Algorithmic HBM bytes of one gate/up launch: the Q4_0 gate and up
    matrices of the U distinct active experts (plus the shared expert) and the
    bf16 activations."""
    per_expert = 2 * cfg.I * cfg.H * 18 // 32
    return (U + (1 if cfg.shared else 0)) * per_expert + cfg.T * cfg.H * 2


def ffn_bytes(cfg, U: int) -> int:
    """Algorithmic HBM bytes of the fused gate/up + down launch: the gate, up
    and down matrices of the U active experts (plus the shared expert) and the
    bf16 activations."""
    return gate_up_bytes(cfg, U) + (U + (1 if cfg.shared else 0)) * cfg.H * cfg.I * 18 // 32


def layer_bytes(cfg, U: int) -> int:
    """Algorithmic HBM bytes of one layer: expert weights of the U active
    experts (+ shared), the fp32 router weight, bf16 x in and fp32 y out."""
    experts = (U + (1 if cfg.shared else 0)) * 3 * cfg.H * cfg.I * 18 // 32
    return experts + cfg.E * cfg.H * 4 + cfg.T * cfg.H * 2 + cfg.T * cfg.H * 4


def expert_bytes(cfg, U: int) -> int:
    """Q4_0 weight bytes of the U active experts (+ shared) of one layer."""
    return (U + (1 if cfg.shared else 0)) * 3 * cfg.H * cfg.I * 18 // 32


def down_flops(cfg) -> int:
    return 2 * cfg.T * (cfg.k + (1 if cfg.shared else 0)) * cfg.H * cfg.I


def gate_up_flops(cfg) -> int:
    return 2 * cfg.T * (cfg.k + (1 if cfg.shared else 0)) * 2 * cfg.H * cfg.I


def layer_flops(cfg) -> int:
    return 2 * cfg.T * (cfg.k + (1 if cfg.shared else 0)) * 3 * cfg.H * cfg.I + 2 * cfg.T * cfg.H * cfg.E


def cpu_info():
    """CPU model and SIMD feature flags of this host (/proc/cpuinfo)."""
    model, flags, ids = "unknown", [], {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key = line.split(":", 1)[0].strip()
                if key == "model name" and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif key in ("cpu family", "model", "stepping") and key not in ids:
                    ids[key] = line.split(":", 1)[1].strip()
                elif key == "flags":
                    flags = line.split(":", 1)[1].split()
                    break
    except OSError:
        pass
    if ids:
        # the family/model/stepping numbers name the part where a hypervisor
        # shortens the model string
        model += " (family %s, model %s, stepping %s)" % (ids.get("cpu family"), ids.get("model"), ids.get("stepping"))
    simd = sorted(f for f in flags if f.startswith(("avx", "amx", "fma", "f16c", "sse4", "vnni")))
    return model, simd


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the cores this process may run on,
    within the OMP_NUM_THREADS share when that is set."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and 0 < int(omp) < n:
        n = int(omp)
    return max(1, n)


def cpu_baseline(cfg, host_layer, budget_s: float):
    """The reference CPU path on layer instance 0, timed on a bounded sample:
    all threads with weights kept packed (the reference's runtime, dequantised
    on every call), one thread, and all threads on weights dequantised once up
    front."""
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    from oracle.ref_cpu_path import RefCPUMoE

    router_w, bias, gate, up, down, shared, xb = host_layer
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)

    def timed(layer, threads, budget, max_n=50):
        torch.set_num_threads(threads)
        layer(x)  # warm-up (allocator, oneDNN kernels)
        n, t0 = 0, time.perf_counter()
        while True:
            layer(x)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget or n >= max_n:
                return n, el

    threads = cpu_threads()
    packed = RefCPUMoE(router_w, gate, up, down, cfg.H, cfg.I, cfg.k, cfg.score, bias, shared)
    share = budget_s / 3.0
    n_all, el_all = timed(packed, threads, share)
    n_one, el_one = timed(packed, 1, share)
    pre = RefCPUMoE(router_w, gate, up, down, cfg.H, cfg.I, cfg.k, cfg.score, bias, shared, predequant=True)
    n_pre, el_pre = timed(pre, threads, share)
    del pre
    model, simd = cpu_info()
    r_all, r_one = cfg.T * n_all / el_all, cfg.T * n_one / el_one
    # value is the faster thread setting of the reference path (weights kept
    # packed).  At decode sizes one thread tends to win: the numpy dequant of
    # the active experts runs on one thread either way, and the small torch
    # ops (one router row, a few-row matmuls) pay a fork/join per op on many.
    best_one = r_one > r_all
    n_b, el_b, th_b = (n_one, el_one, 1) if best_one else (n_all, el_all, threads)
    return {
        "value": round(max(r_all, r_one), 3),
        "unit": "tokens/s",
        "cores": th_b,
        "kind": "port",
        "sample": f"{n_b} forwards of one {cfg.T}-token layer instance ({cfg.T * n_b} tokens, {el_b:.1f} s) on "
                  f"{th_b} thread(s), the faster of 1 and {threads}: torch fp32 router, numpy Q4_0 dequant of every "
                  f"active expert on every call, torch bf16 SwiGLU, index_add_ combine (oracle/ref_cpu_path.py)",
        "all_threads": {"value": round(r_all, 3), "unit": "tokens/s", "cores": threads,
                        "sample": f"{n_all} forwards ({el_all:.1f} s)"},
        "one_thread": {"value": round(r_one, 3), "unit": "tokens/s", "cores": 1,
                       "sample": f"{n_one} forwards ({el_one:.1f} s)"},
        "thread_note": "the numpy dequant of the active experts is single-threaded in both settings; at small "
                       "batches the torch ops are a router row and few-row matmuls, where many threads add a "
                       "fork/join per op, so one thread can be the faster setting",
        "predequantized": {"value": round(cfg.T * n_pre / el_pre, 3), "unit": "tokens/s", "cores": threads,
                           "sample": f"{n_pre} forwards ({el_pre:.1f} s) on bf16 weights dequantised once up front"},
        "cpu": model,
        "simd_flags": simd,
    }


# The reference's neuron-sparse fp16 FFN operator (legacy C ABI), B tokens of
# a D x D_ffn SwiGLU FFN with half the neurons active.
LEGACY_WORKLOADS = {
    "legacy_ffn_b1": dict(B=1, D=4096, D_ffn=14336, sparsity=50.0),
    "legacy_ffn_b8": dict(B=8, D=4096, D_ffn=14336, sparsity=50.0),
}


def bench_legacy(args):
    """sparse_mlp_forward (include/phantom_legacy.h) on resident fp16 weights:
    the call's own event timing (it waits for its stream, as the reference
    does) is the GPU time; tokens/s is over the wall clock of the K calls."""
    import numpy as np
    import torch

    from phantom_moe import legacy

    w = LEGACY_WORKLOADS[args.workload]
    B, D, Dffn, pct = w["B"], w["D"], w["D_ffn"], w["sparsity"]
    dev = torch.device("cuda:0")
    per_layer = 3 * Dffn * D * 2
    L = max(1, min(args.layers or 16, (4 << 30) // per_layer + 1))
    gen = torch.Generator(device=dev)
    layers = []
    for l in range(L):
        gen.manual_seed(1000 + l)
        wg = (torch.randn(Dffn, D, device=dev, generator=gen) / D ** 0.5).half()
        wu = (torch.randn(Dffn, D, device=dev, generator=gen) / D ** 0.5).half()
        wd = (torch.randn(D, Dffn, device=dev, generator=gen) / Dffn ** 0.5).half()
        bg = (torch.randn(Dffn, device=dev, generator=gen) * 0.1).half()
        bu = (torch.randn(Dffn, device=dev, generator=gen) * 0.1).half()
        x = torch.randn(B, D, device=dev, generator=gen).half()
        on = torch.rand(B, Dffn, device=dev, generator=gen) < (1.0 - pct / 100.0)
        idx = torch.zeros(B, Dffn, dtype=torch.int32, device=dev)
        cnt = on.sum(1).to(torch.int32)
        for b in range(B):
            nz = torch.nonzero(on[b]).flatten().to(torch.int32)
            idx[b, : nz.numel()] = nz
        layers.append((x, wg, bg, wu, bu, wd, idx, cnt))
    torch.cuda.synchronize()
    for i in range(args.warmup):
        legacy.sparse_mlp_forward(*layers[i % L], pct)
    torch.cuda.synchronize()
    gpu_ms = []
    t0 = time.perf_counter()
    for i in range(args.steps):
        gpu_ms.append(legacy.sparse_mlp_forward(*layers[i % L], pct)[1])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    counts = [int(layers[i % L][7].sum()) for i in range(args.steps)]
    # algorithmic bytes: the active rows of gate and up, the active columns of
    # down, x in and y out (fp16)
    alg = [3 * c * D * 2 + 2 * B * D * 2 for c in counts]
    ms = float(np.sum(gpu_ms))
    achieved = float(np.sum(alg)) / (ms * 1e-3) / 1e9
    out = {
        "metric": f"legacy sparse_mlp_forward tokens/s (fp16 SwiGLU FFN D={D}, D_ffn={Dffn}, batch {B}, "
                  f"{pct:.0f}% neuron sparsity)",
        "value": round(B * args.steps / elapsed, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 activations and weights, fp32 accumulate",
        "data": "synthetic (seeded): x ~ N(0,1), weights N(0, 1/fan_in), random active sets",
        "config": {"workload": args.workload, "B": B, "D": D, "D_ffn": Dffn, "sparsity_pct": pct,
                   "layer_instances": L, "weights_resident_gb": round(L * per_layer / 1e9, 3),
                   "active_neurons_mean": round(float(np.mean(counts)) / B, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "sparse_mlp_forward call (zero fill + lg_ffn_rows_kernel + lg_down_kernel)",
                     "algorithmic_bytes_per_launch": round(float(np.mean(alg))),
                     "avg_launch_us": round(ms * 1e3 / args.steps, 3)},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, ROOT)
        from oracle import oracle as O

        x, wg, bg, wu, bu, wd, idx, cnt = (t.cpu().numpy() for t in layers[0])
        n, t0 = 0, time.perf_counter()
        while True:
            O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, pct, order=1)
            n += 1
            el = time.perf_counter() - t0
            if el >= min(args.cpu_seconds, 10.0) or n >= 20:
                break
        out["cpu_baseline"] = {"value": round(B * n / el, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
                               "sample": f"{n} calls on layer instance 0 ({el:.1f} s): the reference kernels' "
                                         f"sequential fp32 loops restated in C (oracle/legacy_oracle.c, order 1)"}
    print(json.dumps(out), flush=True)


def bench_moe(args, cfg, with_cpu: bool) -> dict:
    """Time K steps of one MoE workload (eager with stage events, then one
    HIP graph replay); returns its record."""
    import numpy as np
    import torch

    import phantom_moe
    from phantom_moe import _lib, synth

    dev = torch.device("cuda:0")
    L = max(1, args.layers if args.layers else default_layers(cfg))
    K = args.steps

    # ---- resident inputs: L distinct layer instances --------------------
    layers = []
    host0 = None
    for l in range(L):
        dl = synth.device_layer(cfg, dev, layer=l)
        ex = phantom_moe.MoEWeights.from_q4_0(dl.gate, dl.up, dl.down, cfg.H, cfg.I, cfg.E, shared=dl.shared)
        xb = synth.activations(cfg.T, cfg.H, seed=42 + l)
        x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
        if l == 0 and with_cpu:
            host0 = (dl.router_w.cpu().numpy(), None if dl.router_bias is None else dl.router_bias.cpu().numpy(),
                     dl.gate.cpu().numpy(), dl.up.cpu().numpy(), dl.down.cpu().numpy(),
                     None if dl.shared is None else tuple(t.cpu().numpy() for t in dl.shared), xb)
        layers.append(phantom_moe.PreparedForward(ex, dl.router_w, cfg.T, cfg.k, cfg.score, dl.router_bias, x=x))
        del dl
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    lib = _lib.load()
    stream = _lib.stream_handle(dev)
    # Steps run in one continuous rotation over the instances (warm-up, the
    # eager pass, the untimed replay, the timed replays): an instance is
    # touched again only after the L - 1 others, so its weights come from
    # HBM, never from the last-level cache.
    pos = 0
    for i in range(args.warmup):
        layers[pos % L](stream)
        pos += 1
    torch.cuda.synchronize()

    use_events = not args.no_stage_events
    ev = HipEvents()
    n_ev = len(STAGES) + 1
    events = ev.create(n_ev * args.steps) if use_events else []
    arrays = [(ctypes.c_void_p * n_ev)(*events[i * n_ev:(i + 1) * n_ev]) for i in range(args.steps)] if use_events else []

    # ---- eager pass: exactly K steps between two synchronisations, stage
    # events around every stage (stage times, the dominant kernel's roofline)
    eager_layer = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(K):
        if use_events:
            lib.phantom_moe_set_profile_events(arrays[i], n_ev)
        eager_layer.append(pos % L)
        layers[pos % L](stream)
        pos += 1
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    if use_events:
        lib.phantom_moe_set_profile_events(None, 0)
    elapsed = t1 - t0
    # the eager rate without stage events (each forward's five event records
    # cost host time of their own): K more calls back to back, continuing the
    # rotation
    plain_elapsed = elapsed
    if use_events:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(K):
            layers[pos % L](stream)
            pos += 1
        torch.cuda.synchronize()
        plain_elapsed = time.perf_counter() - t0

    # ---- timed replays: the K steps captured in a HIP graph (one graph per
    # replay, each continuing the rotation), an untimed replay first; each
    # timed replay is bracketed by synchronisations, and by two events on its
    # stream queued behind a short spin so the interval is the GPU's time for
    # the K steps.  value and ms_per_step come from the median replay.
    replay_ms = []
    wall_s = []
    replay_layers = []
    if not args.no_graph:
        graphs = []
        for r in range(args.replays + 1):
            graph = torch.cuda.CUDAGraph()
            seq = [(pos + r * K + i) % L for i in range(K)]
            with torch.cuda.graph(graph):
                gstream = _lib.stream_handle(dev)
                for l in seq:
                    layers[l](gstream)
            graphs.append(graph)
            replay_layers.append(seq)
        replay_layers = replay_layers[1:]
        pos += (args.replays + 1) * K
        graphs[0].replay()  # untimed
        torch.cuda.synchronize()
        for graph in graphs[1:]:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            w0 = time.perf_counter()
            torch.cuda._sleep(PRE_REPLAY_SPIN_CYCLES)
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            wall_s.append(time.perf_counter() - w0)
            replay_ms.append(e0.elapsed_time(e1))
        del graphs

    if args.copy_bytes > 0:
        src = torch.ones(args.copy_bytes, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # every call of the single-launch path completed its hand-offs
    status = 0
    for lay in layers:
        status |= _lib.workspace_status(lay.workspace)

    # ---- per-kernel and per-layer times, U per instance --------------------
    U = [int(torch.unique(layers[l].topk_idx).numel()) for l in range(L)]
    stages = {name: [] for name in STAGES}
    layer_ms = []
    if use_events:
        for i in range(K):
            e = events[i * n_ev:(i + 1) * n_ev]
            layer_ms.append(ev.elapsed_ms(e[0], e[-1]))
            for j, name in enumerate(STAGES):
                stages[name].append(ev.elapsed_ms(e[j], e[j + 1]))
        ev.destroy(events)
    steps_U = [U[l] for l in eager_layer]
    resident_gb = round(sum(x.experts.nbytes() for x in layers) / 1e9, 3)
    del layers
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    eager_elapsed = elapsed
    clock_U = steps_U
    if replay_ms:
        med = int(np.argsort(replay_ms)[len(replay_ms) // 2])
        elapsed = replay_ms[med] * 1e-3
        clock_U = [U[l] for l in replay_layers[med]]
    value = cfg.T * args.steps / elapsed
    out = {
        "metric": metric_name(cfg),
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations x int4 (Q4_0) weights, fp32 accumulate; fp64 router logits",
        "data": "synthetic (seeded): x ~ N(0,1) bf16, router N(0,0.02) fp32, Q4_0 q uniform [-8,7], d ~ |N(0,0.02)|",
        "config": {
            "workload": cfg.name,
            "H": cfg.H, "I": cfg.I, "E": cfg.E, "top_k": cfg.k, "tokens_per_step": cfg.T,
            "score": cfg.score, "zipf_bias_s": cfg.zipf, "shared_expert": cfg.shared,
            "layer_instances": L, "weights_resident_gb": resident_gb,
            "active_experts_per_step_mean": round(float(np.mean(steps_U)), 2),
            "timing": (f"median of {len(replay_ms)} HIP graph replays of the K steps, HIP events on the replay "
                       f"stream; one rotation over the instances across warm-up, eager passes and replays"
                       if replay_ms else "eager launches, wall clock"),
        },
        "workspace_status": status,
    }
    if replay_ms:
        out["replays"] = {
            "ms_per_step": [round(m / args.steps, 5) for m in replay_ms],
            "wall_ms_per_step": [round(w * 1e3 / args.steps, 5) for w in wall_s],
            "wall_note": "host clock around each replay (synchronisation to synchronisation): adds the "
                         "pre-replay spin and the host's graph submission",
        }
        out["eager"] = {"tokens_per_s": round(cfg.T * args.steps / plain_elapsed, 2),
                        "ms_per_step": round(plain_elapsed * 1e3 / args.steps, 5),
                        "note": "K calls back to back on the launch stream, host clock between two "
                                "synchronisations, no stage events"}
        if use_events:
            out["eager_with_stage_events"] = {"tokens_per_s": round(cfg.T * args.steps / eager_elapsed, 2),
                                              "ms_per_step": round(eager_elapsed * 1e3 / args.steps, 5)}
    # whole-layer HBM rate on the graph clock, on both bases: all algorithmic
    # bytes, and the active experts' weights alone
    lay_bytes = float(sum(layer_bytes(cfg, u) for u in clock_U))
    exp_bytes = float(sum(expert_bytes(cfg, u) for u in clock_U))
    out["layer_hbm"] = {
        "full_bytes_gbs": round(lay_bytes / elapsed / 1e9, 1),
        "full_bytes_frac": round(lay_bytes / elapsed / 1e9 / HBM_PEAK_GBS, 4),
        "expert_bytes_gbs": round(exp_bytes / elapsed / 1e9, 1),
        "expert_bytes_frac": round(exp_bytes / elapsed / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_step": round(lay_bytes / args.steps),
        "clock": "graph replay (median), launch gaps between kernels included",
    }
    if use_events:
        # the kernel the gate/up stage launches at this shape; one kernel for
        # both stages means the single-launch layer, which the gate/up stage's
        # events bracket (the other stages are then empty)
        names = dict(kv.split("=") for kv in _lib.load().phantom_moe_expert_kernels(
            cfg.T, cfg.H, cfg.I, cfg.E, cfg.k, int(cfg.shared)).decode().split(";"))
        gu_kernel = names["gate_up"]
        fused = names["gate_up"] == names["down"]
        gu_ms = float(np.sum(stages["gate_up"]))
        gu_bytes = float(sum((layer_bytes if fused else gate_up_bytes)(cfg, u) for u in steps_U))
        achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
        traffic = None
        if os.path.exists(pmc_summary(gu_kernel, cfg.name)):
            with open(pmc_summary(gu_kernel, cfg.name)) as f:
                pmc = json.load(f)
            if pmc.get("workload") == cfg.name and pmc.get("kernel") == gu_kernel:
                traffic = pmc.get("hbm_bytes_per_launch")
        # a prefill launch is priced against the MFMA roofline when its arithmetic
        # intensity (flops per algorithmic byte) is above the ridge point, else
        # against HBM (DeepSeek-V3 at 2048 tokens: about 64 positions per
        # expert, 227 flop/B, below the 312 of bf16 peak / HBM peak)
        ridge = BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
        intensity = gate_up_flops(cfg) * args.steps / gu_bytes
        tf = gate_up_flops(cfg) * args.steps / (gu_ms * 1e-3) / 1e12
        if cfg.T >= PREFILL_T and not fused and intensity >= ridge:
            out["roofline"] = {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                               "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                               "algorithmic_flops_per_launch": gate_up_flops(cfg)}
        else:
            out["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                               "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}
        if cfg.T >= PREFILL_T and not fused:
            dn_ms = float(np.sum(stages["down"]))
            dn_tf = down_flops(cfg) * args.steps / (dn_ms * 1e-3) / 1e12
            out["roofline"].update({"intensity_flop_per_byte": round(intensity, 1), "ridge_flop_per_byte": round(ridge, 1),
                                    "achieved_tflops": round(tf, 2), "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                    "down_tflops": round(dn_tf, 2), "down_mfma_frac": round(dn_tf / BF16_PEAK_TFLOPS, 4)})
        out["roofline"].update({
            "kernel": gu_kernel,
            "down_kernel": names["down"],
            "algorithmic_bytes_per_launch": round(gu_bytes / args.steps),
            "avg_launch_us": round(gu_ms * 1e3 / args.steps, 3),
        })
        lay_ms = float(np.sum(layer_ms))
        eager_bytes = float(sum(layer_bytes(cfg, u) for u in steps_U))
        stage_us = {k: round(float(np.mean(v)) * 1e3, 3) for k, v in stages.items()}
        if fused:
            # one kernel: the events around it are the layer; the others
            # bracket nothing but each other
            lay_ms = gu_ms
            stage_us = {"single_launch": stage_us["gate_up"]}
        out["layer"] = {
            "gpu_us_per_step": round(lay_ms * 1e3 / args.steps, 3),
            "stage_us": stage_us,
            "hbm_achieved_gbs": round(eager_bytes / (lay_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(eager_bytes / (lay_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "tflops": round(layer_flops(cfg) * args.steps / (lay_ms * 1e-3) / 1e12, 3),
            "mfma_frac": round(layer_flops(cfg) * args.steps / (lay_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "clock": "eager, events around each step",
        }
        if fused:
            out["layer"]["single_launch"] = True
    out["cpu_baseline"] = None
    if host0 is not None:
        out["cpu_baseline"] = cpu_baseline(cfg, host0, args.cpu_seconds)
    return out


def bench_router_ref(args) -> dict:
    """phantom_moe_route alone at the reference's router benchmark shape
    (hidden 4096, 16 experts, top-2, one fp32 token): K calls timed eagerly
    with events around each, then HIP graph replays of the K calls (events on
    the replay stream, median replay)."""
    import numpy as np
    import torch

    from phantom_moe import _lib

    dev = torch.device("cuda:0")
    H, E, k, T = ROUTER_REF["H"], ROUTER_REF["E"], ROUTER_REF["k"], ROUTER_REF["T"]
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    W = torch.randn((E, H), generator=g, device=dev) * 0.02
    xs = [torch.randn((T, H), generator=g, device=dev) for _ in range(16)]
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    lib = _lib.load()
    nbytes = lib.phantom_moe_workspace_bytes(T, H, 0, E, k, 0)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    stream = _lib.stream_handle(dev)

    def call(i, s):
        rc = lib.phantom_moe_route(xs[i % 16].data_ptr(), 1, W.data_ptr(), None, T, H, E, k, 0, idx.data_ptr(),
                                   w.data_ptr(), ws.data_ptr(), nbytes, s)
        if rc:
            _lib.check(rc, "phantom_moe_route")

    for i in range(args.warmup):
        call(i, stream)
    ev = HipEvents()
    evs = ev.create(2 * args.steps)
    hip = ev.hip
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    torch.cuda.synchronize()
    for i in range(args.steps):
        hip.hipEventRecord(ctypes.c_void_p(evs[2 * i]), ctypes.c_void_p(stream))
        call(i, stream)
        hip.hipEventRecord(ctypes.c_void_p(evs[2 * i + 1]), ctypes.c_void_p(stream))
    torch.cuda.synchronize()
    per = [ev.elapsed_ms(evs[2 * i], evs[2 * i + 1]) * 1e3 for i in range(args.steps)]
    ev.destroy(evs)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gs = _lib.stream_handle(dev)
        for i in range(args.steps):
            call(i, gs)
    graph.replay()
    torch.cuda.synchronize()
    reps = []
    for _ in range(max(1, args.replays)):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(PRE_REPLAY_SPIN_CYCLES)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        reps.append(e0.elapsed_time(e1) * 1e3 / args.steps)
    g_us = float(np.median(reps))
    del graph
    return {
        "metric": "router latency (PhantomTopKRouter.forward: logits, top-k, softmax)",
        "config": {"workload": "router_ref_h4096_e16_k2_t1", "H": H, "E": E, "top_k": k, "tokens": T,
                   "x_dtype": "fp32"},
        "us_per_call_graph": round(g_us, 3),
        "us_per_call_eager_median": round(float(np.median(per)), 3),
        "launches_per_call": 2,
        "reference_published_us": ROUTER_REF_PUBLISHED_US,
        "reference_hardware": "RTX 4050 Laptop GPU (a different GPU; context, not a like-for-like comparison)",
        "reference_source": "docs/testing/test_03_qwen3_30b_a3b.md:50; config tests/test_moe_routing.py:199-203",
    }


def sub_record(rec: dict) -> dict:
    keep = ("metric", "value", "unit", "ms_per_step", "config", "replays", "eager", "layer_hbm", "roofline", "layer",
            "workspace_status")
    return {k: rec[k] for k in keep if k in rec}


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the sharding design is described in DESIGN.md.", file=sys.stderr)
        sys.exit(2)
    if args.workload in LEGACY_WORKLOADS:
        return bench_legacy(args)

    import torch

    from phantom_moe import synth

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.workload:
        if args.workload not in synth.CONFIGS:
            print(f"unknown workload {args.workload!r}; one of {sorted(synth.CONFIGS)} or "
                  f"{sorted(LEGACY_WORKLOADS)}", file=sys.stderr)
            sys.exit(2)
        print(json.dumps(bench_moe(args, synth.CONFIGS[args.workload], not args.no_cpu_baseline)), flush=True)
        return
    cfg = synth.CONFIGS[HEADLINE]
    out = bench_moe(args, cfg, not args.no_cpu_baseline)
    out["metric_detail"] = out["metric"]
    out["metric"] = METRIC
    if not args.no_subs:
        subs = {}
        for name in SUB_WORKLOADS:
            print(f"[bench] {name}", file=sys.stderr, flush=True)
            subs[name] = sub_record(bench_moe(args, synth.CONFIGS[name], False))
        print("[bench] router_ref", file=sys.stderr, flush=True)
        subs["router_ref_h4096_e16_k2_t1"] = bench_router_ref(args)
        out["sub"] = subs
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
