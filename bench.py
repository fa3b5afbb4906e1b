"""Benchmark of the quantized GEMV/GEMM path on one MI355X.

Workload: one Qwen2.5-3B Q4_K_M decode layer through
the quantized path -- Q8_1 quantize of the layer input, QKV / O / gate / up
Q4_K GEMVs, Q8_1 quantize of the FFN activation, Q6_K down GEMV -- at
M = 1 (the unified decode batch size of the headline).  A step is one such
layer.  Weights rotate through replicas totalling >= 512 MB so every step
streams from HBM, not the 256 MB Infinity Cache.

Headline `value`: HBM GB/s of the layer's Q4_K GEMVs at M = 1 (algorithmic
bytes: weights + Q8_1 activations + fp32 outputs, each counted once, over
the summed kernel time).  The JSON line also carries the roofline of the
dominant kernel (the 11008 x 2048 Q4_K GEMV), us per layer at M = 1/4/8,
the other configs (config 1 at M = 1/8, LM head, 14B layer at M = 16/32,
32B prefill GEMMs) and a CPU baseline timed on this host.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
ROTATE_BYTES = 512 << 20
# HBM bytes per launch of the dominant kernel from two rocprofv3 --pmc runs
# (FETCH_SIZE, WRITE_SIZE), each scaled by what the counter reads for a copy
# of exactly 64 MiB; summary and commands in profiles/k_gemv_q4k_11008x2048_m1.md.
DOMINANT_TRAFFIC_BYTES = 12785755


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--quick", action="store_true", help="headline only (no extra configs)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--profile", action="store_true",
                   help="profiling run: only the dominant GEMV (eager launches), the HBM "
                        "read probe and a copy of known size for counter calibration")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; the path shards by weight rows "
              "(see DESIGN.md) and no multi-GPU figure is produced", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from inferflux_amd import ops, synth, workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.profile:
        profile_run(args, dev)
        return

    def ev():
        return torch.cuda.Event(enable_timing=True)

    # ------------------------------------------------------------ inputs
    def make_layer(projs, seed, replicas):
        """Per projection: list of replicated device weight tensors."""
        out = []
        for i, (name, qt, N, K) in enumerate(projs):
            w = torch.from_numpy(synth.blocks(qt, N, K, seed=seed * 100 + i)).to(dev)
            reps = [w] + [w.clone() for _ in range(replicas - 1)]
            out.append((name, qt, N, K, reps))
        return out

    def layer_bytes(projs):
        return sum(ops.weight_bytes(qt, N, K) for _, qt, N, K in projs)

    def n_replicas(total):
        return max(2, -(-ROTATE_BYTES // total))

    def time_loop(fn, steps, warmup):
        """us per fn call.  The calls are captured once into a HIP graph
        (fn(0) .. fn(steps-1), so weight replicas rotate) and the graph is
        replayed, so host launch latency does not leave the GPU idle."""
        for i in range(min(warmup, 3)):
            fn(i)  # eager first calls: one-time kernel attribute set-up
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                fn(i)
        for _ in range(max(1, warmup // steps)):
            g.replay()
        g.replay()
        torch.cuda.synchronize()
        a, b = ev(), ev()
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        del g
        return a.elapsed_time(b) * 1e3 / steps  # us per call

    def decode_layer_runner(layer, M, seed):
        """One decode layer at batch M: 4 quantizes + 5 GEMVs."""
        hidden = layer[0][3]
        ffn = layer[2][2]
        xs = {k: torch.from_numpy(synth.activations(M, K, seed=seed + j, outlier_frac=0.0)).to(dev)
              for j, (k, K) in enumerate((("in", hidden), ("o", layer[1][3]),
                                          ("ffn", hidden), ("down", ffn)))}
        A = {k: torch.empty((M, v.shape[1] // 32 * 36), dtype=torch.uint8, device=dev)
             for k, v in xs.items()}
        Y = {name: torch.empty((M, N), dtype=torch.float32, device=dev)
             for name, _, N, _, _ in layer}
        src = {"qkv": "in", "o": "o", "gate": "ffn", "up": "ffn", "down": "down"}
        R = len(layer[0][4])

        def run(i, which=None):
            r = i % R
            for k in ("in", "o", "ffn", "down"):
                if which is None or which == "quant":
                    ops.quantize_q8_1(xs[k], out=A[k])
            for name, qt, N, K, reps in layer:
                if which is None or which == name:
                    ops.qgemv(qt, reps[r], A[src[name]], M, N, K, out=Y[name])
        return run

    def gemv_bytes(qt, M, N, K):
        return ops.weight_bytes(qt, N, K) + M * (K // 32) * 36 + M * N * 4

    result = {}
    extras = {}

    # ------------------------------------------------ headline: 3B layer
    projs3b = workloads.QWEN3B_LAYER
    R3 = n_replicas(layer_bytes(projs3b))
    layer3b = make_layer(projs3b, seed=1, replicas=R3)
    q4k_names = [p[0] for p in projs3b if p[1] == ops.Q4_K]
    per_m = {}
    for M in (1, 4, 8):
        run = decode_layer_runner(layer3b, M, seed=10 + M)
        steps = args.steps if M == 1 else max(20, args.steps // 2)
        # whole layer: `steps` layers captured in one graph, replayed between
        # synchronisations (the K timed steps of the contract)
        us_layer = time_loop(run, steps, args.warmup)
        # each kernel alone (same rotation), for per-kernel GB/s
        kern = {}
        for name, qt, N, K, _ in layer3b:
            kern[name] = time_loop(lambda i, n=name: run(i, n), steps, args.warmup)
        kern["quant"] = time_loop(lambda i: run(i, "quant"), steps, args.warmup)
        q4_bytes = sum(gemv_bytes(qt, M, N, K) for name, qt, N, K, _ in layer3b if qt == ops.Q4_K)
        q4_us = sum(kern[n] for n in q4k_names)
        all_bytes = sum(gemv_bytes(qt, M, N, K) for _, qt, N, K, _ in layer3b)
        per_m[M] = {
            "us_per_layer": round(us_layer, 2),
            "us_sum_kernels": round(sum(kern.values()), 2),
            "q4k_gemv_GBs": round(q4_bytes / q4_us / 1e3, 1),
            "layer_gemv_GBs": round(all_bytes / sum(kern[n] for n, *_ in layer3b) / 1e3, 1),
            "kernel_us": {k: round(v, 2) for k, v in kern.items()},
            "tokens_per_s_equiv": round(M / (workloads.QWEN3B_LAYERS * us_layer * 1e-6), 1),
        }
        if M == 1:
            ms_per_step = us_layer / 1e3
            headline = q4_bytes / q4_us / 1e3
    extras["qwen3b_layer"] = per_m

    # --------------------------------------- dominant kernel: roofline
    # the 11008 x 2048 Q4_K GEMV (gate), M = 1: events around back-to-back
    # launches on the stream the kernel runs on (torch's current stream)
    name, qt, N, K, reps = layer3b[2]
    M = 1
    x = torch.from_numpy(synth.activations(M, K, seed=0)).to(dev)
    A1 = ops.quantize_q8_1(x)
    Y1 = torch.empty((M, N), dtype=torch.float32, device=dev)
    dom_us = time_loop(lambda i: ops.qgemv(qt, reps[i % len(reps)], A1, M, N, K, out=Y1),
                       max(args.steps, 200), args.warmup)
    dom_bytes = gemv_bytes(qt, M, N, K)
    achieved = dom_bytes / dom_us / 1e3
    result["roofline"] = {
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": DOMINANT_TRAFFIC_BYTES,
        "kernel": f"k_gemv<Q4_K,MC=1> N={N} K={K} M=1", "bytes_per_launch": dom_bytes,
        "us_per_launch": round(dom_us, 3),
    }
    del layer3b
    torch.cuda.empty_cache()

    if not args.quick:
        # ------------------------------------------- config 1: single Q4_K
        c1 = {}
        name, qt, N, K = workloads.SINGLE_Q4K[0]
        w = torch.from_numpy(synth.blocks(qt, N, K, seed=0)).to(dev)
        reps = [w] + [w.clone() for _ in range(n_replicas(ops.weight_bytes(qt, N, K)) - 1)]
        for M in (1, 8):
            A = ops.quantize_q8_1(torch.from_numpy(synth.activations(M, K, seed=0)).to(dev))
            Y = torch.empty((M, N), dtype=torch.float32, device=dev)
            us = time_loop(lambda i: ops.qgemv(qt, reps[i % len(reps)], A, M, N, K, out=Y),
                           max(args.steps, 200), args.warmup)
            gb = gemv_bytes(qt, M, N, K) / us / 1e3
            c1[f"M{M}"] = {"us": round(us, 3), "GBs": round(gb, 1),
                           "frac_hbm": round(gb / HBM_PEAK_GBS, 4)}
        extras["config1_q4k_11008x2048"] = c1
        del reps, w
        torch.cuda.empty_cache()

        # ------------------------------------------------ config 3: LM head
        c3 = {}
        for key, projs in workloads.LM_HEAD.items():
            name, qt, N, K = projs[0]
            w = torch.from_numpy(synth.blocks(qt, N, K, seed=3)).to(dev)
            reps = [w, w.clone()]
            for M in (1, 8):
                A = ops.quantize_q8_1(torch.from_numpy(synth.activations(M, K, seed=3)).to(dev))
                Y = torch.empty((M, N), dtype=torch.float32, device=dev)
                us = time_loop(lambda i: ops.qgemv(qt, reps[i % 2], A, M, N, K, out=Y),
                               max(20, args.steps // 4), 5)
                gb = gemv_bytes(qt, M, N, K) / us / 1e3
                c3[f"{key}_M{M}"] = {"us": round(us, 2), "GBs": round(gb, 1),
                                     "frac_hbm": round(gb / HBM_PEAK_GBS, 4)}
            del reps, w
            torch.cuda.empty_cache()
        extras["config3_lm_head_151936x2048"] = c3

        # ------------------------------------------- config 4: 14B layer
        projs14 = workloads.QWEN14B_LAYER
        layer14 = make_layer(projs14, seed=4, replicas=n_replicas(layer_bytes(projs14)))
        c4 = {}
        for M in (16, 32):
            run = decode_layer_runner(layer14, M, seed=40 + M)
            us_layer = time_loop(run, max(20, args.steps // 4), 5)
            kern = {}
            for name, qt, N, K, _ in layer14:
                kern[name] = time_loop(lambda i, n=name: run(i, n), max(20, args.steps // 4), 5)
            all_bytes = sum(gemv_bytes(qt, M, N, K) for _, qt, N, K, _ in layer14)
            c4[f"M{M}"] = {
                "us_per_layer": round(us_layer, 2),
                "layer_GBs": round(all_bytes / us_layer / 1e3, 1),
                "kernel_us": {k: round(v, 2) for k, v in kern.items()},
                "tokens_per_s_equiv": round(M / (workloads.QWEN14B_LAYERS * us_layer * 1e-6), 1),
            }
        extras["config4_qwen14b_layer"] = c4
        del layer14
        torch.cuda.empty_cache()

        # ----------------------------------------- config 5: 32B prefill
        c5 = {}
        M = 512
        for name, qt, N, K in workloads.PREFILL_32B:
            w = torch.from_numpy(synth.blocks(qt, N, K, seed=5)).to(dev)
            x = torch.from_numpy(synth.activations(M, K, seed=5, outlier_frac=0.01)).to(dev)
            A = ops.quantize_q8_1(x)
            Y = torch.empty((M, N), dtype=torch.float32, device=dev)
            us = time_loop(lambda i: ops.qgemv(qt, w, A, M, N, K, out=Y, prefill=True),
                           max(10, args.steps // 10), 3)
            tops = 2.0 * M * N * K / us / 1e6
            c5[f"{name}_{ops.TYPE_NAMES[qt]}_{N}x{K}"] = {
                "us": round(us, 1), "int8_TOPS": round(tops, 1),
                "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
            del w
            torch.cuda.empty_cache()
        extras["config5_prefill_M512"] = c5

    # --------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)

    line = {
        "metric": "Q4_K dequant-GEMV HBM GB/s (% of peak) at M=1,8; us per decode layer",
        "value": round(headline, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xq4 (int32 dot, fp32 scale)",
        "data": "synthetic (seeded GGUF blocks, N(0,1) activations)",
        "config": {"workload": "qwen2.5-3b Q4_K_M decode layer, M=1 (BASELINE config 2)",
                   "M": 1, "hidden": 2048, "ffn": 11008, "weight_replicas": R3,
                   "value_is": "HBM GB/s of the layer's Q4_K GEMVs (QKV, O, gate, up)",
                   "frac_of_hbm_peak": round(headline / HBM_PEAK_GBS, 4)},
        "roofline": result["roofline"],
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


def probe_lib():
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "inferflux_amd", "libifx_probe.so"))
    for fn in (lib.ifx_probe_read, lib.ifx_probe_copy):
        fn.restype = ctypes.c_int
    lib.ifx_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                   ctypes.c_int, ctypes.c_void_p]
    lib.ifx_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                   ctypes.c_int, ctypes.c_void_p]
    return lib


def profile_run(args, dev):
    """Eager launches for rocprofv3: `steps` launches of the dominant GEMV
    (Q4_K 11008 x 2048, M = 1, rotating weight replicas), 20 copies of
    exactly 64 MiB (k_probe_copy: FETCH_SIZE and WRITE_SIZE per dispatch of
    a known 64 MiB read and 64 MiB write calibrate the counters), and 20
    streaming reads of the GEMV's weight bytes (k_probe_read: the HBM read
    rate at this transfer size).  Prints one JSON line of event timings."""
    import torch

    from inferflux_amd import ops, synth

    stream = torch.cuda.current_stream()
    qt, N, K = ops.Q4_K, 11008, 2048
    w = torch.from_numpy(synth.blocks(qt, N, K, seed=0)).to(dev)
    R = max(2, -(-ROTATE_BYTES // w.numel()))
    reps = [w] + [w.clone() for _ in range(R - 1)]
    A = ops.quantize_q8_1(torch.from_numpy(synth.activations(1, K, seed=0)).to(dev))
    Y = torch.empty((1, N), dtype=torch.float32, device=dev)
    for i in range(args.warmup):
        ops.qgemv(qt, reps[i % R], A, 1, N, K, out=Y)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(args.steps):
        ops.qgemv(qt, reps[i % R], A, 1, N, K, out=Y)
    b.record(stream)
    torch.cuda.synchronize()
    gemv_us = a.elapsed_time(b) * 1e3 / args.steps

    lib = probe_lib()
    sp = stream.cuda_stream
    big = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(big)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    for _ in range(20):
        assert lib.ifx_probe_copy(dst.data_ptr(), big.data_ptr(), big.numel(), 8192, sp) == 0
    nbytes = w.numel()
    for i in range(20):
        assert lib.ifx_probe_read(reps[i % R].data_ptr(), nbytes, sink.data_ptr(), 16384, sp) == 0
    torch.cuda.synchronize()
    print(json.dumps({"profile": "dominant gemv", "kernel": "k_gemv Q4_K N=11008 K=2048 M=1",
                      "launches": args.steps, "event_us_per_launch": round(gemv_us, 3),
                      "copy_bytes": big.numel(), "read_probe_bytes": nbytes}), flush=True)


def cpu_baseline(budget_s):
    """ggml-semantics CPU GEMV (oracle restatement; ggml itself is absent from
    the reference snapshot) on config 1 (Q4_K 11008 x 2048, M = 1), all host
    cores, median over repetitions within about budget_s seconds."""
    import numpy as np

    from inferflux_amd import synth
    from oracle import oracle

    oracle.build()
    cores = len(os.sched_getaffinity(0))
    N, K = 11008, 2048
    w = synth.blocks(12, N, K, seed=0)
    x = synth.activations(1, K, seed=0)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 20:
        t0 = time.perf_counter()
        oracle.ggml_cpu_gemv(12, w, x, N, threads=cores)
        times.append(time.perf_counter() - t0)
        if len(times) >= 20000:
            break
    med = float(np.median(times))
    nbytes = w.nbytes + K * 4 + N * 4
    cpu_model = ""
    try:
        for l in open("/proc/cpuinfo"):
            if l.startswith("model name"):
                cpu_model = l.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"ggml-semantics Q4_K x Q8_K GEMV, N=11008 K=2048 M=1 (config 1), "
                      f"median of {len(times)} reps = {med * 1e6:.1f} us, {cpu_model}"}


if __name__ == "__main__":
    main()
