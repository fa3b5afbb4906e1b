"""Benchmark of the quantized GEMV/GEMM path on one MI355X.

Workload: one Qwen2.5-3B Q4_K_M decode layer at M = 1
(the unified decode batch of the headline) through the quantized path, as a
chain over an fp32 residual stream: RMSNorm + Q8_1 -> grouped Q/K/V GEMV ->
Q8_1 of the attention output -> O accumulated into the residual -> RMSNorm
+ Q8_1 -> grouped gate/up GEMV -> SiLU * up + Q8_1 -> the Q6_K down
projection accumulated into the residual.  The layer is timed in four launch
forms (as the reference launches it, inferflux_amd/workloads.py
DECODE_LAUNCHES; with the Q8_1 producers fused into the GEMVs; with SiLU * up
in the gate/up epilogue as well; with one grid-synchronised FFN launch), and
a step is one layer in the fastest form (config.step names it).  Weights
rotate through replicas totalling >= 512 MB so every step streams from HBM,
not the 256 MB Infinity Cache.

Headline `value`: HBM GB/s of the timed step, i.e. the layer's algorithmic
bytes (weights, activations and outputs, each counted once) over
ms_per_step.  `roofline` is the step's longest launch timed alone, with the
HBM traffic per launch read from the committed rocprofv3 counter summary of
that kernel (profiles/).  The line also carries us per layer at M = 1/4/8,
an HBM read probe at the dominant launch's byte count, the other configs
(config 1 at M = 1/8, LM head, 14B layer at M = 16/32, 32B prefill GEMMs),
per-phase wall times and a CPU baseline timed on this host.

`python bench.py --profile FORM:LAUNCH` runs one launch of a layer form and
the counter calibration kernels, for rocprofv3.
"""
import argparse
import json
import os
import sys
import time

T_START = time.perf_counter()

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0       # MI355X dense fp16 MFMA
ROTATE_BYTES = 512 << 20


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--quick", action="store_true", help="headline only (no extra configs)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--profile", default=None, metavar="FORM:LAUNCH",
                   help="profiling run: eager launches of one launch of a 3B layer form "
                        "(e.g. fused_norm_swiglu:gate_up), the HBM read probe "
                        "at its byte count and a copy of known size for counter calibration")
    p.add_argument("--profile-kernels", action="store_true",
                   help="profiling run of the batch kernels: the 32B prefill GEMMs (fp16 and "
                        "int8 kernels, M = 512) and the 14B gate+up / down decode launches at "
                        "M = 32 (fp16-dequant GEMV), eager launches, plus the 64 MiB copy")
    return p.parse_args()


def gemv_bytes(ops, qt, M, Ns, K):
    """Algorithmic bytes of one launch: weights, one read of the Q8_1
    activations, fp32 outputs."""
    return sum(ops.weight_bytes(qt, N, K) for N in Ns) + M * (K // 32) * 36 + M * sum(Ns) * 4


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; the path would shard by weight rows "
              "and no multi-GPU figure is produced", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from inferflux_amd import ops, synth, workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.profile_kernels:
        profile_kernels_run(args, dev)
        return

    def ev():
        return torch.cuda.Event(enable_timing=True)

    # ------------------------------------------------------------ inputs
    def make_layer(projs, seed, replicas):
        """name -> (quant type, N, K, [replicated device weight tensors])."""
        out = {}
        for i, (name, qt, N, K) in enumerate(projs):
            w = torch.from_numpy(synth.blocks(qt, N, K, seed=seed * 100 + i)).to(dev)
            out[name] = (qt, N, K, [w] + [w.clone() for _ in range(replicas - 1)])
        return out

    def layer_bytes(projs):
        return sum(ops.weight_bytes(qt, N, K) for _, qt, N, K in projs)

    def n_replicas(total):
        return max(2, -(-ROTATE_BYTES // total))

    def time_loop(fn, steps, warmup):
        """us per fn call.  The calls are captured once into a HIP graph
        (fn(0) .. fn(steps-1), so weight replicas rotate) and the graph is
        replayed, so host launch latency does not leave the GPU idle.  The
        events are recorded on torch's current stream, the stream every
        kernel here is launched on."""
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

    def spread(fn, steps, reps=15):
        """median / p10 / p90 of us per call over `reps` replays of one graph
        of `steps` calls, each replay timed on its own (events on torch's
        current stream, the stream the kernels run on)."""
        fn(0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        samples = []
        for _ in range(reps):
            a, b = ev(), ev()
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            samples.append(a.elapsed_time(b) * 1e3 / steps)
        del g
        p10, med, p90 = np.percentile(samples, [10, 50, 90])
        return {"median_us": round(float(med), 2), "p10_us": round(float(p10), 2),
                "p90_us": round(float(p90), 2), "replays": reps, "calls_per_replay": steps}

    def tiled_layer(layer):
        """The layer's weights as tiled copies (ifx_repack_tiled), per replica."""
        return {name: (qt + 200, N, K, [ops.repack_tiled(qt, w, N, K)[1] for w in reps])
                for name, (qt, N, K, reps) in layer.items()}

    def decode_layer_runner(layer, M, seed, fused=False, split_down=False, tiled=None,
                            ordered=False):
        """One decode layer at batch M as a chain over an fp32 residual
        stream: RMSNorm+Q8_1 -> grouped QKV -> Q8_1 of the attention output
        (synthetic: attention itself is not on this path) -> O accumulated
        into the residual -> RMSNorm+Q8_1 -> grouped gate/up -> SiLU*up+Q8_1
        -> down accumulated into the residual.  4 producers + 4 GEMVs.
        fused: the two RMSNorm+Q8_1 producers and the Q8_1 quantize of the
        attention output run inside the QKV, gate/up and O launches
        (ifx_qgemv_grouped_rmsnorm; Q4_K, M <= 2): 1 producer + 4 GEMVs.
        fused == "swiglu": in addition gate/up computes SiLU(gate)*up and
        writes its Q8_1 blocks for down itself
        (ifx_qgemv_gate_up_silu_rmsnorm): 4 launches, no producer.
        fused == "batch_swiglu" (M <= 8; tiled copies M <= 32): the Q8_1
        producers as launches of their own, except SiLU * up + Q8_1, which the
        gate/up launch computes (ifx_qgemv_gate_up_silu, with the workspace
        its ordered K split needs from M = 17): 3 producers + 4 GEMVs.
        split_down: the down projection reads a row-split copy of its Q6_K
        weights (ifx_repack, M <= 2).
        tiled: the layer's tiled copy (tiled_layer) the GEMVs read instead
        (M <= 32).  ordered: K-split launches reduce in split order through a
        workspace per launch (ifx_qgemv_ws / ifx_qgemv_grouped_ws).
        run(i, which) runs one launch kind alone ("qkv", "o", "gate_up",
        "down", "producers")."""
        if tiled is not None:
            layer = tiled
        hidden, q_dim, ffn = layer["q"][2], layer["o"][2], layer["down"][2]
        rng = np.random.default_rng(seed)
        resid = torch.from_numpy(rng.standard_normal((M, hidden)).astype(np.float32)).to(dev)
        attn = torch.from_numpy(synth.activations(M, q_dim, seed=seed + 1)).to(dev)
        norm_w = {k: torch.from_numpy(rng.uniform(0.5, 1.5, hidden).astype(np.float16)).to(dev)
                  for k in ("attn", "ffn")}
        A = {"attn_in": (M, hidden), "attn_out": (M, q_dim), "ffn_in": (M, hidden),
             "ffn_act": (M, ffn)}
        A = {k: torch.empty((m, K // 32 * 36), dtype=torch.uint8, device=dev)
             for k, (m, K) in A.items()}
        Y = {name: torch.zeros((M, v[1]), dtype=torch.float32, device=dev)
             for name, v in layer.items()}
        Y["o"] = Y["down"] = resid  # O and down accumulate into the residual
        R = len(layer["q"][3])
        launches = {l[0]: l for l in workloads.DECODE_LAUNCHES}
        down_w = layer["down"]
        if split_down:
            qt, N, K, reps = layer["down"]
            down_w = (ops.Q6_K_R, N, K, [ops.repack(qt, w, N, K)[1] for w in reps])
        wsd = {}
        if ordered:
            for l in workloads.DECODE_LAUNCHES:
                qt_, _, K_, _ = layer[l[1][0]]
                nb = ops.qgemv_workspace_bytes(qt_, [layer[p][1] for p in l[1]], M, K_)
                if nb:
                    wsd[l[0]] = torch.zeros(nb, dtype=torch.uint8, device=dev)
        if fused == "batch_swiglu":
            qt_, N_, K_, _ = layer["gate"]
            nb = ops.gate_up_silu_workspace_bytes(qt_, M, N_, K_)
            if nb:
                wsd["gate_up_silu"] = torch.zeros(nb, dtype=torch.uint8, device=dev)

        def gemv(lname, r):
            _, projs, src, accum = launches[lname]
            qt, _, K, _ = layer[projs[0]]
            mode = ops.ACCUM if accum else ops.STORE
            if len(projs) == 1:
                p = down_w if projs[0] == "down" else layer[projs[0]]
                qt = p[0]
                ops.qgemv(qt, p[3][r], A[src], M, p[1], K, out=Y[projs[0]], mode=mode,
                          workspace=wsd.get(lname))
            else:
                ops.qgemv_grouped(qt, [layer[p][3][r] for p in projs], A[src], M,
                                  [layer[p][1] for p in projs], K,
                                  outs=[Y[p] for p in projs], mode=mode,
                                  workspace=wsd.get(lname))

        def gemv_norm(lname, r, x, nw):
            _, projs, _, accum = launches[lname]
            qt, _, K, _ = layer[projs[0]]
            ops.qgemv_grouped_rmsnorm(qt, [layer[p][3][r] for p in projs], x, nw, M,
                                      [layer[p][1] for p in projs], K,
                                      outs=[Y[p] for p in projs],
                                      mode=ops.ACCUM if accum else ops.STORE)

        def run(i, which=None):
            r = i % R
            if fused == "batch_swiglu":
                prod = which is None or which == "producers"
                if prod:
                    ops.rmsnorm_quantize_q8_1(resid, norm_w["attn"], out=A["attn_in"])
                if which is None or which == "qkv":
                    gemv("qkv", r)
                if prod:
                    ops.quantize_q8_1(attn, out=A["attn_out"])
                if which is None or which == "o":
                    gemv("o", r)
                if prod:
                    ops.rmsnorm_quantize_q8_1(resid, norm_w["ffn"], out=A["ffn_in"])
                if which is None or which == "gate_up":
                    qt, N, K, _ = layer["gate"]
                    ops.qgemv_gate_up_silu(qt, layer["gate"][3][r], layer["up"][3][r],
                                           A["ffn_in"], M, N, K, want_h=False,
                                           q8_1_out=A["ffn_act"],
                                           workspace=wsd.get("gate_up_silu"))
                if which is None or which == "down":
                    gemv("down", r)
                return
            prod = which is None or which == "producers"
            if prod and not fused:
                ops.rmsnorm_quantize_q8_1(resid, norm_w["attn"], out=A["attn_in"])
            if which is None or which == "qkv":
                gemv_norm("qkv", r, resid, norm_w["attn"]) if fused else gemv("qkv", r)
            if prod and not fused:
                ops.quantize_q8_1(attn, out=A["attn_out"])
            if which is None or which == "o":
                gemv_norm("o", r, attn, None) if fused else gemv("o", r)
            if prod and not fused:
                ops.rmsnorm_quantize_q8_1(resid, norm_w["ffn"], out=A["ffn_in"])
            if which is None or which == "gate_up":
                if fused == "swiglu":
                    qt, N, K, _ = layer["gate"]
                    ops.qgemv_gate_up_silu_rmsnorm(qt, layer["gate"][3][r], layer["up"][3][r],
                                                   resid, norm_w["ffn"], M, N, K, want_h=False,
                                                   q8_1_out=A["ffn_act"])
                elif fused:
                    gemv_norm("gate_up", r, resid, norm_w["ffn"])
                else:
                    gemv("gate_up", r)
            if prod and fused != "swiglu":
                ops.silu_mul_quantize_q8_1(Y["gate"], Y["up"], out=A["ffn_act"])
            if which is None or which == "down":
                gemv("down", r)
        return run

    def launch_bytes(layer, lname, M):
        projs = dict((l[0], l[1]) for l in workloads.DECODE_LAUNCHES)[lname]
        qt, _, K, _ = layer[projs[0]]
        return qt, gemv_bytes(ops, qt, M, [layer[p][1] for p in projs], K)

    def form_kernel_bytes(layer, M, form):
        """Algorithmic bytes of each launch of a layer form (weights, inputs
        and outputs each counted once; fp32 residual, fp16 norm weights)."""
        hidden, q_dim, ffn = layer["q"][2], layer["o"][2], layer["down"][2]
        wb = {n: ops.weight_bytes(v[0], v[1], v[2]) for n, v in layer.items()}
        a = lambda K: M * (K // 32) * 36  # Q8_1 activations
        qkv_n = sum(layer[p][1] for p in ("q", "k", "v"))
        if form == "reference":
            return {l[0]: launch_bytes(layer, l[0], M)[1] for l in workloads.DECODE_LAUNCHES}
        out = {"qkv": wb["q"] + wb["k"] + wb["v"] + M * hidden * 4 + hidden * 2 + M * qkv_n * 4,
               "o": wb["o"] + M * q_dim * 4 + M * hidden * 4}
        out["gate_up"] = (wb["gate"] + wb["up"] + M * hidden * 4 + hidden * 2 +
                          (a(ffn) if form == "swiglu" else 2 * M * ffn * 4))
        out["down"] = wb["down"] + a(ffn) + M * hidden * 4
        return out

    if args.profile:
        # eager launches of one launch of a 3B layer form, for rocprofv3
        form, kind = args.profile.split(":")
        fused = {"reference": False, "fused_norm": True, "fused_norm_swiglu": "swiglu",
                 "fused_norm_swiglu_split_down": "swiglu"}[form]
        projs3b = workloads.QWEN3B_LAYER
        R3 = n_replicas(layer_bytes(projs3b))
        layer3b = make_layer(projs3b, seed=1, replicas=R3)
        run = decode_layer_runner(layer3b, 1, seed=11, fused=fused,
                                  split_down=form.endswith("split_down"))
        profile_run(args, dev, lambda i: run(i, kind), f"{form}:{kind}",
                    form_kernel_bytes(layer3b, 1, {False: "reference", True: "norm",
                                                   "swiglu": "swiglu"}[fused])[kind])
        return

    result = {}
    extras = {}
    phase = {"setup_s": round(time.perf_counter() - T_START, 2)}
    t_gpu = time.perf_counter()

    # ------------------------------------------------ headline: 3B layer
    projs3b = workloads.QWEN3B_LAYER
    R3 = n_replicas(layer_bytes(projs3b))
    layer3b = make_layer(projs3b, seed=1, replicas=R3)
    layer_alg_bytes = {M: sum(launch_bytes(layer3b, l[0], M)[1] for l in workloads.DECODE_LAUNCHES)
                       for M in (1, 4, 8)}
    per_m = {}
    forms = {}  # M = 1 layer forms: name -> (runner, us per layer, kernel us, kernel bytes)
    layer3b_t = tiled_layer(layer3b)  # the batch forms' tiled copy (M = 4, 8)
    for M in (1, 4, 8):
        run = decode_layer_runner(layer3b, M, seed=10 + M)
        steps = args.steps if M == 1 else max(20, args.steps // 2)
        # whole layer: `steps` layers captured in one graph, replayed between
        # synchronisations (the K timed steps of the contract)
        us_layer = time_loop(run, steps, args.warmup)
        # each launch alone (same rotation), for per-kernel GB/s
        kern = {l[0]: time_loop(lambda i, n=l[0]: run(i, n), steps, args.warmup)
                for l in workloads.DECODE_LAUNCHES}
        kern["producers_x4"] = time_loop(lambda i: run(i, "producers"), steps, args.warmup)
        q4 = [l[0] for l in workloads.DECODE_LAUNCHES if launch_bytes(layer3b, l[0], M)[0] == ops.Q4_K]
        q4_bytes = sum(launch_bytes(layer3b, n, M)[1] for n in q4)
        q4_us = sum(kern[n] for n in q4)
        gemv_us = sum(kern[l[0]] for l in workloads.DECODE_LAUNCHES)
        per_m[M] = {
            "us_per_layer": round(us_layer, 2),
            "layer_GBs": round(layer_alg_bytes[M] / us_layer / 1e3, 1),
            "us_sum_kernels": round(sum(kern.values()), 2),
            "q4k_gemv_GBs": round(q4_bytes / q4_us / 1e3, 1),
            "layer_gemv_GBs": round(layer_alg_bytes[M] / gemv_us / 1e3, 1),
            "kernel_us": {k: round(v, 2) for k, v in kern.items()},
            "tokens_per_s_equiv": round(M / (workloads.QWEN3B_LAYERS * us_layer * 1e-6), 1),
        }
        if M > 2:
            # SiLU * up + Q8_1 in the epilogue of the gate/up launch
            runb = decode_layer_runner(layer3b, M, seed=10 + M, fused="batch_swiglu")
            us_b = time_loop(runb, steps, args.warmup)
            per_m[M]["fused_swiglu"] = {
                "us_per_layer": round(us_b, 2),
                "layer_GBs": round(layer_alg_bytes[M] / us_b / 1e3, 1),
                "kernel_us": {n: round(time_loop(lambda i, n=n: runb(i, n), steps, args.warmup), 2)
                              for n in ("qkv", "o", "gate_up", "down", "producers")},
                "tokens_per_s_equiv": round(M / (workloads.QWEN3B_LAYERS * us_b * 1e-6), 1),
            }
            # the same on the tiled weights: K splits added with fp32 atomics
            # (the plain entries, as the reference), and reduced in split
            # order through a workspace (the deterministic _ws entries)
            for tname, ordered in (("tiled_swiglu", False), ("tiled_swiglu_ordered", True)):
                runt = decode_layer_runner(layer3b, M, seed=10 + M, fused="batch_swiglu",
                                           tiled=layer3b_t, ordered=ordered)
                us_t = time_loop(runt, steps, args.warmup)
                per_m[M][tname] = {
                    "us_per_layer": round(us_t, 2),
                    "layer_GBs": round(layer_alg_bytes[M] / us_t / 1e3, 1),
                    "kernel_us": {n: round(time_loop(lambda i, n=n: runt(i, n), steps,
                                                     args.warmup), 2)
                                  for n in ("qkv", "o", "gate_up", "down", "producers")},
                    "tokens_per_s_equiv": round(M / (workloads.QWEN3B_LAYERS * us_t * 1e-6), 1),
                }
        if M == 1:
            fb = form_kernel_bytes(layer3b, M, "reference")
            forms["reference"] = (run, us_layer, {k: kern[k] for k in fb}, fb)
            for form, fused, kinds in (("fused_norm", True, ("qkv", "o", "gate_up", "down")),
                                       ("fused_norm_swiglu", "swiglu", ("qkv", "o", "gate_up", "down")),
                                       ("fused_norm_swiglu_split_down", "swiglu",
                                        ("qkv", "o", "gate_up", "down"))):
                runf = decode_layer_runner(layer3b, M, seed=10 + M, fused=fused,
                                           split_down=form.endswith("split_down"))
                us_f = time_loop(runf, steps, args.warmup)
                kus = {n: time_loop(lambda i, n=n: runf(i, n), steps, args.warmup) for n in kinds}
                fb = form_kernel_bytes(layer3b, M, {"fused_norm": "norm", "fused_norm_swiglu": "swiglu",
                                                    "fused_norm_swiglu_split_down": "swiglu"}[form])
                fb = {k: fb[k] for k in kinds}
                forms[form] = (runf, us_f, kus, fb)
                per_m[M][form] = {
                    "us_per_layer": round(us_f, 2),
                    "layer_GBs": round(layer_alg_bytes[M] / us_f / 1e3, 1),
                    "kernel_us": {k: round(v, 2) for k, v in kus.items()},
                    "kernel_GBs": {k: round(fb[k] / kus[k] / 1e3, 1) for k in kinds},
                    "tokens_per_s_equiv": round(M / (workloads.QWEN3B_LAYERS * us_f * 1e-6), 1),
                }
    extras["qwen3b_layer"] = per_m
    FORM_TEXT = {
        "reference": "layer as the reference launches it (4 Q8_1 producers + 4 GEMVs)",
        "fused_norm": "Q8_1 producers of QKV, O and gate/up fused into them (5 launches)",
        "fused_norm_swiglu": "producers fused and SiLU*up + Q8_1 in the gate/up epilogue (4 launches)",
        "fused_norm_swiglu_split_down": "as fused_norm_swiglu, with the down projection on a "
                                        "row-split copy of its Q6_K weights (ifx_repack)",
    }
    step_form = min(forms, key=lambda f: forms[f][1])
    step_run, step_us, step_kus, step_kbytes = forms[step_form]
    ms_per_step = step_us / 1e3
    # headline: HBM GB/s of the timed step (the layer's algorithmic bytes over
    # the step time), the same layer form that ms_per_step times
    headline = layer_alg_bytes[1] / step_us / 1e3
    step_spread = spread(step_run, max(20, args.steps // 10))

    # --------------------------------------- dominant kernel: roofline
    # the timed step's longest launch, timed alone (events around graph-
    # replayed launches on torch's current stream, the stream it runs on)
    dom = max(step_kus, key=step_kus.get)
    dom_us = time_loop(lambda i: step_run(i, dom), max(args.steps, 200), args.warmup)
    dom_spread = spread(lambda i: step_run(i, dom), max(args.steps, 200))
    dom_bytes = step_kbytes[dom]
    with ops.launch_log() as lg:
        step_run(0, dom)
        torch.cuda.synchronize()
    dom_kernels = lg.kernels
    achieved = dom_bytes / dom_us / 1e3
    traffic, traffic_src = profile_traffic(dom_kernels[-1])
    result["roofline"] = {
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
        "kernel": ";".join(dom_kernels), "launch": dom,
        "bytes_per_launch": dom_bytes, "us_per_launch": round(dom_us, 3),
        "traffic_source": traffic_src,
    }
    # what a plain streaming read of the same number of bytes achieves
    # (the size-dependent ceiling: launch ramp and drain are fixed costs)
    probe = probe_lib()
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    wbytes = (dom_bytes // 256) * 256
    big = torch.empty(max(ROTATE_BYTES * 2, 8 * wbytes), dtype=torch.uint8, device=dev)
    nrot = big.numel() // wbytes

    def probe_step(i, nbytes=wbytes):
        off = (i % nrot) * nbytes
        rc = probe.ifx_probe_read(big.data_ptr() + off, nbytes, sink.data_ptr(), 1 << 20,
                                  torch.cuda.current_stream().cuda_stream)
        assert rc == 0
    p_us = time_loop(probe_step, 200, 10)
    result["roofline"]["read_probe_same_bytes_GBs"] = round(wbytes / p_us / 1e3, 1)
    del big
    del layer3b, layer3b_t, forms, step_run
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
            gb = gemv_bytes(ops, qt, M, [N], K) / us / 1e3
            c1[f"M{M}"] = {"us": round(us, 3), "GBs": round(gb, 1),
                           "frac_hbm": round(gb / HBM_PEAK_GBS, 4)}
        # the same weights as a tiled copy (ifx_repack_tiled) at M = 8; GB/s
        # over the raw layout's algorithmic bytes
        treps = [ops.repack_tiled(qt, w_, N, K)[1] for w_ in reps]
        A = ops.quantize_q8_1(torch.from_numpy(synth.activations(8, K, seed=0)).to(dev))
        Y = torch.empty((8, N), dtype=torch.float32, device=dev)
        us = time_loop(lambda i: ops.qgemv(ops.Q4_K_T, treps[i % len(treps)], A, 8, N, K, out=Y),
                       max(args.steps, 200), args.warmup)
        gb = gemv_bytes(ops, qt, 8, [N], K) / us / 1e3
        c1["M8_tiled"] = {"us": round(us, 3), "GBs": round(gb, 1), "frac_hbm": round(gb / HBM_PEAK_GBS, 4)}
        del treps
        # the packed-activation path (per-row symmetric int8 codes, fp16
        # out) on the same weights; bytes: weights, M x K codes, M scales,
        # fp16 outputs; and the row quantizer that produces the codes
        for M in (1, 2):
            x = torch.from_numpy(synth.activations(M, K, seed=0)).to(dev)
            codes, scales = ops.quantize_rows_symmetric(x)
            Yh = torch.empty((M, N), dtype=torch.float16, device=dev)
            us = time_loop(lambda i: ops.qgemv_packed(qt, [reps[i % len(reps)]], codes, scales, M,
                                                      [N], K, outs=[Yh]),
                           max(args.steps, 200), args.warmup)
            gb = (ops.weight_bytes(qt, N, K) + M * K + M * 4 + M * N * 2) / us / 1e3
            c1[f"M{M}_packed"] = {"us": round(us, 3), "GBs": round(gb, 1),
                                  "frac_hbm": round(gb / HBM_PEAK_GBS, 4)}
            if M == 1:
                c1["quantize_rows_symmetric_M1_us"] = round(
                    time_loop(lambda i: ops.quantize_rows_symmetric(x, codes, scales), 200,
                              args.warmup), 3)
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
                gb = gemv_bytes(ops, qt, M, [N], K) / us / 1e3
                c3[f"{key}_M{M}"] = {"us": round(us, 2), "GBs": round(gb, 1),
                                     "frac_hbm": round(gb / HBM_PEAK_GBS, 4)}
            # the same weights as a row-split copy (ifx_repack), M = 1 and 2;
            # GB/s over the raw layout's algorithmic bytes
            rreps = [ops.repack(qt, w_, N, K)[1] for w_ in reps]
            rt = ops.Q8_0_R if qt == ops.Q8_0 else ops.Q6_K_R
            for M in (1, 2):
                A = ops.quantize_q8_1(torch.from_numpy(synth.activations(M, K, seed=3)).to(dev))
                Y = torch.empty((M, N), dtype=torch.float32, device=dev)
                us = time_loop(lambda i: ops.qgemv(rt, rreps[i % 2], A, M, N, K, out=Y),
                               max(20, args.steps // 4), 5)
                gb = gemv_bytes(ops, qt, M, [N], K) / us / 1e3
                c3[f"{key}_row_split_M{M}"] = {"us": round(us, 2), "GBs": round(gb, 1),
                                               "frac_hbm": round(gb / HBM_PEAK_GBS, 4)}
            del rreps
            # the tiled copy (ifx_repack_tiled) at M = 8
            treps = [ops.repack_tiled(qt, w_, N, K)[1] for w_ in reps]
            A = ops.quantize_q8_1(torch.from_numpy(synth.activations(8, K, seed=3)).to(dev))
            Y = torch.empty((8, N), dtype=torch.float32, device=dev)
            us = time_loop(lambda i: ops.qgemv(qt + 200, treps[i % 2], A, 8, N, K, out=Y),
                           max(20, args.steps // 4), 5)
            gb = gemv_bytes(ops, qt, 8, [N], K) / us / 1e3
            c3[f"{key}_tiled_M8"] = {"us": round(us, 2), "GBs": round(gb, 1),
                                     "frac_hbm": round(gb / HBM_PEAK_GBS, 4)}
            del treps
            del reps, w
            torch.cuda.empty_cache()
        extras["config3_lm_head_151936x2048"] = c3

        # ------------------------------------------- config 4: 14B layer
        projs14 = workloads.QWEN14B_LAYER
        layer14 = make_layer(projs14, seed=4, replicas=n_replicas(layer_bytes(projs14)))
        c4 = {}
        layer14_t = tiled_layer(layer14)
        for M in (16, 32):
            all_bytes = sum(launch_bytes(layer14, l[0], M)[1] for l in workloads.DECODE_LAUNCHES)
            steps = max(20, args.steps // 4)
            forms14 = [(f"M{M}", {}), (f"M{M}_tiled", {"tiled": layer14_t}),
                       (f"M{M}_tiled_ordered", {"tiled": layer14_t, "ordered": True})]
            # SiLU * up + Q8_1 in the gate/up launch (tiled; M = 32: the
            # fp16-dequant GEMV with its ordered K split)
            forms14.append((f"M{M}_tiled_swiglu", {"tiled": layer14_t, "fused": "batch_swiglu"}))
            for key, kw in forms14:
                run = decode_layer_runner(layer14, M, seed=40 + M, **kw)
                us_layer = time_loop(run, steps, 5)
                kern = {l[0]: time_loop(lambda i, n=l[0]: run(i, n), steps, 5)
                        for l in workloads.DECODE_LAUNCHES}
                kern["producers_x3" if kw.get("fused") else "producers_x4"] = time_loop(
                    lambda i: run(i, "producers"), steps, 5)
                c4[key] = {
                    "us_per_layer": round(us_layer, 2),
                    "layer_GBs": round(all_bytes / us_layer / 1e3, 1),
                    "gemv_GBs": round(all_bytes / sum(v for k, v in kern.items()
                                                      if not k.startswith("producers")) / 1e3, 1),
                    "kernel_us": {k: round(v, 2) for k, v in kern.items()},
                    "tokens_per_s_equiv": round(M / (workloads.QWEN14B_LAYERS * us_layer * 1e-6), 1),
                }
        del layer14_t
        # the Q4_K launches of the 14B layer at M = 1 and 8 (the 70 %-of-HBM
        # target names the 3B and the 14B shapes at those M)
        q4 = {}
        for M in (1, 8):
            run = decode_layer_runner(layer14, M, seed=50 + M)
            steps = max(20, args.steps // 4)
            for l in workloads.DECODE_LAUNCHES:
                qt, nb = launch_bytes(layer14, l[0], M)
                if qt != ops.Q4_K:
                    continue
                us = time_loop(lambda i, n=l[0]: run(i, n), steps, 5)
                q4[f"{l[0]}_M{M}"] = {"us": round(us, 2), "GBs": round(nb / us / 1e3, 1),
                                      "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
            if M == 1:
                # the gate/up pair on packed (per-row symmetric int8) activations
                qt, N, K, greps = layer14["gate"]
                ureps = layer14["up"][3]
                x = torch.from_numpy(synth.activations(1, K, seed=51)).to(dev)
                codes, scales = ops.quantize_rows_symmetric(x)
                outs = [torch.empty((1, N), dtype=torch.float16, device=dev) for _ in range(2)]
                us = time_loop(lambda i: ops.qgemv_packed(qt, [greps[i % len(greps)],
                                                              ureps[i % len(ureps)]],
                                                          codes, scales, 1, [N, N], K, outs=outs),
                               steps, 5)
                nb = 2 * ops.weight_bytes(qt, N, K) + K + 4 + 2 * N * 2
                q4["gate_up_M1_packed"] = {"us": round(us, 2), "GBs": round(nb / us / 1e3, 1),
                                           "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
        c4["q4k_launches_M1_M8"] = q4
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
            res = {}
            for kname, kern in (("f16", ops.PREFILL_F16), ("int8", ops.PREFILL_INT8)):
                us = time_loop(lambda i, kern=kern: ops.qgemm_prefill_kernel(
                    qt, w, A, M, N, K, kern, out=Y), max(10, args.steps // 10), 3)
                tops = 2.0 * M * N * K / us / 1e6
                res[kname] = {"us": round(us, 1), "TOPS": round(tops, 1),
                              "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
            res["f16"]["frac_f16_peak"] = round(res["f16"]["TOPS"] / F16_PEAK_TFLOPS, 4)
            # the fp16 GEMM with a caller workspace: activations converted
            # once (pre-pass launch included in the time), same bits
            ws = torch.empty(max(16, ops.prefill_workspace_bytes(qt, M, N, K)), dtype=torch.uint8,
                             device=dev)
            us = time_loop(lambda i: ops.qgemm_prefill_ws(qt, w, A, M, N, K, ws, out=Y),
                           max(10, args.steps // 10), 3)
            tops = 2.0 * M * N * K / us / 1e6
            res["f16_workspace"] = {"us": round(us, 1), "TOPS": round(tops, 1),
                                    "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                    "frac_f16_peak": round(tops / F16_PEAK_TFLOPS, 4)}
            del ws
            # the ordered K split (ifx_qgemm_prefill_ordered), where the shape splits
            nbo = ops.prefill_ordered_workspace_bytes(qt, M, N, K)
            if nbo > ops.prefill_workspace_bytes(qt, M, N, K):
                ws = torch.empty(nbo, dtype=torch.uint8, device=dev)
                us = time_loop(lambda i: ops.qgemm_prefill_ordered(qt, w, A, M, N, K, ws, out=Y),
                               max(10, args.steps // 10), 3)
                tops = 2.0 * M * N * K / us / 1e6
                res["f16_ordered"] = {"us": round(us, 1), "TOPS": round(tops, 1),
                                      "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                      "frac_f16_peak": round(tops / F16_PEAK_TFLOPS, 4)}
                del ws
            res["default"] = "f16" if ops.kernel_family(qt, M, N, K) == 4 else "int8"
            # The reference's prefill path recreated on this GPU: dequantize W
            # to an FP16 scratch copy (ifx_dequantize, the counterpart of
            # dequantize_q4_k / q6_k) and multiply it with the vendor
            # library's FP16 GEMM (torch.matmul -> hipBLASLt / rocBLAS,
            # fp32 accumulate) by fp16 activations.
            w16 = torch.empty((N, K), dtype=torch.float16, device=dev)
            x16 = x.to(torch.float16)
            y16 = torch.empty((M, N), dtype=torch.float16, device=dev)
            deq_us = time_loop(lambda i: ops.dequantize(qt, w, N, K, out=w16),
                               max(10, args.steps // 10), 3)
            gemm_us = time_loop(lambda i: torch.matmul(x16, w16.t(), out=y16),
                                max(10, args.steps // 10), 3)
            res["reference_path"] = {
                "dequant_fp16_us": round(deq_us, 1), "library_fp16_gemm_us": round(gemm_us, 1),
                "total_us": round(deq_us + gemm_us, 1),
                "fused_f16_speedup": round((deq_us + gemm_us) / res["f16"]["us"], 2),
                "fused_f16_workspace_speedup": round((deq_us + gemm_us) / res["f16_workspace"]["us"], 2)}
            del w16, x16, y16
            c5[f"{name}_{ops.TYPE_NAMES[qt]}_{N}x{K}"] = res
            del w
            torch.cuda.empty_cache()
        extras["config5_prefill_M512"] = c5

    phase["gpu_s"] = round(time.perf_counter() - t_gpu, 2)
    # --------------------------------------------------- CPU baseline
    cpu = None
    t_cpu = time.perf_counter()
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds, layer_alg_bytes[1])
    phase["cpu_baseline_s"] = round(time.perf_counter() - t_cpu, 2)

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
                   "step": step_form, "step_is": FORM_TEXT[step_form],
                   "step_launch_us": {k: round(v, 2) for k, v in step_kus.items()},
                   "spread": {"step": step_spread, "dominant_kernel": dom_spread},
                   "value_is": "HBM GB/s of the timed step: the layer's algorithmic bytes "
                               "(Q4_K + Q6_K weights, Q8_1/fp32 activations, fp32 outputs, "
                               "each once) over us per layer",
                   "layer_bytes": layer_alg_bytes[1],
                   "frac_of_hbm_peak": round(headline / HBM_PEAK_GBS, 4),
                   "wall_s": phase},
        "roofline": result["roofline"],
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


def profile_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (profiles/*.md holding the lines "kernel: <instance>" and
    "traffic_bytes_per_launch: <n>", from FETCH_SIZE and WRITE_SIZE runs
    scaled by a copy of known size), or (None, reason)."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        kern = traffic = None
        for line in open(path):
            if line.startswith("kernel: "):
                kern = line.split(":", 1)[1].strip()
            elif line.startswith("traffic_bytes_per_launch: "):
                traffic = int(line.split(":", 1)[1].strip())
        if kern == kernel and traffic is not None:
            return traffic, os.path.relpath(path, ROOT)
    return None, "no counter summary for " + kernel + " under profiles/"


PROBE_LIB = os.path.join(ROOT, "libbench_probe.so")


def build_probe():
    """Builds the benchmark's bandwidth probes (bench_probe.hip: a plain
    streaming read and a copy of known size, for the read-rate line and the
    counter calibration; not part of the library)."""
    import subprocess
    tmp = PROBE_LIB + ".tmp"
    subprocess.run([os.environ.get("HIPCC", "/opt/rocm/bin/hipcc"), "--offload-arch=gfx950", "-O3",
                    "-std=c++17", "-fPIC", "-shared", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", "-o", tmp, os.path.join(ROOT, "bench_probe.hip")],
                   check=True, capture_output=True)
    os.replace(tmp, PROBE_LIB)


def probe_lib():
    import ctypes
    lib = ctypes.CDLL(PROBE_LIB)
    for fn in (lib.ifx_probe_read, lib.ifx_probe_copy):
        fn.restype = ctypes.c_int
    lib.ifx_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                   ctypes.c_int, ctypes.c_void_p]
    lib.ifx_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                   ctypes.c_int, ctypes.c_void_p]
    return lib


def profile_run(args, dev, launch, name, nbytes):
    """Launches for rocprofv3: `warmup` eager launches, then `steps` launches
    of one launch of the 3B layer (weight replicas rotating) captured in a
    HIP graph and replayed twice, as the benchmark times them; 20 copies of exactly 64 MiB (k_probe_copy:
    FETCH_SIZE and WRITE_SIZE per dispatch of a known 64 MiB read and 64 MiB
    write calibrate the counters), and 20 streaming reads of the launch's
    algorithmic byte count (k_probe_read: the HBM read rate at this size).
    Prints one JSON line of event timings."""
    import torch

    from inferflux_amd import ops

    stream = torch.cuda.current_stream()
    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    with ops.launch_log() as lg:
        launch(0)
        torch.cuda.synchronize()
    # the launches captured in a graph and replayed, as the benchmark times them
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(args.steps):
            launch(i)
    stream = torch.cuda.current_stream()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    g.replay()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / args.steps
    del g

    lib = probe_lib()
    sp = stream.cuda_stream
    big = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(big)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    for _ in range(20):
        assert lib.ifx_probe_copy(dst.data_ptr(), big.data_ptr(), big.numel(), 8192, sp) == 0
    rb = (nbytes // 256) * 256
    src = torch.empty(rb, dtype=torch.uint8, device=dev)
    for i in range(20):
        assert lib.ifx_probe_read(src.data_ptr(), rb, sink.data_ptr(), 1 << 20, sp) == 0
    torch.cuda.synchronize()
    print(json.dumps({"profile": name, "kernels": lg.kernels, "launches": args.steps,
                      "event_us_per_launch": round(us, 3), "bytes_per_launch": nbytes,
                      "copy_bytes": big.numel(), "read_probe_bytes": rb}), flush=True)


def profile_kernels_run(args, dev):
    """Eager launches for rocprofv3 counter runs of the batch kernels:
    `steps` launches each of the config-5 prefill GEMMs on the fp16 kernel
    (and, where the shape uses one, with the activation workspace) and (a
    quarter as many) on the int8 kernel, of the config-4 14B grouped
    gate+up and down launches at M = 32 (and the fused gate/up/SiLU
    launch on tiled rows, the bench's form), and of config 1 and the 3B down
    projection at M = 8 on raw and on tiled rows (weights rotating over
    >= 512 MB of replicas), then 20 copies of exactly 64 MiB for counter
    calibration.  Prints one JSON line of event timings."""
    import torch

    from inferflux_amd import ops, synth, workloads

    def timed(fn, n):
        for i in range(2):
            fn(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(n):
            fn(i)
        b.record()
        torch.cuda.synchronize()
        return round(a.elapsed_time(b) * 1e3 / n, 2)

    out = {"profile": "batch kernels"}
    M = 512
    for name, qt, N, K in workloads.PREFILL_32B:
        w = torch.from_numpy(synth.blocks(qt, N, K, seed=5)).to(dev)
        A = ops.quantize_q8_1(torch.from_numpy(
            synth.activations(M, K, seed=5, outlier_frac=0.01)).to(dev))
        Y = torch.empty((M, N), dtype=torch.float32, device=dev)
        for kname, kern, n in (("f16", ops.PREFILL_F16, args.steps),
                               ("int8", ops.PREFILL_INT8, max(1, args.steps // 4))):
            out[f"prefill_{name}_{kname}_us"] = timed(
                lambda i, kern=kern: ops.qgemm_prefill_kernel(qt, w, A, M, N, K, kern, out=Y), n)
        need = ops.prefill_workspace_bytes(qt, M, N, K)
        if need:  # the fp16 kernel with the activations converted once
            wsp = torch.empty(need, dtype=torch.uint8, device=dev)
            out[f"prefill_{name}_f16_workspace_us"] = timed(
                lambda i: ops.qgemm_prefill_ws(qt, w, A, M, N, K, wsp, out=Y), args.steps)
            del wsp
        del w
    M = 32
    layer = {n: (qt, N, K) for n, qt, N, K in workloads.QWEN14B_LAYER}
    for launch, names in (("gate_up", ["gate", "up"]), ("down", ["down"])):
        qt, _, K = layer[names[0]]
        Ns = [layer[n][1] for n in names]
        ws = [torch.from_numpy(synth.blocks(qt, N, K, seed=7 + j)).to(dev)
              for j, N in enumerate(Ns)]
        R = max(2, -(-ROTATE_BYTES // sum(w.numel() for w in ws)))
        reps = [ws] + [[w.clone() for w in ws] for _ in range(R - 1)]
        A = ops.quantize_q8_1(torch.from_numpy(synth.activations(M, K, seed=8)).to(dev))
        Ys = [torch.empty((M, N), dtype=torch.float32, device=dev) for N in Ns]
        out[f"decode14b_{launch}_m32_us"] = timed(
            lambda i: ops.qgemv_grouped(qt, reps[i % R], A, M, Ns, K, outs=Ys), args.steps)
        if launch == "gate_up":  # the bench's form: tiled rows, SiLU * up and Q8_1 fused in
            treps = [[ops.repack_tiled(qt, w, N, K)[1] for w, N in zip(r, Ns)] for r in reps]
            del reps
            Q = torch.empty((M, Ns[0] // 32 * 36), dtype=torch.uint8, device=dev)
            nb = ops.gate_up_silu_workspace_bytes(qt + 200, M, Ns[0], K)
            wsd = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
            out["decode14b_gate_up_silu_tiled_m32_us"] = timed(
                lambda i: ops.qgemv_gate_up_silu(qt + 200, treps[i % R][0], treps[i % R][1], A, M,
                                                 Ns[0], K, want_h=False, q8_1_out=Q,
                                                 workspace=wsd if nb else None), args.steps)
            reps = treps
        del reps, ws
        torch.cuda.empty_cache()
    # raw against tiled rows (ifx_repack_tiled) on the slot-packed GEMV: config 1
    # and the 3B down projection at M = 8 (down: ordered K split on the tiled copy)
    for key, qt, N, K in (("config1", ops.Q4_K, 11008, 2048), ("down3b", ops.Q6_K, 2048, 11008)):
        M = 8
        w = torch.from_numpy(synth.blocks(qt, N, K, seed=9)).to(dev)
        R = max(2, -(-ROTATE_BYTES // w.numel()))
        reps = [w] + [w.clone() for _ in range(R - 1)]
        treps = [ops.repack_tiled(qt, x, N, K)[1] for x in reps]
        A = ops.quantize_q8_1(torch.from_numpy(synth.activations(M, K, seed=9)).to(dev))
        Y = torch.empty((M, N), dtype=torch.float32, device=dev)
        nb = ops.qgemv_workspace_bytes(qt + 200, [N], M, K)
        wsd = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev) if nb else None
        out[f"{key}_m8_raw_us"] = timed(lambda i: ops.qgemv(qt, reps[i % R], A, M, N, K, out=Y),
                                        args.steps)
        out[f"{key}_m8_tiled_us"] = timed(
            lambda i: ops.qgemv(qt + 200, treps[i % R], A, M, N, K, out=Y, workspace=wsd),
            args.steps)
        del reps, treps, w
        torch.cuda.empty_cache()
    lib = probe_lib()
    big = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(big)
    for _ in range(20):
        assert lib.ifx_probe_copy(dst.data_ptr(), big.data_ptr(), big.numel(), 8192,
                                  torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    print(json.dumps(out), flush=True)


def cpu_baseline(budget_s, layer_bytes):
    """CPU baseline on the headline's workload: one Qwen2.5-3B decode layer at
    M = 1 (Q/K/V, O, gate, up Q4_K and down Q6_K) as
    ggml-semantics GEMVs (the oracle's restatement of ggml's CPU path: x to
    Q8_K, integer block dots, fp32 scaling; ggml itself is absent from the
    reference snapshot) on all host cores, one projection after another,
    median over repetitions within about budget_s / 2 seconds.  `value` is the
    layer's algorithmic bytes (the headline's numerator) over that time.
    Beside it: the Q8_1-semantics oracle GEMVs on the same layer (the
    arithmetic the GPU path follows), and the config-1 GEMV alone."""
    import numpy as np

    from inferflux_amd import synth, workloads
    from oracle import oracle

    oracle.build()
    cores = len(os.sched_getaffinity(0))
    projs = workloads.QWEN3B_LAYER
    ws = [(qt, N, K, synth.blocks(qt, N, K, seed=7 + i)) for i, (_, qt, N, K) in enumerate(projs)]
    xs = {K: synth.activations(1, K, seed=K) for _, _, K, _ in ws}
    aq = {K: oracle.quantize_q8_1(x) for K, x in xs.items()}

    def median_time(fn, budget):
        times = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end or len(times) < 5:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if len(times) >= 20000:
                break
        return float(np.median(times)), len(times)

    def ggml_layer():
        for qt, N, K, w in ws:
            oracle.ggml_cpu_gemv(qt, w, xs[K], N, threads=cores)

    def oracle_layer():
        for qt, N, K, w in ws:
            oracle.gemv_q8_1(qt, w, aq[K], 1, N, K, threads=cores)

    t_ggml, n_ggml = median_time(ggml_layer, budget_s * 0.5)
    t_orc, n_orc = median_time(oracle_layer, budget_s * 0.25)
    N1, K1 = 11008, 2048
    w1 = synth.blocks(12, N1, K1, seed=0)
    x1 = synth.activations(1, K1, seed=0)
    t_c1, n_c1 = median_time(lambda: oracle.ggml_cpu_gemv(12, w1, x1, N1, threads=cores),
                             budget_s * 0.25)
    c1_bytes = w1.nbytes + K1 // 32 * 36 + N1 * 4
    cpu_model = ""
    try:
        for l in open("/proc/cpuinfo"):
            if l.startswith("model name"):
                cpu_model = l.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(layer_bytes / t_ggml / 1e9, 2), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"the headline workload: one Qwen2.5-3B Q4_K_M decode layer at M = 1 "
                      f"(7 GEMVs, ggml semantics: Q8_K activations), {cores} threads, median of "
                      f"{n_ggml} layers = {t_ggml * 1e6:.1f} us, {cpu_model}",
            "us_per_layer": round(t_ggml * 1e6, 1),
            "oracle_q8_1_layer": {"us_per_layer": round(t_orc * 1e6, 1),
                                  "GBs": round(layer_bytes / t_orc / 1e9, 2), "reps": n_orc,
                                  "is": "the Q8_1-semantics oracle GEMVs (the GPU path's "
                                        "arithmetic) on the same layer"},
            "config1_q4k_11008x2048": {"us": round(t_c1 * 1e6, 1),
                                       "GBs": round(c1_bytes / t_c1 / 1e9, 2), "reps": n_c1}}


if __name__ == "__main__":
    main()
