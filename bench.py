#!/usr/bin/env python3
"""IR forward throughput of the catnn MI355X backend on one GPU.

Workload: the GEMM-heavy MLP forward, fp32,
batch 8192, 4096 → 16384 (bias, GELU) → 4096 (bias), built through the
reference's `.catnn` spec path (parse → architecture → lower) with the
Linear+GELU fusion that place::propose_fusions records, installed as one
program (params and input resident in HBM) and run step after step.

A step is one forward of the whole graph: two launches of the fp32 MFMA
GEMM kernel (fc1 with the bias+GELU epilogue, fc2 with the bias
epilogue).  Reported:
  * value       — algorithmic GFLOP/s of the step (2·M·K·N per Linear);
  * roofline    — that GEMM kernel's algorithmic TFLOP/s per launch over its
                  average launch duration, timed with hipEvents on the
                  program's stream inside the timed region, against the
                  157.3 TFLOP/s dense fp32 MFMA peak;
  * cpu_baseline — the oracle's restatement of the reference CPU path
                  (cpu::linear with OpenMP over rows where the reference uses
                  Rayon, then cpu::gelu and the bias pass) on a row subset of
                  the same inputs, timed on this host;
  * secondary   — the same measurement for the MoE layer (config 4,
                  tokens/s) and the pre-LN transformer block (config 3), and
                  the config-5 training step (block + MoE, forward, MSE,
                  backward, SGD).
Only one GPU is used: --gpus above 1 exits with a message.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cat-nn-compiler_amd"))

FP32_MFMA_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_program(dev, prog, x, steps, warmup):
    """Upload x, run `warmup` untimed forwards, then time `steps` forwards
    with hipEvents on the program's stream (synchronised on both sides)."""
    prog.forward(x)  # uploads the input into the program's input buffer
    for _ in range(warmup):
        prog.forward_resident()
    dev.sync()
    prog.profile(True)
    dev.sync()
    t0 = time.perf_counter()
    dev.timer_start()
    for _ in range(steps):
        prog.forward_resident()
    ms = dev.timer_stop()
    dev.sync()
    wall = time.perf_counter() - t0
    timings = prog.timings()
    prog.profile(False)
    return ms / steps, wall, timings


BF16_MFMA_PEAK_TFLOPS = 2500.0


def time_train_step(dev, steps, warmup, opt="sgd"):
    """Config 5: one training step (forward, MSE, backward, SGD) of the
    config-3 block followed by the config-4 MoE layer.  The timed steps run
    back to back after the warm-up steps, each updating the weights the next
    one reads, between one pair of hipEvents.  With opt="adam" the same step
    ends in Adam::put at Adam's default lr 1e-3.  `first_step_loss` is the
    loss of one more step from the installed weights."""
    import catnn_amd
    from catnn_amd import configs

    wl = configs.config5()
    log(f"config 5 built ({opt})")
    tr = catnn_amd.Trainer(dev, wl.graph, wl.lr if opt == "sgd" else 1e-3, opt=opt)
    tr.set_batch(wl.x, wl.target)
    for _ in range(warmup):
        tr.step(sync=False)
    dev.sync()
    dev.timer_start()
    for _ in range(steps):
        tr.step(sync=False)
    total = dev.timer_stop()
    last = tr.step()
    if not math.isfinite(last):
        raise RuntimeError(f"config 5 ({opt}): loss {last} after the timed steps; the steps "
                           "timed diverged and are not the workload")
    tr.reset()
    loss = tr.step()
    allocs, reserved = tr.arena()
    tr.free()
    ms = total / steps
    tflops = wl.flops / (ms / 1e3) / 1e12
    log(f"config 5 ({opt}): {ms:.3f} ms/step, {tflops:.1f} TFLOP/s algorithmic, loss {loss:.3f}")
    return {"ms_per_step": round(ms, 4), "tokens_per_s": round(wl.tokens / (ms / 1e3)),
            "algorithmic_TFLOP_per_s": round(tflops, 2),
            "bf16_mfma_frac": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4),
            "flop_per_step": wl.flops, "first_step_loss": round(loss, 4),
            "loss_after_timed_steps": round(last, 4),
            "arena_reserved_bytes": reserved, "arena_buffers": len(allocs),
            "precision": "bf16 MFMA, fp32 accumulation and master weights; split-bf16 forward "
                         "GEMMs for the attention projections, split-bf16 input to the MoE gate/up "
                         "GEMM; attention core on bf16 MFMA with normalised P rounded to bf16"}


def time_mixtral(dev, steps, warmup):
    """A Mixtral-style decoder forward through the (f)3 ops: the
    mixtral_architecture chain (embed → [RMSNorm → GQA+RoPE → RMSNorm → MoE]
    × 2 → RMSNorm → LmHead) at the config-4 MoE shape, 16 heads × 64 with 4
    K/V heads, a 32000-token vocabulary, on 8192 tokens; fp32."""
    import catnn_amd
    from catnn_amd import configs
    from catnn_amd.configs import MixtralShape

    shape = MixtralShape(vocab=32000, hidden=1024, inter=3584, layers=2, heads=16, kv_heads=4, experts=8,
                         top_k=2, sliding_window=4096)
    wl = configs.mixtral(batch=4, seq=2048, shape=shape)
    log("mixtral decoder built")
    prog = catnn_amd.Program(dev, wl.graph)
    ms, _, timings = time_program(dev, prog, wl.x, steps, warmup)
    prog.free()
    rate = wl.flops / (ms / 1e3)
    log(f"mixtral decoder: {ms:.3f} ms/step, {rate / 1e12:.1f} TFLOP/s")
    return {"tokens_per_s": round(wl.tokens / (ms / 1e3)), "ms_per_step": round(ms, 4),
            "GFLOP_per_s": round(rate / 1e9, 1), "mfma_frac": round(rate / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
            "shape": {"tokens": wl.tokens, "hidden": 1024, "heads": 16, "kv_heads": 4, "head_dim": 64,
                      "experts": 8, "top_k": 2, "intermediate": 3584, "vocab": 32000, "layers": 2},
            "steps_ms": {t[0]: round(t[3] / max(t[2], 1), 4) for t in timings}}


def _host_cpus():
    """The CPUs this process may run on (nproc); `cores` is the threads used."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline_mlp(wl, target_s):
    """Oracle restatement of the reference CPU path on a row subset."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle

    x = wl.x.numpy()
    p1, p2 = wl.graph.nodes[1].params, wl.graph.nodes[3].params
    w1, b1, w2, b2 = (p1["w"].numpy(), p1["b"].numpy(), p2["w"].numpy(), p2["b"].numpy())
    d, hidden = w1.shape

    def run(rows):
        t0 = time.perf_counter()
        h = oracle.gelu(oracle.linear(x[:rows], w1, b1))
        oracle.linear(h, w2, b2)
        return time.perf_counter() - t0

    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    probe_rows = max(2, min(cores, 16))
    t = run(probe_rows)
    rows = int(min(x.shape[0], max(probe_rows, probe_rows * target_s / max(t, 1e-3))))
    rows = max(probe_rows, (rows // probe_rows) * probe_rows)
    t = run(rows)
    flops = 2 * rows * (d * hidden + hidden * d)
    return {"value": round(flops / t / 1e9, 3), "unit": "GFLOP/s", "cores": cores,
            "host_cpus": _host_cpus(), "kind": "port",
            "sample": f"{rows} of {x.shape[0]} rows of the config-2 forward (fc1+bias, GELU, "
                      f"fc2+bias) in {t:.1f} s; OpenMP over rows where the reference uses Rayon"}


def cpu_baseline_moe(wl, target_s):
    """Config 4's MoE layer on the oracle's restatement of moe::moe
    (moe.rs:197-223): the router over all tokens, then a sequential token
    loop of per-expert SwiGLU calls, single-threaded as the reference is.
    Timed as the routing alone plus the expert work of a token prefix; per
    token cost is constant, so the layer's time is scaled to all tokens."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle

    node = wl.graph.nodes[1]
    E, k, H, I = node.op.fields
    P = node.params
    x = wl.x.numpy().reshape(-1, H)
    T = x.shape[0]
    gate = P["gate"].numpy()
    w1s = np.stack([P[f"e{e}.w1"].numpy().reshape(H, I) for e in range(E)])
    w3s = np.stack([P[f"e{e}.w3"].numpy().reshape(H, I) for e in range(E)])
    w2s = np.stack([P[f"e{e}.w2"].numpy().reshape(I, H) for e in range(E)])

    def run(n):
        t0 = time.perf_counter()
        oracle.moe(x, gate, w1s, w3s, w2s, k, tokens=np.arange(n, dtype=np.int64))
        return time.perf_counter() - t0

    t_route = run(0)
    per_tok = max(run(2) - t_route, 1e-6) / 2
    n = int(max(2, min(T, (target_s - t_route) / per_tok)))
    per_tok = max(run(n) - t_route, 1e-6) / n
    layer_s = t_route + T * per_tok
    return {"value": round(T / layer_s, 2), "unit": "tokens/s", "cores": 1, "host_cpus": _host_cpus(),
            "kind": "port",
            "sample": f"routing of all {T} tokens ({t_route:.2f} s) plus the expert loop over the first {n} "
                      f"tokens ({per_tok * 1e3:.1f} ms per token), scaled to {T} tokens; sequential as "
                      f"moe::moe"}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_f32_config2_hbm_traffic.txt")
COPY_FLOATS = 128 << 20  # 512 MiB read + 512 MiB written by the calibration copy


def measured_traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE scaled by a copy kernel of known size)."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def pmc_probe(which):
    """Kernel sequence for the rocprofv3 --pmc runs: a plain copy kernel
    (act_f32 with no activation: reads and writes COPY_FLOATS·4 bytes),
    then the workload's forwards."""
    import catnn_amd
    from catnn_amd import configs
    from catnn_amd import device as D

    dev = catnn_amd.Device(0)
    a, b = dev.alloc(COPY_FLOATS * 4), dev.alloc(COPY_FLOATS * 4)
    a.zero()
    for i in range(3):
        D.act(dev, a, b, COPY_FLOATS, 0)
        dev.sync()
        log(f"copy {i} done")
    a.free()
    b.free()
    builders = {"config2": configs.config2, "config3": configs.config3, "config4": configs.config4}
    if which == "config5":
        wl = configs.config5()
        tr = catnn_amd.Trainer(dev, wl.graph, wl.lr)
        tr.set_batch(wl.x, wl.target)
        for i in range(3):
            tr.step()
            log(f"config5: step {i} done")
        tr.free()
        dev.close()
        return
    for name in (builders if which == "all" else [which]):
        wl = builders[name]()
        prog = catnn_amd.Program(dev, wl.graph)
        prog.forward(wl.x)
        for _ in range(2):
            prog.forward_resident()
        dev.sync()
        log(f"{name}: 3 forwards done")
        prog.free()
    dev.close()


def gemm_probe(shapes):
    """The training step's bf16 GEMM kernel (catnn_hip_gemm_bf16_nt, C = A·Bᵀ
    with fp32 output) beside torch.matmul on the same bf16 operands (the
    hipBLASLt library GEMM, bf16 output) on M×N×K shapes: five launches of
    each for rocprofv3 --pmc, then hipEvent timings of twenty."""
    import torch
    import catnn_amd
    from catnn_amd import device as D

    dev = catnn_amd.Device(0)
    for (m, n, k) in shapes:
        a = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(n, k, device="cuda", dtype=torch.bfloat16)
        bt = b.t().contiguous()
        c = torch.empty(m, n, device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        ours = lambda: D.gemm_bf16_nt(dev, a.data_ptr(), k, b.data_ptr(), k, c.data_ptr(), n, m, n, k)
        for _ in range(5):
            ours()
        dev.sync()
        for _ in range(5):
            torch.matmul(a, bt)
        torch.cuda.synchronize()
        dev.timer_start()
        for _ in range(20):
            ours()
        t_ours = dev.timer_stop() / 20
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            torch.matmul(a, bt)
        e1.record()
        torch.cuda.synchronize()
        t_lib = e0.elapsed_time(e1) / 20
        fl = 2.0 * m * n * k
        print(f"{m}x{n}x{k}: gemm_bf16 {t_ours * 1e3:8.1f} us {fl / t_ours / 1e9:6.0f} TFLOP/s | "
              f"hipBLASLt {t_lib * 1e3:8.1f} us {fl / t_lib / 1e9:6.0f} TFLOP/s", flush=True)
        del a, b, bt, c
    dev.close()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--pmc-probe", choices=["config2", "config3", "config4", "config5", "all"],
                    help="run the copy calibration and the workload for rocprofv3 --pmc, then exit")
    ap.add_argument("--gemm-probe", nargs="*", metavar="MxNxK",
                    help="time the bf16 training GEMM beside hipBLASLt on these shapes (default: the "
                         "training step's), then exit")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    args = ap.parse_args()
    if args.pmc_probe:
        pmc_probe(args.pmc_probe)
        return
    if args.gemm_probe is not None:
        shapes = [tuple(int(v) for v in s.split("x")) for s in args.gemm_probe] or [
            (8192, 3072, 3072), (8192, 4096, 1024), (8192, 1024, 4096), (1024, 4096, 8192),
            (16384, 7168, 2048), (16384, 1024, 3584), (8192, 8192, 8192)]
        gemm_probe(shapes)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build runs on a single MI355X "
              "(no collectives); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import catnn_amd
    from catnn_amd import configs

    dev = catnn_amd.Device(0)
    name, hbm, cus = dev.info()
    log(f"device {name}, {hbm / 2**30:.0f} GiB HBM, {cus} CUs")

    wl = configs.config2()
    log("config 2 built")
    prog = catnn_amd.Program(dev, wl.graph)
    ms, wall, timings = time_program(dev, prog, wl.x, args.steps, args.warmup)
    value = wl.flops / (ms / 1e3) / 1e9
    gemm = [t for t in timings if t[1] == "linear"]
    launches = sum(t[2] for t in gemm)
    gemm_ms = sum(t[3] for t in gemm) / max(launches, 1)
    M, K, N = 8192, 4096, 16384
    per_launch = 2 * M * K * N  # both Linear layers do the same FLOPs
    achieved = per_launch / (gemm_ms / 1e3) / 1e12
    log(f"config 2: {ms:.3f} ms/step, {value:.0f} GFLOP/s; GEMM {gemm_ms:.3f} ms/launch "
        f"({achieved:.1f} TFLOP/s); steps {[(t[0], round(t[3] / max(t[2], 1), 3)) for t in timings]}")
    prog.free()

    result = {
        "metric": "IR fwd GFLOP/s",
        "value": round(value, 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64/Box-Muller, N(0,1/fan_in) weights)",
        "config": {"workload": "config2: MLP forward 8192x(4096->16384->4096), bias+GELU, fp32, "
                               "IR program via .catnn spec path",
                   "batch": M, "layers": [K, N, K], "activation": "gelu"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "gemm_dma_kernel<4 stages> 128x128x16 direct-to-LDS (fp32 MFMA 32x32x2)",
                     "per_launch_flop": per_launch, "avg_launch_ms": round(gemm_ms, 4)},
    }

    if not args.no_secondary:
        sec = {}
        w4 = configs.config4()
        p4 = catnn_amd.Program(dev, w4.graph)
        ms4, _, t4 = time_program(dev, p4, w4.x, max(3, args.steps // 2), 2)
        sec["moe_layer_config4"] = {
            "tokens_per_s": round(w4.tokens / (ms4 / 1e3)), "ms_per_step": round(ms4, 4),
            "GFLOP_per_s": round(w4.flops / (ms4 / 1e3) / 1e9, 1),
            "mfma_frac": round(w4.flops / (ms4 / 1e3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4)}
        p4.free()
        log(f"config 4: {ms4:.3f} ms/step")
        if not args.no_cpu_baseline:
            cb = cpu_baseline_moe(w4, args.cpu_seconds)
            sec["moe_layer_config4"]["cpu_baseline"] = cb
            sec["moe_layer_config4"]["vs_cpu"] = round(sec["moe_layer_config4"]["tokens_per_s"] / cb["value"], 1)
            log(f"config 4 cpu baseline: {cb}")
        del w4
        w3 = configs.config3()
        p3 = catnn_amd.Program(dev, w3.graph)
        ms3, _, t3 = time_program(dev, p3, w3.x, max(3, args.steps // 2), 2)
        sec["prenorm_block_config3"] = {
            "ms_per_step": round(ms3, 4), "GFLOP_per_s": round(w3.flops / (ms3 / 1e3) / 1e9, 1),
            "steps_ms": {t[0]: round(t[3] / max(t[2], 1), 4) for t in t3}}
        p3.free()
        del w3
        log(f"config 3: {ms3:.3f} ms/step")
        sec["train_step_config5"] = time_train_step(dev, max(3, args.steps // 2), 2)
        sec["train_step_config5_adam"] = time_train_step(dev, max(3, args.steps // 4), 1, opt="adam")
        sec["mixtral_decoder"] = time_mixtral(dev, max(3, args.steps // 4), 2)
        result["secondary"] = sec

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_mlp(wl, args.cpu_seconds)
        log(f"cpu baseline: {result['cpu_baseline']}")
    dev.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
