"""Benchmark of the quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload (one "step"): the linear layers of one Qwen2.5-0.5B decode step at
M=1, 4-bit group-64 affine weights with bf16 scales/biases:
24 layers x {q 896->896, k 896->128, v 896->128, o 896->896, gate 896->4864,
up 896->4864, down 4864->896} + lm_head 896->151936.  Weights are random
(seeded, generated on the device); x ~ N(0,1) is drawn per layer input, as in
the model: q, k and v read the attention input, gate and up the MLP input,
o and down their own.  The step runs q/k/v and gate/up as one grouped call
each (miqmm_quantized_matmul_grouped), 97 launches; the same step with one
launch per projection (169 launches) is reported beside it.  The launches of
a step are captured once per weight replica into a HIP graph and replayed;
three replicas (838 MB) rotate so consecutive steps never find their weights
in the 256 MB Infinity Cache.

Printed: one JSON line with the step throughput (value, GB/s), the roofline
of the dominant kernel (the lm_head GEMV, 76.9 MB per launch), headline
numbers (qmv 4096x14336 at M=1, qmm at M=2048) and the CPU baseline (the C
oracle's fp32 path on the host cores, same step, one replica).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sen-mlx_amd"))

METRIC = "qmv GB/s (% of HBM peak) at M=1; qmm TFLOP/s at M=2048, 4-bit g64"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

QWEN05_LAYER = [("q", 896, 896), ("k", 128, 896), ("v", 128, 896), ("o", 896, 896),
                ("gate", 4864, 896), ("up", 4864, 896), ("down", 896, 4864)]
QWEN05_LAYERS = 24
LM_HEAD = ("lm_head", 151936, 896)


def qbytes(M, N, K, bits=4, g=64, sb=2, xb=2, yb=2):
    """algorithmic bytes: packed codes + scales + biases + x + y"""
    return N * K * bits // 8 + 2 * N * (K // g) * sb + M * K * xb + M * N * yb


def group_bytes(Ns, K, M=1):
    """a grouped call reads x once: the projections' bytes minus the repeated x"""
    return sum(qbytes(M, N, K) for N in Ns) - (len(Ns) - 1) * M * K * 2


def step_shapes():
    shapes = []
    for layer in range(QWEN05_LAYERS):
        for name, N, K in QWEN05_LAYER:
            shapes.append((f"l{layer}.{name}", N, K))
    shapes.append(LM_HEAD)
    return shapes


class Proj:
    __slots__ = ("name", "N", "K", "x", "w", "s", "b", "y")


def make_replica(miqmm, torch, replica, shapes):
    projs = []
    for i, (name, N, K) in enumerate(shapes):
        p = Proj()
        p.name, p.N, p.K = name, N, K
        p.x, p.w, p.s, p.b = miqmm.synth_problem(1, N, K, 64, 4, seed=replica, stream_id=i)
        p.y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
        projs.append(p)
    # one x per layer input: k and v read q's input, up reads gate's
    for layer in range(QWEN05_LAYERS):
        q, k, v, o, gate, up, down = projs[layer * 7:layer * 7 + 7]
        k.x = v.x = q.x
        up.x = gate.x
    return projs


def run_step(miqmm, projs):
    """one launch per projection (169)"""
    for p in projs:
        miqmm.quantized_matmul(p.x, p.w, p.s, p.b, True, 64, 4, out=p.y)


def run_step_grouped(miqmm, projs):
    """q/k/v and gate/up as one grouped call each (97 launches)"""
    for layer in range(QWEN05_LAYERS):
        q, k, v, o, gate, up, down = projs[layer * 7:layer * 7 + 7]
        for grp in ((q, k, v), (o,), (gate, up), (down,)):
            if len(grp) == 1:
                p = grp[0]
                miqmm.quantized_matmul(p.x, p.w, p.s, p.b, True, 64, 4, out=p.y)
            else:
                miqmm.quantized_matmul_grouped([p.x for p in grp], [p.w for p in grp], [p.s for p in grp],
                                               [p.b for p in grp], 64, 4, outs=[p.y for p in grp])
    p = projs[-1]
    miqmm.quantized_matmul(p.x, p.w, p.s, p.b, True, 64, 4, out=p.y)


def step_bytes_grouped():
    per_layer = group_bytes([896, 128, 128], 896) + qbytes(1, 896, 896) + group_bytes([4864, 4864], 896) + \
        qbytes(1, 896, 4864)
    return QWEN05_LAYERS * per_layer + qbytes(1, LM_HEAD[1], LM_HEAD[2])


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def time_graphs(torch, graphs, reps):
    """events on the replay stream around `reps` replays; returns seconds"""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(reps):
        graphs[i % len(graphs)].replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3


def kernel_roofline(miqmm, torch, N, K, M, replicas, launches_per_graph, reps, g=64, bits=4, sb_dtype=None):
    """average duration of back-to-back launches of one shape over rotating
    weight replicas (cold in the Infinity Cache); returns (avg_s, bytes_per_launch)"""
    sb_dtype = sb_dtype or torch.bfloat16
    ydt = miqmm.result_type(torch.bfloat16, sb_dtype)
    sets = []
    for r in range(replicas):
        x, w, s, b = miqmm.synth_problem(M, N, K, g, bits, sb_dtype=sb_dtype, seed=100 + r, stream_id=N + K)
        sets.append((x, w, s, b, torch.empty((M, N), dtype=ydt, device="cuda")))

    def body():
        for i in range(launches_per_graph):
            x, w, s, b, y = sets[i % replicas]
            miqmm.quantized_matmul(x, w, s, b, True, g, bits, out=y)

    body()
    torch.cuda.synchronize()
    graph = capture(torch, body)
    graph.replay()
    t = time_graphs(torch, [graph], reps)
    del sets
    return t / (reps * launches_per_graph), qbytes(M, N, K, bits, g, yb=4 if ydt == torch.float32 else 2)


def qmm_tflops(miqmm, torch, M, N, K, iters):
    x, w, s, b = miqmm.synth_problem(M, N, K, 64, 4, seed=7, stream_id=N + K)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    for _ in range(2):
        miqmm.quantized_matmul(x, w, s, b, True, 64, 4, out=y)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        miqmm.quantized_matmul(x, w, s, b, True, 64, 4, out=y)
    end.record()
    torch.cuda.synchronize()
    t = start.elapsed_time(end) / 1e3 / iters
    return 2.0 * M * N * K / t / 1e12, t


def dense_bf16_tflops(torch, M, N, K, iters):
    """hipBLASLt dense bf16 GEMM of the same shape (cross-check of the MFMA ceiling)"""
    a = torch.randn((M, K), dtype=torch.bfloat16, device="cuda")
    bt = torch.randn((N, K), dtype=torch.bfloat16, device="cuda")
    for _ in range(2):
        torch.matmul(a, bt.t())
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        torch.matmul(a, bt.t())
    end.record()
    torch.cuda.synchronize()
    t = start.elapsed_time(end) / 1e3 / iters
    return 2.0 * M * N * K / t / 1e12


def cpu_baseline(miqmm, torch, projs, budget_s=15.0):
    """the C oracle's fp32 path (OpenMP over N) on the host cores, on the same
    decode step (one replica), repeated until ~budget_s of CPU time"""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    O.build_c_oracle()
    threads = min(16, os.cpu_count() or 1)
    host = []
    for p in projs:
        host.append((p.x.view(torch.int16).cpu().numpy().view(np.uint16),
                     p.w.cpu().numpy().view(np.uint32),
                     p.s.view(torch.int16).cpu().numpy().view(np.uint16),
                     p.b.view(torch.int16).cpu().numpy().view(np.uint16), p.N, p.K))
    step_bytes = sum(qbytes(1, N, K) for (_, _, _, _, N, K) in host)
    steps = 0
    t0 = time.perf_counter()
    while True:
        for (x, w, s, b, N, K) in host:
            O.c_qmm_f32(x, w, s, b, 1, N, K, 64, 4, nthreads=threads)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": round(step_bytes * steps / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{steps} full decode steps (169 GEMVs, {step_bytes} B each) of one weight replica, "
                      f"C oracle fp32 path (oracle/miqmm_oracle.c, gcc -O3 -fopenmp), {threads} threads, "
                      f"{el:.1f} s; MLX's CPU backend is not available offline",
            "ms_per_step": round(el / steps * 1e3, 3)}


def graph_avg(torch, fns, launches, reps):
    """average time of one call, over a HIP graph of `launches` calls cycling
    through `fns` (one per weight replica, so the weights come cold from HBM)"""
    for f in fns:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(launches):
            fns[i % len(fns)]()
    g.replay()
    torch.cuda.synchronize()
    t = time_graphs(torch, [g], reps)
    return t / (reps * launches)


def small_m_and_large_vocab(miqmm, torch):
    """the GEMV routes beyond the decode step: speculative-verify / small-batch
    rows M in {1, 2, 4, 8, 16} on the Llama-3-8B projections (4-bit g64), and
    the Gemma-3-27B-class head K = 5376, N = 262144 at M in {1, 8} with fp16
    scales, 4-bit g32 and 8-bit g64; weights cold (rotating replicas)"""
    res = {}
    for (N, K) in [(6144, 4096), (4096, 4096), (14336, 4096), (4096, 14336)]:
        for M in (1, 2, 4, 8, 16):
            avg, nb = kernel_roofline(miqmm, torch, N, K, M, replicas=10, launches_per_graph=40, reps=3)
            res[f"qmv_m{M}_{K}to{N}"] = {"us": round(avg * 1e6, 2), "GB/s": round(nb / avg / 1e9, 1),
                                         "frac_hbm": round(nb / avg / 1e9 / HBM_PEAK_GBS, 4)}
        torch.cuda.empty_cache()
    for (bits, g) in [(4, 32), (8, 64)]:
        for M in (1, 8):
            avg, nb = kernel_roofline(miqmm, torch, 262144, 5376, M, replicas=2, launches_per_graph=8, reps=3,
                                      g=g, bits=bits, sb_dtype=torch.float16)
            res[f"head_5376to262144_m{M}_{bits}bit_g{g}_f16"] = {
                "us": round(avg * 1e6, 2), "GB/s": round(nb / avg / 1e9, 1),
                "frac_hbm": round(nb / avg / 1e9 / HBM_PEAK_GBS, 4)}
        torch.cuda.empty_cache()
    return res


def moe_and_embedding(miqmm, torch):
    """the rows after the quantized projections: gather_qmm on DeepSeek-V2-Lite's
    routed experts (64 experts, top-6, hidden 2048, expert inter 1408, 4-bit g64)
    and the quantized embedding lookup of Qwen2.5-0.5B (151936 x 896)"""
    E, H, I, top_k, g = 64, 2048, 1408, 6, 64
    res = {}
    stacks = []
    for r in range(4):  # 4 layers' experts: 4 x 3 x 92 MB, cold in the 256 MB cache
        gate = [t.reshape(E, I, -1) for t in miqmm.synth_problem(1, E * I, H, g, 4, seed=60 + r, stream_id=1)[1:]]
        down = [t.reshape(E, H, -1) for t in miqmm.synth_problem(1, E * H, I, g, 4, seed=70 + r, stream_id=2)[1:]]
        stacks.append((gate, down))
    for T in (1, 16, 64, 1024):
        gen = torch.Generator().manual_seed(T)
        idx = torch.stack([torch.randperm(E, generator=gen)[:top_k] for _ in range(T)]).to(torch.int32).cuda()
        x = torch.randn(T, 1, 1, H, device="cuda").to(torch.bfloat16)
        h = torch.randn(T, top_k, 1, I, device="cuda").to(torch.bfloat16)
        yg = torch.empty(T, top_k, 1, I, device="cuda", dtype=torch.bfloat16)
        yd = torch.empty(T, top_k, 1, H, device="cuda", dtype=torch.bfloat16)
        n = 64 if T < 1024 else 16
        tg = graph_avg(torch, [lambda s=s: miqmm.gather_qmm(x, *s[0], idx, True, g, 4, out=yg) for s in stacks],
                       n, 5)
        td = graph_avg(torch, [lambda s=s: miqmm.gather_qmm(h, *s[1], idx, True, g, 4, out=yd) for s in stacks],
                       n, 5)
        fl = 2 * T * top_k * H * I
        S = T * top_k
        path = ("expert-grouped tiled matmul" if S >= miqmm.GROUPED_MIN_PER_EXPERT * E else
                "expert-grouped MFMA GEMV" if S >= miqmm.GROUPED_GEMV_MIN_PER_EXPERT * E else
                "per-selection v_dot2 GEMV")
        # bytes the path must stream: each selection's expert (per-selection),
        # or each distinct selected expert once (grouped)
        streams = S if path.startswith("per-selection") else len(set(idx.flatten().tolist()))
        nb = streams * qbytes(1, I, H)
        res[f"gather_qmm_T{T}"] = {"gate_2048to1408_us": round(tg * 1e6, 2), "down_1408to2048_us": round(td * 1e6, 2),
                                   "gate_TFLOP/s": round(fl / tg / 1e12, 1), "path": path,
                                   "weight_bytes": nb, "gate_GB/s": round(nb / tg / 1e9, 1)}
    del stacks
    V, K = 151936, 896
    tabs = [miqmm.synth_problem(1, V, K, g, 4, seed=80 + r, stream_id=3)[1:] for r in range(3)]
    for T in (1, 2048):
        ids = torch.randint(0, V, (T,), device="cuda", dtype=torch.int32)
        out = torch.empty(T, K, device="cuda", dtype=torch.bfloat16)
        t = graph_avg(torch, [lambda tb=tb: miqmm.quantized_embedding(ids, *tb, g, 4, out=out) for tb in tabs], 64, 5)
        nb = T * (K // 2 + 2 * (K // g) * 2 + K * 2)
        res[f"embedding_T{T}"] = {"us": round(t * 1e6, 2), "bytes": nb, "GB/s": round(nb / t / 1e9, 1)}
    return res


PROFILE_DIR = os.path.join(ROOT, "profiles")
ROOFLINE_PROFILE = os.path.join(PROFILE_DIR, "qmv_lm_head_151936x896_m1.md")


def measured_traffic(path=ROOFLINE_PROFILE):
    """HBM bytes per launch of the roofline kernel from its committed rocprofv3
    summary (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy), or None"""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def profile_section(miqmm, torch, target):
    """one measured section alone, so a rocprofv3 run of this command holds only
    its kernel: the roofline launches, the qmv or qmm headline, or a plain
    512 MiB device copy (the FETCH_SIZE / WRITE_SIZE calibration)"""
    if target == "roofline":
        avg, nb = kernel_roofline(miqmm, torch, LM_HEAD[1], LM_HEAD[2], 1, replicas=8,
                                  launches_per_graph=64, reps=8)
        return {"section": target, "shape": "M=1 N=151936 K=896", "timed_launches": 512,
                "avg_launch_us": round(avg * 1e6, 3), "bytes_per_launch": nb, "GB/s": round(nb / avg / 1e9, 1)}
    if target == "qmv":
        avg, nb = kernel_roofline(miqmm, torch, 14336, 4096, 1, replicas=24, launches_per_graph=96, reps=6)
        return {"section": target, "shape": "M=1 N=14336 K=4096", "timed_launches": 576,
                "avg_launch_us": round(avg * 1e6, 3), "bytes_per_launch": nb, "GB/s": round(nb / avg / 1e9, 1)}
    if target == "qmm":
        tf, tsec = qmm_tflops(miqmm, torch, 2048, 14336, 4096, iters=10)
        return {"section": target, "shape": "M=2048 N=14336 K=4096", "timed_launches": 10,
                "avg_launch_us": round(tsec * 1e6, 2), "TFLOP/s": round(tf, 1)}
    n = 512 << 20
    a = torch.empty(n // 4, dtype=torch.int32, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    return {"section": target, "bytes_read_per_launch": n, "bytes_written_per_launch": n, "launches": 4}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replicas", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-headline", action="store_true")
    ap.add_argument("--profile-target", choices=["roofline", "qmv", "qmm", "copy"], default=None,
                    help="run only this measured section and print its figures (for rocprofv3 summaries)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the quantized-matmul path has no multi-GPU leg here "
              "(sharding is described in DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import miqmm

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (torch.cuda.is_available() is False)", file=sys.stderr)
        sys.exit(2)
    miqmm.lib()
    torch.cuda.set_device(0)
    if args.profile_target:
        print(json.dumps(profile_section(miqmm, torch, args.profile_target)), flush=True)
        return

    shapes = step_shapes()
    step_bytes = step_bytes_grouped()
    step_bytes_single = sum(qbytes(1, N, K) for _, N, K in shapes)
    replicas = [make_replica(miqmm, torch, r, shapes) for r in range(args.replicas)]
    for projs in replicas:  # eager warm-up (loads the code objects before capture)
        run_step(miqmm, projs)
        run_step_grouped(miqmm, projs)
    torch.cuda.synchronize()
    graphs = [capture(torch, (lambda p=projs: run_step_grouped(miqmm, p))) for projs in replicas]
    time_graphs(torch, graphs, max(args.warmup, 1))
    print(f"# timing {args.steps} decode steps (97 launches each)", file=sys.stderr, flush=True)
    t = time_graphs(torch, graphs, args.steps)
    gbs = step_bytes * args.steps / t / 1e9
    ms_per_step = t / args.steps * 1e3
    del graphs
    graphs = [capture(torch, (lambda p=projs: run_step(miqmm, p))) for projs in replicas]
    time_graphs(torch, graphs, max(args.warmup, 1))
    t1 = time_graphs(torch, graphs, args.steps)
    single = {"us_per_step": round(t1 / args.steps * 1e6, 2), "launches": len(shapes),
              "GB/s": round(step_bytes_single * args.steps / t1 / 1e9, 2), "bytes_per_step": step_bytes_single}

    # dominant kernel of the step: the lm_head GEMV (N=151936, K=896)
    lm_avg, lm_bytes = kernel_roofline(miqmm, torch, LM_HEAD[1], LM_HEAD[2], 1, replicas=8,
                                       launches_per_graph=64, reps=8)
    lm_gbs = lm_bytes / lm_avg / 1e9
    out = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "accumulate": "fp32",
        "data": "synthetic (seeded on-device generator; random-init 4-bit g64 weights)",
        "config": {"workload": "qwen2.5-0.5b decode step, linear layers only: 24 x {q 896->896, k 896->128, "
                               "v 896->128, o 896->896, gate 896->4864, up 896->4864, down 4864->896} + "
                               "lm_head 896->151936; M=1, 4-bit, group 64, bf16 x/scales/biases/y; "
                               "q/k/v and gate/up as one grouped call each",
                   "launches_per_step": 97, "bytes_per_step": step_bytes,
                   "weight_replicas": args.replicas, "hip_graph": True},
        "roofline": {"kernel": "lm_head 896->151936 M=1 (qmvx_kernel<4, 0, 1, 6>: 4-bit, bf16 scales, 1 row of x, group 64)", "bound": "hbm",
                     "achieved": round(lm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(lm_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "avg_launch_us": round(lm_avg * 1e6, 3), "bytes_per_launch": lm_bytes},
    }
    out["step_one_launch_per_projection"] = single
    print(f"# step {ms_per_step * 1e3:.1f} us, {gbs:.1f} GB/s (one launch per projection: "
          f"{single['us_per_step']:.1f} us); lm_head {lm_avg * 1e6:.2f} us {lm_gbs:.1f} GB/s",
          file=sys.stderr, flush=True)
    del graphs, replicas
    torch.cuda.empty_cache()

    if not args.no_headline:
        head = {}
        avg, nb = kernel_roofline(miqmm, torch, 14336, 4096, 1, replicas=24, launches_per_graph=96, reps=6)
        head["qmv_m1_4096x14336"] = {"us": round(avg * 1e6, 3), "GB/s": round(nb / avg / 1e9, 1),
                                     "frac_hbm": round(nb / avg / 1e9 / HBM_PEAK_GBS, 4), "bytes": nb}
        print(f"# qmv 4096x14336 M=1: {avg * 1e6:.2f} us {nb / avg / 1e9:.1f} GB/s", file=sys.stderr, flush=True)
        avg, nb = kernel_roofline(miqmm, torch, 4096, 14336, 1, replicas=24, launches_per_graph=96, reps=6)
        head["qmv_m1_14336x4096"] = {"us": round(avg * 1e6, 3), "GB/s": round(nb / avg / 1e9, 1),
                                     "frac_hbm": round(nb / avg / 1e9 / HBM_PEAK_GBS, 4), "bytes": nb}
        print(f"# qmv 14336x4096 M=1: {avg * 1e6:.2f} us {nb / avg / 1e9:.1f} GB/s", file=sys.stderr, flush=True)
        for (N, K) in [(14336, 4096), (4096, 14336), (6144, 4096), (4096, 4096)]:
            tf, tsec = qmm_tflops(miqmm, torch, 2048, N, K, iters=10)
            head[f"qmm_m2048_{K}to{N}"] = {"TFLOP/s": round(tf, 1), "us": round(tsec * 1e6, 1),
                                           "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
            print(f"# qmm M=2048 {K}->{N}: {tf:.1f} TFLOP/s ({tsec * 1e6:.1f} us)", file=sys.stderr, flush=True)
        head["dense_bf16_gemm_m2048_4096to14336_torch"] = {
            "TFLOP/s": round(dense_bf16_tflops(torch, 2048, 14336, 4096, 10), 1)}
        out["headline"] = head
        torch.cuda.empty_cache()
        out["small_m_and_large_vocab"] = small_m_and_large_vocab(miqmm, torch)
        print(f"# small M / large vocab: {json.dumps(out['small_m_and_large_vocab'])}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        out["moe_and_embedding"] = moe_and_embedding(miqmm, torch)
        print(f"# moe/embedding: {json.dumps(out['moe_and_embedding'])}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        projs = make_replica(miqmm, torch, 0, shapes)
        out["cpu_baseline"] = cpu_baseline(miqmm, torch, projs)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
