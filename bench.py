"""Benchmark of the quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-headline]
    python bench.py --profile-target {step,qkv,o,gateup,down,lm_head,qmv,qmv_down,config0,qmv_m8,qmv_m8_down,
                                      qmv_m16,qmv_m16_down,qmm,read33,read77,copy}

Workload (one "step", the line's `value`): the linear layers of one
Qwen2.5-0.5B decode step at M=1, 4-bit group-64 affine weights with bf16
scales/biases: 24 layers x {q 896->896, k 896->128, v 896->128, o 896->896,
gate 896->4864, up 896->4864, down 4864->896} + lm_head 896->151936.  Weights
are random (seeded, generated on the device); x ~ N(0,1) is drawn per layer
input, as in the model: q, k and v read the attention input, gate and up the
MLP input, o and down their own.  q/k/v and gate/up run as one grouped call
each, their weights stored contiguously per layer (as a loader that fuses
them lays them out; the same step on separately allocated weights, and with
one launch per projection, is reported beside it): 97 launches per step,
captured once per weight replica into a HIP graph; three replicas (838 MB) rotate so no step finds its weights in the
256 MB Infinity Cache.  W untimed steps, then exactly K timed steps between
two device synchronizations, with HIP events on the replay stream.

Every kernel-level figure follows one protocol: the calls are captured into
a HIP graph cycling through enough distinct weight replicas that the bytes
read exceed 512 MB (so nothing is served from the Infinity Cache), the graph
is replayed at least 20 times with events around each replay, and the
median per-call time is reported.  `roofline` is the step's kernel with the
most time per step, measured this way on the step's own shapes.

Printed: one JSON line (stdout) with the step throughput, the roofline of the
dominant kernel, the headline numbers (qmv at M=1 on 4096x14336 and
14336x4096 beside a bare streaming read of the same bytes; qmm at M=2048 and
at the reference's prefill chunk M=512; configuration 0), the small-M and
large-vocab sweeps, the expert gather and embedding rows, and the CPU
baseline (the C oracle's fp32 path on the host cores, same decode step).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sen-mlx_amd"))

METRIC = "qmv GB/s (% of HBM peak) at M=1; qmm TFLOP/s at M=2048, 4-bit g64"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
COLD_BYTES = 600e6   # distinct bytes one timed graph cycles through (> 2 x the 256 MB Infinity Cache)
REPS = 20            # timed graph replays per figure (median reported)

QWEN05_LAYER = [("q", 896, 896), ("k", 128, 896), ("v", 128, 896), ("o", 896, 896),
                ("gate", 4864, 896), ("up", 4864, 896), ("down", 896, 4864)]
QWEN05_LAYERS = 24
LM_HEAD = ("lm_head", 151936, 896)
SHAPES_8B = [(6144, 4096), (4096, 4096), (14336, 4096), (4096, 14336)]  # (N, K)


def qbytes(M, N, K, bits=4, g=64, sb=2, xb=2, yb=2):
    """algorithmic bytes: packed codes + scales + biases + x + y"""
    return N * K * bits // 8 + 2 * N * (K // g) * sb + M * K * xb + M * N * yb


def group_bytes(Ns, K, M=1):
    """a grouped call reads x once: the projections' bytes minus the repeated x"""
    return sum(qbytes(M, N, K) for N in Ns) - (len(Ns) - 1) * M * K * 2


# the step's launch types: (name, output rows of each grouped projection, K, launches per step)
STEP_TYPES = [("qkv", [896, 128, 128], 896, QWEN05_LAYERS), ("o", [896], 896, QWEN05_LAYERS),
              ("gateup", [4864, 4864], 896, QWEN05_LAYERS), ("down", [896], 4864, QWEN05_LAYERS),
              ("lm_head", [LM_HEAD[1]], LM_HEAD[2], 1)]


def step_shapes():
    shapes = []
    for layer in range(QWEN05_LAYERS):
        for name, N, K in QWEN05_LAYER:
            shapes.append((f"l{layer}.{name}", N, K))
    shapes.append(LM_HEAD)
    return shapes


class Proj:
    __slots__ = ("name", "N", "K", "x", "w", "s", "b", "y")


def split_rows(miqmm, torch, Ns, K, seed, stream_id):
    """projections stored one after another, as a loader that fuses q/k/v or
    gate/up lays them out: one generated matrix of sum(Ns) rows, returned as
    row views (x, [(w, s, b) per projection])"""
    x, w, s, b = miqmm.synth_problem(1, sum(Ns), K, 64, 4, seed=seed, stream_id=stream_id)
    views, o = [], 0
    for N in Ns:
        views.append((w[o:o + N], s[o:o + N], b[o:o + N]))
        o += N
    return x, views


def make_replica(miqmm, torch, replica, shapes, fused=True):
    """one set of the step's weights; fused: each layer's q/k/v and gate/up
    stored contiguously (row views of one matrix), else every projection in
    its own allocation"""
    projs = []
    for i, (name, N, K) in enumerate(shapes):
        p = Proj()
        p.name, p.N, p.K = name, N, K
        if not fused or not (name.endswith((".q", ".k", ".v", ".gate", ".up"))):
            p.x, p.w, p.s, p.b = miqmm.synth_problem(1, N, K, 64, 4, seed=replica, stream_id=i)
        p.y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
        projs.append(p)
    for layer in range(QWEN05_LAYERS):
        q, k, v, o, gate, up, down = projs[layer * 7:layer * 7 + 7]
        if fused:
            for grp, sid in (((q, k, v), layer * 7), ((gate, up), layer * 7 + 4)):
                x, views = split_rows(miqmm, torch, [p.N for p in grp], grp[0].K, replica, sid)
                for p, (w, s_, b) in zip(grp, views):
                    p.x, p.w, p.s, p.b = x, w, s_, b
        # one x per layer input: k and v read q's input, up reads gate's
        k.x = v.x = q.x
        up.x = gate.x
    return projs


def call(miqmm, p):
    miqmm.quantized_matmul(p.x, p.w, p.s, p.b, True, 64, 4, out=p.y)


def call_group(miqmm, grp):
    if len(grp) == 1:
        call(miqmm, grp[0])
    else:
        miqmm.quantized_matmul_grouped([p.x for p in grp], [p.w for p in grp], [p.s for p in grp],
                                       [p.b for p in grp], 64, 4, outs=[p.y for p in grp])


def run_step(miqmm, projs):
    """one launch per projection (169)"""
    for p in projs:
        call(miqmm, p)


def run_step_grouped(miqmm, projs):
    """q/k/v and gate/up as one grouped call each (97 launches)"""
    for layer in range(QWEN05_LAYERS):
        q, k, v, o, gate, up, down = projs[layer * 7:layer * 7 + 7]
        for grp in ((q, k, v), (o,), (gate, up), (down,)):
            call_group(miqmm, grp)
    call(miqmm, projs[-1])


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
    """events on the replay stream around `reps` replays (cycling `graphs`); seconds"""
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


def graph_median(torch, fns, launches, reps=REPS):
    """median over `reps` replays of the time per call, one graph of `launches`
    calls cycling through `fns` (one per weight replica); seconds"""
    for f in fns:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(launches):
            fns[i % len(fns)]()
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    times = []
    for _ in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        g.replay()
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end) / 1e3 / launches)
    del g
    times.sort()
    return times[len(times) // 2]


def replicas_for(nbytes, minimum=2):
    return max(minimum, math.ceil(COLD_BYTES / nbytes))


def gemv_line(miqmm, torch, M, N, K, g=64, bits=4, sb_dtype=None, reps=REPS):
    """per-call median of one shape over cold rotating replicas: (seconds, algorithmic bytes)"""
    sb_dtype = sb_dtype or torch.bfloat16
    ydt = miqmm.result_type(torch.bfloat16, sb_dtype)
    nb = qbytes(M, N, K, bits, g, yb=4 if ydt == torch.float32 else 2)
    sets = []
    for r in range(replicas_for(nb)):
        x, w, s, b = miqmm.synth_problem(M, N, K, g, bits, sb_dtype=sb_dtype, seed=100 + r, stream_id=N + K)
        sets.append((x, w, s, b, torch.empty((M, N), dtype=ydt, device="cuda")))
    fns = [lambda t=t: miqmm.quantized_matmul(t[0], t[1], t[2], t[3], True, g, bits, out=t[4]) for t in sets]
    sec = graph_median(torch, fns, max(len(fns), 40), reps)
    del sets, fns
    return sec, nb


def read_ceiling(miqmm, torch, nbytes, reps=REPS):
    """a bare streaming read of nbytes (rounded up to 16 KiB) over cold rotating buffers"""
    nb = (nbytes + 16383) // 16384 * 16384
    bufs = [torch.full((nb,), r + 1, dtype=torch.uint8, device="cuda") for r in range(replicas_for(nb))]
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    fns = [lambda b=b: miqmm.stream_read(b, sink) for b in bufs]
    sec = graph_median(torch, fns, max(len(fns), 40), reps)
    del bufs
    return sec, nb


def line(sec, nb):
    gbs = nb / sec / 1e9
    return {"us": round(sec * 1e6, 3), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "bytes": nb}


def step_type_line(miqmm, torch, Ns, K, reps=REPS, fused=True):
    """one of the step's launch types on its own: grouped projections (shared x;
    fused: stored contiguously, as in the step) or a single one, cold
    replicas; (seconds per launch, algorithmic bytes per launch)"""
    nb = group_bytes(Ns, K) if len(Ns) > 1 else qbytes(1, Ns[0], K)
    groups = []
    for r in range(replicas_for(nb)):
        grp = []
        if fused and len(Ns) > 1:
            x, views = split_rows(miqmm, torch, Ns, K, 200 + r, sum(Ns))
        else:
            x, views = None, [None] * len(Ns)
        for j, (N, v) in enumerate(zip(Ns, views)):
            p = Proj()
            p.N, p.K = N, K
            if v is None:
                p.x, p.w, p.s, p.b = miqmm.synth_problem(1, N, K, 64, 4, seed=200 + r, stream_id=10 * j + N)
                x = p.x if x is None else x
            else:
                p.w, p.s, p.b = v
            p.x = x
            p.y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
            grp.append(p)
        groups.append(grp)
    fns = [lambda grp=grp: call_group(miqmm, grp) for grp in groups]
    sec = graph_median(torch, fns, max(len(fns), 64), reps)
    del groups, fns
    return sec, nb


def qmm_line(miqmm, torch, M, N, K, launches=50, reps=REPS, check=False):
    """tiled matmul, graph-timed over `launches` calls (two weight replicas),
    median of `reps` replays; optional elementwise check against a float32
    reference (exactly dequantized W, float32 matmul)"""
    sets = []
    for r in range(2):
        x, w, s, b = miqmm.synth_problem(M, N, K, 64, 4, seed=7 + r, stream_id=N + K)
        sets.append((x, w, s, b, torch.empty((M, N), dtype=torch.bfloat16, device="cuda")))
    fns = [lambda t=t: miqmm.quantized_matmul(t[0], t[1], t[2], t[3], True, 64, 4, out=t[4]) for t in sets]
    sec = graph_median(torch, fns, launches, reps)
    tf = 2.0 * M * N * K / sec / 1e12
    out = {"TFLOP/s": round(tf, 1), "us": round(sec * 1e6, 2), "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4),
           "route": miqmm.query_route(M, N, K, 64, 4)[1]}
    if check:
        x, w, s, b, y = sets[0]
        miqmm.quantized_matmul(x, w, s, b, True, 64, 4, out=y)
        wd = miqmm.dequantize(w, s, b, 64, 4, dtype=torch.float32)
        prev = torch.backends.cuda.matmul.allow_tf32
        torch.backends.cuda.matmul.allow_tf32 = False
        ref = x.float() @ wd.T
        torch.backends.cuda.matmul.allow_tf32 = prev
        err = (y.float() - ref).abs()
        out["elem_ok_frac"] = round(((err <= 1e-3 + 1e-2 * ref.abs()).float().mean()).item(), 5)
        out["max_err_over_max_ref"] = round((err.max() / ref.abs().max()).item(), 6)
        del wd, ref, err
    del sets, fns
    return out


def dense_bf16_tflops(torch, M, N, K, launches=50, reps=REPS):
    """hipBLASLt dense bf16 GEMM of the same shape (cross-check of the MFMA ceiling)"""
    a = torch.randn((M, K), dtype=torch.bfloat16, device="cuda")
    bt = torch.randn((N, K), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    sec = graph_median(torch, [lambda: torch.matmul(a, bt.t(), out=y)], launches, reps)
    return round(2.0 * M * N * K / sec / 1e12, 1)


def host_info():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "model": model,
            "affinity": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None}


def cpu_baseline(miqmm, torch, projs, budget_s=15.0):
    """the C oracle's fp32 path (OpenMP over N) on the host cores, on the same
    decode step (one replica), repeated until ~budget_s of wall time"""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    O.build_c_oracle()
    info = host_info()
    # the host's CPU share: OMP_NUM_THREADS when set (a shared host's scheduler sets it), else every core
    # available
    threads = int(os.environ.get("OMP_NUM_THREADS") or info["affinity"] or info["nproc"] or 1)
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
                      f"C oracle fp32 path (oracle/miqmm_oracle.c, gcc -O3 -fopenmp), {threads} threads "
                      f"(host: {info['nproc']} logical CPUs, {info['affinity']} in this process's affinity, "
                      f"{info['model']}), {el:.1f} s; MLX's CPU backend is not available offline",
            "host": info, "ms_per_step": round(el / steps * 1e3, 3)}


def small_m_and_large_vocab(miqmm, torch):
    """the GEMV routes beyond the decode step: speculative-verify / small-batch
    rows M in {1, 2, 4, 8, 16} on the Llama-3-8B projections (4-bit g64), and
    the Gemma-3-27B-class head K = 5376, N = 262144 at M in {1, 8} with fp16
    scales, 4-bit g32 and 8-bit g64; cold weights, median of 20 replays"""
    res = {}
    for (N, K) in SHAPES_8B:
        for M in (1, 2, 4, 8, 16):
            sec, nb = gemv_line(miqmm, torch, M, N, K)
            res[f"qmv_m{M}_{K}to{N}"] = line(sec, nb)
        torch.cuda.empty_cache()
    for (bits, g) in [(4, 32), (8, 64)]:
        for M in (1, 8):
            sec, nb = gemv_line(miqmm, torch, M, 262144, 5376, g=g, bits=bits, sb_dtype=torch.float16)
            res[f"head_5376to262144_m{M}_{bits}bit_g{g}_f16"] = line(sec, nb)
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
        tg = graph_median(torch, [lambda s=s: miqmm.gather_qmm(x, *s[0], idx, True, g, 4, out=yg) for s in stacks], n)
        td = graph_median(torch, [lambda s=s: miqmm.gather_qmm(h, *s[1], idx, True, g, 4, out=yd) for s in stacks], n)
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
        t = graph_median(torch, [lambda tb=tb: miqmm.quantized_embedding(ids, *tb, g, 4, out=out) for tb in tabs], 64)
        nb = T * (K // 2 + 2 * (K // g) * 2 + K * 2)
        res[f"embedding_T{T}"] = {"us": round(t * 1e6, 2), "bytes": nb, "GB/s": round(nb / t / 1e9, 1)}
    return res


PROFILE_DIR = os.path.join(ROOT, "profiles")


def measured_traffic(kernel):
    """HBM bytes per launch of the roofline kernel from its committed rocprofv3
    summary (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy), or None"""
    path = os.path.join(PROFILE_DIR, f"step_{kernel}_m1.md")
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return int(ln.split(":")[1])
    except OSError:
        pass
    return None


def step_types(miqmm, torch):
    """each launch type of the step on its own (cold, median of 20 replays):
    time per launch, bytes per launch, and time per step (launches x time)"""
    res = {}
    for name, Ns, K, count in STEP_TYPES:
        sec, nb = step_type_line(miqmm, torch, Ns, K)
        r = line(sec, nb)
        r["launches_per_step"] = count
        r["us_per_step"] = round(sec * 1e6 * count, 2)
        # a contiguous group runs as one matrix of all its rows
        r["route"] = miqmm.query_route(1, sum(Ns), K, 64, 4)[0]
        if len(Ns) > 1:
            r["grouped"] = "contiguous, one launch"
        res[name] = r
        torch.cuda.empty_cache()
    return res


def profile_section(miqmm, torch, target):
    """one measured section alone, so a rocprofv3 run of this command holds only
    its kernels: a step launch type, the qmv / qmm headline shapes, config 0,
    a bare streaming read, the decode step, or a plain 512 MiB device copy (the
    FETCH_SIZE / WRITE_SIZE calibration)"""
    types = {n: (Ns, K) for n, Ns, K, _ in STEP_TYPES}
    if target in types:
        Ns, K = types[target]
        sec, nb = step_type_line(miqmm, torch, Ns, K)
        return {"section": target, "shapes": [(N, K) for N in Ns], "replays": REPS,
                **line(sec, nb)}
    gemvs = {"qmv": (1, 14336, 4096), "qmv_down": (1, 4096, 14336), "config0": (1, 4864, 896),
             "qmv_m8": (8, 14336, 4096), "qmv_m8_down": (8, 4096, 14336),
             "qmv_m16": (16, 14336, 4096), "qmv_m16_down": (16, 4096, 14336)}
    if target in gemvs:
        M, N, K = gemvs[target]
        sec, nb = gemv_line(miqmm, torch, M, N, K)
        return {"section": target, "shape": f"M={M} N={N} K={K}", "replays": REPS, **line(sec, nb)}
    if target in ("read33", "read77"):
        sec, nb = read_ceiling(miqmm, torch, 33067008 if target == "read33" else 76881408)
        return {"section": target, "replays": REPS, **line(sec, nb)}
    if target == "qmm":
        return {"section": target, "shape": "M=2048 N=14336 K=4096", **qmm_line(miqmm, torch, 2048, 14336, 4096)}
    if target == "step":
        shapes = step_shapes()
        replicas = [make_replica(miqmm, torch, r, shapes) for r in range(3)]
        for projs in replicas:
            run_step_grouped(miqmm, projs)
        torch.cuda.synchronize()
        graphs = [capture(torch, (lambda p=projs: run_step_grouped(miqmm, p))) for projs in replicas]
        time_graphs(torch, graphs, 3)
        t = time_graphs(torch, graphs, 30)
        return {"section": target, "steps": 30, "us_per_step": round(t / 30 * 1e6, 2)}
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
    ap.add_argument("--profile-target", default=None,
                    choices=["step", "qkv", "o", "gateup", "down", "lm_head", "qmv", "qmv_down", "config0",
                             "qmv_m8", "qmv_m8_down", "qmv_m16", "qmv_m16_down", "qmm", "read33", "read77", "copy"],
                    help="run only this measured section and print its figures (for rocprofv3 summaries)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the quantized-matmul path has no multi-GPU leg "
              "(each GPU would run its shard of the projections with these kernels); run with --gpus 1",
              file=sys.stderr)
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
    del graphs, replicas
    torch.cuda.empty_cache()
    # the same grouped step with every projection in its own allocation
    replicas = [make_replica(miqmm, torch, r, shapes, fused=False) for r in range(args.replicas)]
    for projs in replicas:
        run_step_grouped(miqmm, projs)
    torch.cuda.synchronize()
    graphs = [capture(torch, (lambda p=projs: run_step_grouped(miqmm, p))) for projs in replicas]
    time_graphs(torch, graphs, max(args.warmup, 1))
    t2 = time_graphs(torch, graphs, args.steps)
    separate = {"us_per_step": round(t2 / args.steps * 1e6, 2), "launches": 97,
                "GB/s": round(step_bytes * args.steps / t2 / 1e9, 2), "bytes_per_step": step_bytes}
    del graphs, replicas
    torch.cuda.empty_cache()

    # the step's launch types on their own; the roofline kernel is the one with the most time per step
    types = step_types(miqmm, torch)
    dom = max(types, key=lambda k: types[k]["us_per_step"])
    d = types[dom]
    out = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "accumulate": "fp32",
        "data": "synthetic (seeded on-device generator; random-init 4-bit g64 weights)",
        "config": {"workload": "qwen2.5-0.5b decode step, linear layers only: 24 x {q 896->896, k 896->128, "
                               "v 896->128, o 896->896, gate 896->4864, up 896->4864, down 4864->896} + "
                               "lm_head 896->151936; M=1, 4-bit, group 64, bf16 x/scales/biases/y; "
                               "q/k/v and gate/up as one grouped call each, each layer's q/k/v and gate/up "
                               "weights stored contiguously (fused at load)",
                   "launches_per_step": 97, "bytes_per_step": step_bytes,
                   "weight_replicas": args.replicas, "hip_graph": True},
        "roofline": {"kernel": f"{dom}: the step's launch type with the most time per step "
                               f"({d['launches_per_step']} launches x {d['us']} us = {d['us_per_step']} us of "
                               f"{round(ms_per_step * 1e3, 1)} us; route {d['route']})",
                     "bound": "hbm", "achieved": d["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": d["frac_hbm"], "traffic": measured_traffic(dom),
                     "avg_launch_us": d["us"], "bytes_per_launch": d["bytes"]},
        "step_types": types,
        "step_one_launch_per_projection": single,
        "step_grouped_separate_allocations": separate,
    }
    print(f"# step {ms_per_step * 1e3:.1f} us, {gbs:.1f} GB/s (one launch per projection: "
          f"{single['us_per_step']:.1f} us; grouped, separate allocations: {separate['us_per_step']:.1f} us); "
          f"types {json.dumps(types)}", file=sys.stderr, flush=True)
    torch.cuda.empty_cache()

    if not args.no_headline:
        head = {}
        for name, (N, K) in {"qmv_m1_4096x14336": (14336, 4096), "qmv_m1_14336x4096": (4096, 14336),
                             "config0_qmv_m1_896x4864": (4864, 896)}.items():
            sec, nb = gemv_line(miqmm, torch, 1, N, K)
            head[name] = line(sec, nb)
            head[name]["route"] = miqmm.query_route(1, N, K, 64, 4)[0]
        for name, nbytes in {"bare_read_33MB": 33067008, "bare_read_77MB": 76881408}.items():
            sec, nb = read_ceiling(miqmm, torch, nbytes)
            head[name] = line(sec, nb)
        print(f"# qmv / read: {json.dumps(head)}", file=sys.stderr, flush=True)
        for M in (2048, 512):
            for (N, K) in [(14336, 4096), (4096, 14336), (6144, 4096), (4096, 4096)]:
                head[f"qmm_m{M}_{K}to{N}"] = qmm_line(miqmm, torch, M, N, K, check=(M == 2048))
                print(f"# qmm M={M} {K}->{N}: {json.dumps(head[f'qmm_m{M}_{K}to{N}'])}", file=sys.stderr,
                      flush=True)
            torch.cuda.empty_cache()
        head["qmm_m512_896to151936_lm_head"] = qmm_line(miqmm, torch, 512, 151936, 896)
        head["dense_bf16_gemm_m2048_4096to14336_torch"] = {"TFLOP/s": dense_bf16_tflops(torch, 2048, 14336, 4096)}
        head["dense_bf16_gemm_m512_4096to14336_torch"] = {"TFLOP/s": dense_bf16_tflops(torch, 512, 14336, 4096)}
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
