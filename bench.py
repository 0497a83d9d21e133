#!/usr/bin/env python3
"""bench.py — SwarmLLM's quantized matmul path on one MI355X (gfx950).

One step = one Llama-3-8B-shaped decode layer's weight products at M = 1
q/o 4096x4096, k/v 1024x4096 and gate/up
14336x4096 in Q4_K, down 4096x14336 in Q6_K, each activation quantized once
and shared where the reference shares it (q/k/v, gate/up: QMatMul::
forward_shared, vendor/candle/candle-core/src/quantized/mod.rs:1221-1263).
The launches go through libqmm's C ABI; a step is captured once as a HIP
graph and replayed. Weights are N(0, 0.02) quantized on the device (bit-exact
to the reference's from_float); activations N(0, 1). Several copies of the
layer (>= 1 GiB together) are rotated so the 256 MB last-level cache cannot
serve the weights: every step streams its weights from HBM.

value = algorithmic bytes of the layer (weights + f32 inputs + f32 outputs,
138,149,888 B) per second, whole job, inputs resident in HBM.
roofline = the dominant kernel (the Q4_K matvec of the 14336x4096 gate
projection) timed live on its own stream with HIP events, against 8 TB/s.
cpu_baseline = the CPU restatement of candle's path (oracle/, the reference's
k_quants::matmul with its AVX2 kernels) on this host's cores, on the same
layer's bytes.

Prints ONE JSON line. --gpus N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
Q4K, Q6K = 12, 14
ACT_Q8K = 0
# (name, type, n, k): the C2 layer
LAYER = [("q", Q4K, 4096, 4096), ("k", Q4K, 1024, 4096), ("v", Q4K, 1024, 4096), ("o", Q4K, 4096, 4096),
         ("gate", Q4K, 14336, 4096), ("up", Q4K, 14336, 4096), ("down", Q6K, 4096, 14336)]
# products sharing one quantized activation, in launch order
GROUPS = [("attn_in", 4096, ["q", "k", "v"]), ("attn_out", 4096, ["o"]), ("ffn_in", 4096, ["gate", "up"]),
          ("ffn_mid", 14336, ["down"])]
CONFIG_SEED = 2


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def type_bytes(t: int, n: int, k: int) -> int:
    return n * (k // 256) * (144 if t == Q4K else 210)


def layer_bytes() -> dict:
    w = sum(type_bytes(t, n, k) for _, t, n, k in LAYER)
    xin = sum(4 * k for _, _, _, k in LAYER)
    out = sum(4 * n for _, _, n, _ in LAYER)
    return {"weights": w, "inputs": xin, "outputs": out, "total": w + xin + out}


class Layer:
    """Device buffers of one layer's weights (a LAYER-like spec), quantized on
    the device from N(0, 0.02) with seeds (config, copy, product)."""

    def __init__(self, copy: int, acts: dict, spec=None, config_seed: int = CONFIG_SEED):
        import torch

        from swarmllm_amd import GgmlDType, QTensor, fill_normal

        self.spec = spec or LAYER
        self.w = {}
        for p, (name, t, n, k) in enumerate(self.spec):
            seed = (config_seed << 40) | (copy << 8) | p
            wf = fill_normal(n * k, seed=seed, std=0.02).reshape(n, k)
            self.w[name] = QTensor.quantize(wf, GgmlDType(t))
            del wf
        torch.cuda.synchronize()
        self.acts = acts


def make_acts(spec=None, groups=None, rows: int = 1, config_seed: int = CONFIG_SEED):
    """Per group of products sharing an activation: the f32 rows (N(0,1)) and
    a workspace sized by the plan call; the outputs of every product."""
    import torch

    from swarmllm_amd import fill_normal
    from swarmllm_amd._lib import check, lib

    spec, groups = spec or LAYER, groups or GROUPS
    shape = {name: (t, n, k) for name, t, n, k in spec}
    L = lib()
    acts = {}
    need = ctypes.c_size_t(0)
    for i, (g, k, names) in enumerate(groups):
        x = fill_normal(rows * k, seed=(config_seed << 40) | (0xA0 + i)).reshape(rows, k)
        t = shape[names[0]][0]
        if len(names) == 1:
            check("qmm_forward", L.qmm_forward(t, None, None, k, None, shape[names[0]][1], None, 0,
                                               ctypes.byref(need), k, shape[names[0]][1], rows, 0, 0))
        else:
            cnt = len(names)
            ns = (ctypes.c_int64 * cnt)(*[shape[nm][1] for nm in names])
            nulls = (ctypes.c_void_p * cnt)()
            check("qmm_forward_shared", L.qmm_forward_shared(t, cnt, nulls, ns, nulls, ns, None, k, None, 0,
                                                             ctypes.byref(need), k, rows, 0, 0))
        ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device="cuda")
        acts[g] = (x, ws)
    outs = {name: torch.empty((rows, n), dtype=torch.float32, device="cuda") for name, _, n, _ in spec}
    return acts, outs


def enqueue_step(layer: Layer, outs: dict, stream: int, groups=None, rows: int = 1) -> None:
    """The layer's products: per group of weights sharing an activation one
    qmm_forward_shared (QMatMul::forward_shared), or qmm_forward for one."""
    from swarmllm_amd._lib import check, lib

    L = lib()
    shape = {name: (t, n, k) for name, t, n, k in layer.spec}
    need = ctypes.c_size_t(0)
    for g, k, names in groups or GROUPS:
        x, ws = layer.acts[g]
        t = shape[names[0]][0]
        if len(names) == 1:
            name = names[0]
            _, n, _ = shape[name]
            check("qmm_forward", L.qmm_forward(t, layer.w[name].data_.data_ptr(), x.data_ptr(), k,
                                               outs[name].data_ptr(), n, ws.data_ptr(), ws.numel(),
                                               ctypes.byref(need), k, n, rows, 1, stream))
            continue
        cnt = len(names)
        wp = (ctypes.c_void_p * cnt)(*[layer.w[nm].data_.data_ptr() for nm in names])
        ns = (ctypes.c_int64 * cnt)(*[shape[nm][1] for nm in names])
        dp = (ctypes.c_void_p * cnt)(*[outs[nm].data_ptr() for nm in names])
        check("qmm_forward_shared", L.qmm_forward_shared(t, cnt, wp, ns, dp, ns, x.data_ptr(), k, ws.data_ptr(),
                                                         ws.numel(), ctypes.byref(need), k, rows, 1, stream))


def capture(fn, stream):
    import torch

    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            fn(stream.cuda_stream)
    torch.cuda.synchronize()
    return g


class Replayer:
    """Runs exactly `steps` steps as replays of graphs over the layer copies."""

    def __init__(self, layers, outs, stream):
        self.layers, self.outs, self.stream = layers, outs, stream
        self.graphs = {}

    def graph(self, count: int):
        if count not in self.graphs:
            def fn(s, count=count):
                for c in range(count):
                    enqueue_step(self.layers[c], self.outs, s)
            self.graphs[count] = capture(fn, self.stream)
        return self.graphs[count]

    def prepare(self, steps: int) -> None:
        """Capture every graph run(steps) replays, so that no capture (and
        none of the synchronisation capture does) falls inside a timed
        region."""
        C = len(self.layers)
        full, rem = divmod(steps, C)
        if full:
            self.graph(C)
        if rem:
            self.graph(rem)

    def run(self, steps: int) -> None:
        C = len(self.layers)
        full, rem = divmod(steps, C)
        if (full and C not in self.graphs) or (rem and rem not in self.graphs):
            raise RuntimeError("Replayer.run: call prepare(steps) first (no capture inside a timed run)")
        g = self.graphs[C] if full else None
        for _ in range(full):
            g.replay()
        if rem:
            self.graphs[rem].replay()


def time_gpu(fn, stream) -> float:
    """Milliseconds of fn() on `stream`, between HIP events recorded on it."""
    import torch

    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b)


SETTLE_MS = 40.0


def settle(replay, stream, ms: float = SETTLE_MS) -> None:
    """Untimed replays until about `ms` of GPU time has passed, so the timed
    region that follows sees the GPU at its sustained clock (the first
    ~10 ms of back-to-back launches run measurably slower while the clock
    ramps)."""
    import torch

    spent, n = 0.0, 1
    while spent < ms:
        spent += time_gpu(lambda: [replay() for _ in range(n)], stream)
        n = min(2 * n, 64)


def single_matvec(layers, stream, reps: int) -> dict:
    """The product BASELINE.json's target names: ONE Q4_K 14336x4096 matvec
    at M = 1 (the gate projection alone, qmm_forward: one launch that
    quantizes the activation in LDS), back to back over the layer copies'
    gate weights in one graph, timed with HIP events on the stream it runs
    on. Algorithmic bytes = the weight + the f32 activation + the f32 output."""
    import torch

    from swarmllm_amd._lib import check, lib

    L = lib()
    x, ws = layers[0].acts["ffn_in"]
    n, k = 14336, 4096
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    per_graph = 4 * len(layers)
    need = ctypes.c_size_t(0)

    def fn(st):
        for i in range(per_graph):
            lay = layers[i % len(layers)]
            check("qmm_forward", L.qmm_forward(Q4K, lay.w["gate"].data_.data_ptr(), x.data_ptr(), k, out.data_ptr(),
                                               n, ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, 1, 1, st))

    g = capture(fn, stream)
    kernel = L.qmm_last_kernel().decode()
    settle(g.replay, stream)
    ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
    launches = reps * per_graph
    us = ms * 1e3 / launches
    alg = 14336 * 16 * 144 + 4 * 4096 + 4 * 14336
    gbs = alg / (us * 1e-6) / 1e9
    return {"kernel": f"mv_q4k_stream_kernel, one Q4_K 14336x4096 at M=1 ({kernel})", "us": us, "launches": launches,
            "alg_bytes": alg, "gbs": gbs}


def dominant_kernel(layers, outs, stream, reps: int) -> dict:
    """The step's dominant launch, the gate+up products (two Q4_K 14336x4096
    weights sharing one activation: one streaming launch quantizing the
    activation in LDS), back to back over the copies in one graph: its
    average launch, timed with HIP events on the stream it runs on."""
    from swarmllm_amd._lib import check, lib

    L = lib()
    x, ws = layers[0].acts["ffn_in"]
    n, k = 14336, 4096
    per_graph = 4 * len(layers)
    need = ctypes.c_size_t(0)
    ns = (ctypes.c_int64 * 2)(n, n)
    dp = (ctypes.c_void_p * 2)(outs["gate"].data_ptr(), outs["up"].data_ptr())

    def fn(st):
        for i in range(per_graph):
            lay = layers[i % len(layers)]
            wp = (ctypes.c_void_p * 2)(lay.w["gate"].data_.data_ptr(), lay.w["up"].data_.data_ptr())
            check("qmm_forward_shared", L.qmm_forward_shared(Q4K, 2, wp, ns, dp, ns, x.data_ptr(), k, ws.data_ptr(),
                                                             ws.numel(), ctypes.byref(need), k, 1, 1, st))

    g = capture(fn, stream)
    settle(g.replay, stream)
    ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
    launches = reps * per_graph
    us = ms * 1e3 / launches
    alg = 2 * 14336 * 16 * 144 + 4 * 4096 + 2 * 4 * 14336
    gbs = alg / (us * 1e-6) / 1e9
    return {"kernel": "mv_q4k_stream_kernel<1,1,FUSED,16,PF> (gate+up: two Q4_K 14336x4096, M=1, one launch)",
            "us": us, "launches": launches, "alg_bytes": alg, "gbs": gbs}


def gate_up_glu(layers, stream, reps: int) -> dict:
    """The gate+up+GLU launch (qmm_forward_glu, SiLU): the gate+up products of
    the C2 layer at M = 1 and silu(gate) * up written once, back to back over
    the copies in one graph, timed with HIP events on its stream. Algorithmic
    bytes: the two weights, the f32 activation and the n f32 outputs."""
    import torch

    from swarmllm_amd._lib import check, lib

    L = lib()
    x, ws = layers[0].acts["ffn_in"]
    n, k = 14336, 4096
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    per_graph = 4 * len(layers)
    need = ctypes.c_size_t(0)
    check("qmm_forward_glu", L.qmm_forward_glu(Q4K, 0, None, None, None, k, None, n, None, 0, ctypes.byref(need), k,
                                               n, 1, 0, 0))
    buf = torch.empty(need.value, dtype=torch.uint8, device="cuda")

    def fn(st):
        for i in range(per_graph):
            lay = layers[i % len(layers)]
            check("qmm_forward_glu", L.qmm_forward_glu(Q4K, 0, lay.w["gate"].data_.data_ptr(),
                                                       lay.w["up"].data_.data_ptr(), x.data_ptr(), k, out.data_ptr(),
                                                       n, buf.data_ptr(), buf.numel(), ctypes.byref(need), k, n, 1,
                                                       1, st))

    g = capture(fn, stream)
    kernel = L.qmm_last_kernel().decode()
    settle(g.replay, stream)
    ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
    us = ms * 1e3 / (reps * per_graph)
    alg = 2 * 14336 * 16 * 144 + 4 * 4096 + 4 * 14336
    gbs = alg / (us * 1e-6) / 1e9
    return {"kernel": kernel, "us_per_launch": round(us, 4), "alg_bytes_per_launch": alg, "gbs": round(gbs, 2),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def read_floor(layers, stream, reps: int) -> dict:
    """The bare streaming read the decode launches are held against
    (qmm_read_floor: one launch that reads the bytes once and does nothing
    else), over the gate weight (33 MB, the single product's bytes) and the
    gate and up weights together (66 MB, the gate+up launch's), back to back
    over the layer copies in one graph, timed with HIP events on its stream."""
    import torch

    from swarmllm_amd._lib import check, lib

    L = lib()
    sink = torch.empty(L.qmm_read_floor_sink_bytes(), dtype=torch.uint8, device="cuda")
    per_graph = 4 * len(layers)
    gate_bytes = 14336 * 16 * 144
    res = {"kernel": "read_kernel (qmm_read_floor: 1024 workgroups x 512 threads, 16-byte nontemporal loads)"}
    for name, two in (("bytes_33mb", False), ("bytes_66mb", True)):
        def fn(st, two=two):
            for i in range(per_graph):
                lay = layers[i % len(layers)]
                check("qmm_read_floor", L.qmm_read_floor(lay.w["gate"].data_.data_ptr(), gate_bytes,
                                                         lay.w["up"].data_.data_ptr() if two else None,
                                                         gate_bytes if two else 0, sink.data_ptr(), st))

        g = capture(fn, stream)
        settle(g.replay, stream)
        ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
        us = ms * 1e3 / (reps * per_graph)
        nbytes = gate_bytes * (2 if two else 1)
        res[name] = {"bytes": nbytes, "us_per_launch": round(us, 4), "gbs": round(nbytes / (us * 1e-6) / 1e9, 2)}
    return res


def prefill_inputs(M: int, n: int, k: int):
    """C3's activation (N(0,1), 1% of channels x20) quantized once to Q8_K
    planes, and the output buffer."""
    import torch

    from swarmllm_amd import fill_normal
    from swarmllm_amd._lib import check, lib

    L = lib()
    x = fill_normal(M * k, seed=(3 << 40) | 0xB0).reshape(M, k)
    g = torch.Generator().manual_seed(3)
    ch = torch.randperm(k, generator=g)[: k // 100].to(x.device)
    x[:, ch] *= 20.0
    xq = torch.empty(L.qmm_act_bytes(ACT_Q8K, k, M), dtype=torch.uint8, device="cuda")
    out = torch.empty((M, n), dtype=torch.float32, device="cuda")
    check("qmm_quantize_act", L.qmm_quantize_act(x.data_ptr(), xq.data_ptr(), ACT_Q8K, k, M, k,
                                                 torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return xq, out


def prefill_gemm(layers, stream, reps: int, name: str = "gate") -> dict:
    """One product of BASELINE C3 alone: the Q4_K gate projection 14336x4096
    (C3's headline) or the Q6_K down projection 4096x14336 at M = 512
    (activations N(0,1) with 1% of channels scaled x20), the activation
    quantized once (qmm_quantize_act), then the int8 matrix-core GEMM alone
    (qmm_matmul) back to back over the layer copies' weights in one graph,
    timed with HIP events on its stream. ops = 2*M*N*K per launch."""
    from swarmllm_amd._lib import check, lib

    L = lib()
    t, n, k = {nm: (tt, nn, kk) for nm, tt, nn, kk in LAYER}[name]
    M = 512
    xq, out = prefill_inputs(M, n, k)
    before = L.qmm_gemm_launches()

    def fn(st):
        for lay in layers:
            check("qmm_matmul", L.qmm_matmul(t, lay.w[name].data_.data_ptr(), xq.data_ptr(), out.data_ptr(), n, k,
                                             n, M, st))

    graph = capture(fn, stream)
    if L.qmm_gemm_launches() <= before:
        raise RuntimeError("the prefill product did not run the GEMM")
    kernel = L.qmm_last_kernel().decode()
    settle(graph.replay, stream)
    ms = time_gpu(lambda: [graph.replay() for _ in range(reps)], stream)
    us = ms * 1e3 / (reps * len(layers))
    ops = 2.0 * M * n * k
    tops = ops / (us * 1e-6) / 1e12
    tname = "Q4_K" if t == Q4K else "Q6_K"
    # the same product as the layer runs it: qmm_forward with its planned
    # workspace (quantizer + GEMM, cut along K when its tiles leave CUs idle)
    import torch

    from swarmllm_amd import fill_normal

    x = fill_normal(M * k, seed=(3 << 40) | 0xB1).reshape(M, k)
    need = ctypes.c_size_t(0)
    check("qmm_forward", L.qmm_forward(t, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, M, 0, 0))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device="cuda")

    def fwd(st):
        for lay in layers:
            check("qmm_forward", L.qmm_forward(t, lay.w[name].data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n,
                                               ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, M, 1, st))

    g2 = capture(fwd, stream)
    fkernel = L.qmm_last_kernel().decode()
    settle(g2.replay, stream)
    fus = time_gpu(lambda: [g2.replay() for _ in range(reps)], stream) * 1e3 / (reps * len(layers))
    return {"workload": f"C3: {tname} {name} {n}x{k} at M=512, int8 MFMA GEMM (activation quantized once, Q8_K)",
            "us_per_launch": round(us, 3), "ops_per_launch": int(ops), "tops": round(tops, 2),
            "forward": {"us": round(fus, 3), "tops": round(ops / (fus * 1e-6) / 1e12, 2), "kernel": fkernel,
                        "what": "qmm_forward with its planned workspace: activation quantizer + GEMM (cut along K "
                                "when its tiles leave CUs idle), as the C3 layer runs the product"},
            "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": 5000.0, "unit": "TOP/s",
                         "frac": round(tops / 5000.0, 4), "kernel": kernel,
                         "traffic": measured_traffic("prefill_gemm" if name == "gate" else f"prefill_{name}")}}


def prefill_layer(layers, stream, reps: int) -> dict:
    """BASELINE C3 as a whole layer: the C2 layer's 7 products at M = 512
    (activations N(0,1), 1% of channels x20), launched as a decode step
    launches them (each shared activation quantized once: qmm_forward_shared
    for q/k/v and gate/up, qmm_forward for o and down), over the layer copies
    in one graph, timed with HIP events on its stream.
    ops = 2 * 512 * sum(n * k) = 223.3 G per layer."""
    import types

    import torch

    M = 512
    acts, outs = make_acts(rows=M, config_seed=3)
    g = torch.Generator().manual_seed(3)
    for x, _ in acts.values():
        k = x.shape[1]
        ch = torch.randperm(k, generator=g)[: k // 100].to(x.device)
        x[:, ch] *= 20.0
    views = [types.SimpleNamespace(spec=lay.spec, w=lay.w, acts=acts) for lay in layers]

    def fn(st):
        for v in views:
            enqueue_step(v, outs, st, rows=M)

    graph = capture(fn, stream)
    settle(graph.replay, stream)
    ms = time_gpu(lambda: [graph.replay() for _ in range(reps)], stream)
    us = ms * 1e3 / (reps * len(layers))
    ops = 2.0 * M * sum(n * k for _, _, n, k in LAYER)
    tops = ops / (us * 1e-6) / 1e12
    return {"workload": "C3: the Llama-3-8B layer's 7 products at M=512 (q/k/v/o/gate/up Q4_K, down Q6_K), "
                        "activations quantized once per shared input (Q8_K), int8 MFMA GEMMs",
            "us_per_layer": round(us, 2), "ops_per_layer": int(ops), "tops": round(tops, 2),
            "frac_of_int8_peak": round(tops / 5000.0, 4)}


def cpu_baseline(layers, budget_s: float) -> dict:
    """The oracle (CPU restatement of candle's k_quants::matmul + AVX2 dots) on
    the same layers' bytes, rotating over the copies as the GPU does (so the
    weights come from DRAM, not the host's last-level cache), min over trials
    of one full rotation, on this host's cores."""
    import numpy as np

    from oracle import qref

    usable = len(os.sched_getaffinity(0))
    logical, physical = usable, physical_cores(usable)
    wbs = [{name: np.frombuffer(lay.w[name].data(), np.uint8) for name, _, _, _ in LAYER} for lay in layers]
    xs = {g: layers[0].acts[g][0].cpu().numpy() for g, _, _ in GROUPS}
    shape = {name: (t, n, k) for name, t, n, k in LAYER}
    alg = layer_bytes()["total"]

    def timed(threads: int, seconds: float):
        def rotation():
            for wb in wbs:
                for g, _, names in GROUPS:
                    for name in names:
                        t, n, _ = shape[name]
                        qref.matmul(t, xs[g], wb[name], n, threads=threads)

        rotation()  # warm
        best, t_end, trials = float("inf"), time.perf_counter() + seconds, 0
        while trials < 2 or (time.perf_counter() < t_end and trials < 100):
            t0 = time.perf_counter()
            rotation()
            best = min(best, (time.perf_counter() - t0) / len(wbs))
            trials += 1
        return best, trials

    # the reference shows decode peaking below the full core count
    # (src/inference/cpu_pools.rs:3-25): 1, 4, physical/2 and physical threads
    counts = sorted({c for c in (1, 4, max(1, physical // 2), physical) if c <= usable})
    sweep = {}
    for c in counts:
        if c == physical:
            continue
        best, trials = timed(c, budget_s / 4)
        sweep[str(c)] = {"gbs": round(alg / best / 1e9, 3), "ms_per_layer": round(best * 1e3, 4), "trials": trials}
    best, trials = timed(physical, budget_s)
    sweep[str(physical)] = {"gbs": round(alg / best / 1e9, 3), "ms_per_layer": round(best * 1e3, 4), "trials": trials}
    return {"value": round(alg / best / 1e9, 3), "unit": "GB/s", "cores": physical, "kind": "port",
            "sample": f"C2 decode layer at M=1 (7 products, 138.1 MB of Q4_K/Q6_K weights) rotated over "
                      f"{len(wbs)} copies, oracle/ restatement of candle k_quants::matmul with its AVX2 vec_dot "
                      f"kernels, {physical} threads (one per physical core of the {logical} logical CPUs this "
                      f"process may use), min of {trials} rotations: {best * 1e3:.3f} ms/layer",
            "cpu": cpu_name(), "logical_cpus_usable": logical, "physical_cores_usable": physical,
            "logical_cpus_host": os.cpu_count(), "threads_sweep": sweep}


# BASELINE C5: one peer's shard of a Llama-3.3-70B-shaped model, 40 layers
C5_LAYER = [("q", Q4K, 8192, 8192), ("k", Q4K, 1024, 8192), ("v", Q4K, 1024, 8192), ("o", Q4K, 8192, 8192),
            ("gate", Q4K, 28672, 8192), ("up", Q4K, 28672, 8192), ("down", Q6K, 8192, 28672)]
C5_GROUPS = [("attn_in", 8192, ["q", "k", "v"]), ("attn_out", 8192, ["o"]), ("ffn_in", 8192, ["gate", "up"]),
             ("ffn_mid", 28672, ["down"])]
C5_LAYERS = 40


def c5_shard(stream, rows_list=(1, 8, 16), reps: int = 5) -> dict:
    """BASELINE C5: the 40 layers resident (21.67 GB of Q4_K / Q6_K weights,
    each layer its own N(0,0.02) draw), one forward = every layer's 7
    products (4 launches a layer: q+k+v and gate+up share their activation)
    captured as one HIP graph, at each speculative-verification width M.
    GB/s = the shard's weight bytes per forward time (the weights are read
    once per forward at any M <= 16 on the kernels that take M in one pass)."""
    import torch

    t0 = time.perf_counter()
    layers = [Layer(c, None, spec=C5_LAYER, config_seed=5) for c in range(C5_LAYERS)]
    wbytes = C5_LAYERS * sum(type_bytes(t, n, k) for _, t, n, k in C5_LAYER)
    log(f"C5: {C5_LAYERS} layers ({wbytes / 1e9:.2f} GB) quantized in {time.perf_counter() - t0:.1f} s")
    out = {"workload": "C5: Llama-3.3-70B shard, 40 layers, Q4_K (q/k/v/o/gate/up) + Q6_K (down), "
                       "7 products a layer in 4 launches, one graph per forward",
           "weight_bytes": wbytes, "by_rows": {}}
    for rows in rows_list:
        acts, outs = make_acts(C5_LAYER, C5_GROUPS, rows, config_seed=5)
        for lay in layers:
            lay.acts = acts

        def fn(s, outs=outs, rows=rows):
            for lay in layers:
                enqueue_step(lay, outs, s, C5_GROUPS, rows)

        g = capture(fn, stream)
        settle(g.replay, stream)
        ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream) / reps
        gbs = wbytes / (ms * 1e-3) / 1e9
        out["by_rows"][str(rows)] = {"ms_per_forward": round(ms, 4), "weight_gbs": round(gbs, 1),
                                     "percent_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}
        log(f"C5 M={rows}: {ms:.3f} ms per forward, {gbs:.0f} GB/s")
        del g
    del layers
    torch.cuda.empty_cache()
    return out


MXFP4 = 39


def c4_moe(stream, reps: int = 20, copies: int = 2, profile_reps: int = 0) -> dict:
    """BASELINE C4: gpt-oss-20b-shaped experts, 32 MXFP4 experts with gate_up
    [5760, 2880] and down [2880, 2880]; 8 tokens routed top-4 from seeded
    N(0,1) logits (ties to the lower index), entries sorted by (expert,
    pair). One step = the gate_up grouped product (per-token inputs) and the
    down grouped product (per-pair inputs, routing weights), back to back
    over `copies` weight stacks. Algorithmic bytes = the touched experts'
    weights + f32 inputs and outputs. With profile_reps, the step runs that
    many times outside any graph and nothing is timed (rocprofv3 passes)."""
    import numpy as np
    import torch

    from swarmllm_amd import GgmlDType, QTensor, fill_normal
    from swarmllm_amd._lib import check, lib

    L = lib()
    E, tokens, topk, hidden, inter = 32, 8, 4, 2880, 2880
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((tokens, E)).astype(np.float32)
    choice = np.argsort(-logits, axis=1, kind="stable")[:, :topk]
    pairs = sorted((int(choice[t, j]), t * topk + j) for t in range(tokens) for j in range(topk))
    eids = torch.tensor([e for e, _ in pairs], dtype=torch.int32, device="cuda")
    sids = torch.tensor([p for _, p in pairs], dtype=torch.int32, device="cuda")
    sel = np.take_along_axis(logits, choice, axis=1).astype(np.float64)
    wts = np.exp(sel - sel.max(axis=1, keepdims=True))
    wts /= wts.sum(axis=1, keepdims=True)
    topk_w = torch.tensor(wts.reshape(-1), dtype=torch.float32, device="cuda")
    touched = len(set(e for e, _ in pairs))

    def stack(n, k, seed):
        parts = [QTensor.quantize(fill_normal(n * k, seed=(seed << 8) | i, std=0.02).reshape(n, k), GgmlDType(MXFP4))
                 for i in range(E)]
        return torch.cat([p.data_ for p in parts])

    gu = [stack(2 * inter, hidden, 40 + 2 * c) for c in range(copies)]
    dn = [stack(hidden, inter, 41 + 2 * c) for c in range(copies)]
    x1 = fill_normal(tokens * hidden, seed=(4 << 40) | 1).reshape(tokens, hidden)
    x2 = fill_normal(tokens * topk * inter, seed=(4 << 40) | 2).reshape(tokens * topk, inter)
    y1 = torch.empty((tokens * topk, 2 * inter), dtype=torch.float32, device="cuda")
    y2 = torch.empty((tokens * topk, hidden), dtype=torch.float32, device="cuda")
    need = ctypes.c_size_t(0)
    size_m = tokens * topk
    check("qmm_moe_forward", L.qmm_moe_forward(MXFP4, None, E, None, hidden, None, None, None, topk, None, 2 * inter,
                                               None, 0, ctypes.byref(need), hidden, 2 * inter, size_m, 0, 0))
    ws1 = torch.empty(need.value, dtype=torch.uint8, device="cuda")
    check("qmm_moe_forward", L.qmm_moe_forward(MXFP4, None, E, None, inter, None, None, ctypes.c_void_p(16), topk,
                                               None, hidden, None, 0, ctypes.byref(need), inter, hidden, size_m, 0, 0))
    ws2 = torch.empty(need.value, dtype=torch.uint8, device="cuda")
    before = L.qmm_moe_launches()

    def fn(s):
        for c in range(copies):
            check("qmm_moe_forward", L.qmm_moe_forward(
                MXFP4, gu[c].data_ptr(), E, x1.data_ptr(), hidden, sids.data_ptr(), eids.data_ptr(), None, topk,
                y1.data_ptr(), 2 * inter, ws1.data_ptr(), ws1.numel(), ctypes.byref(need), hidden, 2 * inter, size_m,
                1, s))
            check("qmm_moe_forward", L.qmm_moe_forward(
                MXFP4, dn[c].data_ptr(), E, x2.data_ptr(), inter, sids.data_ptr(), eids.data_ptr(),
                topk_w.data_ptr(), topk, y2.data_ptr(), hidden, ws2.data_ptr(), ws2.numel(), ctypes.byref(need),
                inter, hidden, size_m, 1, s))

    if profile_reps:
        for _ in range(profile_reps):
            fn(stream.cuda_stream)
        torch.cuda.synchronize()
        log(f"profile c4: {profile_reps} MoE steps over {copies} weight stacks ({touched} experts touched)")
        return {}
    g = capture(fn, stream)
    if L.qmm_moe_launches() < before + 2 * copies:
        raise RuntimeError("the C4 step did not run the grouped expert kernels")
    settle(g.replay, stream)
    ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
    us = ms * 1e3 / (reps * copies)
    per_expert = 2 * inter * (hidden // 32) * 17 + hidden * (inter // 32) * 17
    alg = touched * per_expert + 4 * (tokens * hidden + size_m * inter + size_m * 2 * inter + size_m * hidden)
    gbs = alg / (us * 1e-6) / 1e9
    log(f"C4: {us:.2f} us per MoE step ({touched} experts touched), {gbs:.0f} GB/s")
    return {"workload": "C4: gpt-oss-20b MoE, 32 MXFP4 experts, 8 tokens top-4, gate_up + down grouped products",
            "experts_touched": touched, "us_per_step": round(us, 3), "alg_bytes": alg, "gbs": round(gbs, 1),
            "percent_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}


def moe_kquant(stream, reps: int = 10, copies: int = 2) -> dict:
    """Grouped K-quant experts: 128 experts of a 2048-wide MoE layer (expert
    width 768), gate_up [1536, 2048] in Q4_K and down [2048, 768] in Q6_K,
    routed top-8 from seeded N(0,1) logits (entries sorted by expert, pair);
    one step = the gate_up product (per-token inputs) and the down product
    (per-pair inputs, routing weights), at a decode step (1 token) and at a
    512-token prompt, over `copies` weight stacks. Decode reports the
    touched experts' bytes per step; the prompt its int8 ops per step."""
    import numpy as np
    import torch

    from swarmllm_amd import GgmlDType, QTensor, fill_normal
    from swarmllm_amd._lib import check, lib

    L = lib()
    E, topk, hidden, inter = 128, 8, 2048, 768

    def stack(t, n, k, seed):
        parts = [QTensor.quantize(fill_normal(n * k, seed=(seed << 8) | i, std=0.02).reshape(n, k), GgmlDType(t))
                 for i in range(E)]
        return torch.cat([p.data_ for p in parts])

    gu = [stack(Q4K, 2 * inter, hidden, 60 + 2 * c) for c in range(copies)]
    dn = [stack(Q6K, hidden, inter, 61 + 2 * c) for c in range(copies)]
    out = {}
    for tokens in (1, 512):
        rng = np.random.default_rng(6 + tokens)
        logits = rng.standard_normal((tokens, E)).astype(np.float32)
        choice = np.argsort(-logits, axis=1, kind="stable")[:, :topk]
        pairs = sorted((int(choice[t, j]), t * topk + j) for t in range(tokens) for j in range(topk))
        eids = torch.tensor([e for e, _ in pairs], dtype=torch.int32, device="cuda")
        sids = torch.tensor([p for _, p in pairs], dtype=torch.int32, device="cuda")
        sel = np.take_along_axis(logits, choice, axis=1).astype(np.float64)
        wts = np.exp(sel - sel.max(axis=1, keepdims=True))
        wts /= wts.sum(axis=1, keepdims=True)
        topk_w = torch.tensor(wts.reshape(-1), dtype=torch.float32, device="cuda")
        touched = len(set(e for e, _ in pairs))
        size_m = tokens * topk
        x1 = fill_normal(tokens * hidden, seed=(6 << 40) | tokens).reshape(tokens, hidden)
        x2 = fill_normal(size_m * inter, seed=(7 << 40) | tokens).reshape(size_m, inter)
        y1 = torch.empty((size_m, 2 * inter), dtype=torch.float32, device="cuda")
        y2 = torch.empty((size_m, hidden), dtype=torch.float32, device="cuda")
        need = ctypes.c_size_t(0)
        check("qmm_moe_forward", L.qmm_moe_forward(Q4K, None, E, None, hidden, None, None, None, topk, None,
                                                   2 * inter, None, 0, ctypes.byref(need), hidden, 2 * inter, size_m,
                                                   0, 0))
        ws1 = torch.empty(need.value, dtype=torch.uint8, device="cuda")
        check("qmm_moe_forward", L.qmm_moe_forward(Q6K, None, E, None, inter, None, None, ctypes.c_void_p(16), topk,
                                                   None, hidden, None, 0, ctypes.byref(need), inter, hidden, size_m,
                                                   0, 0))
        ws2 = torch.empty(need.value, dtype=torch.uint8, device="cuda")
        before = L.qmm_moe_launches()

        def fn(s):
            for c in range(copies):
                check("qmm_moe_forward", L.qmm_moe_forward(
                    Q4K, gu[c].data_ptr(), E, x1.data_ptr(), hidden, sids.data_ptr(), eids.data_ptr(), None, topk,
                    y1.data_ptr(), 2 * inter, ws1.data_ptr(), ws1.numel(), ctypes.byref(need), hidden, 2 * inter,
                    size_m, 1, s))
                check("qmm_moe_forward", L.qmm_moe_forward(
                    Q6K, dn[c].data_ptr(), E, x2.data_ptr(), inter, sids.data_ptr(), eids.data_ptr(),
                    topk_w.data_ptr(), topk, y2.data_ptr(), hidden, ws2.data_ptr(), ws2.numel(), ctypes.byref(need),
                    inter, hidden, size_m, 1, s))

        g = capture(fn, stream)
        if L.qmm_moe_launches() < before + 2 * copies:
            raise RuntimeError("the K-quant MoE step did not run the grouped kernels")
        settle(g.replay, stream)
        ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
        us = ms * 1e3 / (reps * copies)
        per_expert = 2 * inter * (hidden // 256) * 144 + hidden * (inter // 256) * 210
        alg = touched * per_expert + 4 * (tokens * hidden + size_m * inter + size_m * 2 * inter + size_m * hidden)
        ops = 2.0 * size_m * (2 * inter * hidden + hidden * inter)
        key = "decode" if tokens == 1 else "prompt"
        out[key] = {"tokens": tokens, "entries": size_m, "experts_touched": touched, "us_per_step": round(us, 3),
                    "alg_bytes": alg, "gbs": round(alg / (us * 1e-6) / 1e9, 1),
                    "tops": round(ops / (us * 1e-6) / 1e12, 2)}
        log(f"K-quant MoE, {tokens} token(s): {us:.2f} us per step ({touched} experts touched), "
            f"{out[key]['gbs']:.0f} GB/s, {out[key]['tops']:.1f} TOP/s")
        if tokens > 8:
            out["prompt_mfma"] = moe_prompt_step(stream, Q4K, Q6K, gu, dn, E, hidden, inter, topk, tokens, sids, eids,
                                                 topk_w, x1, x2, touched, reps)
    out["workload"] = ("grouped K-quant experts: 128 experts, hidden 2048, expert width 768, gate_up Q4_K "
                       "[1536, 2048] + down Q6_K [2048, 768], top-8, at 1 token and 512 tokens (prompt: the "
                       "one-row-per-pair kernels, and prompt_mfma: the f16 matrix-core kernels of "
                       "qmm_moe_forward_prefill)")
    return out


def moe_prompt_step(stream, qg, qd, gu, dn, E, hidden, inter, topk, tokens, sids, eids, topk_w, x1, x2, touched,
                    reps) -> dict:
    """One MoE step of a prompt through qmm_moe_forward_prefill (the
    reference's moe_gemm_gguf_prefill): the gate_up product (per-token f32
    inputs, rounded to f16 in the launch's prologue) and the down product
    (per-pair inputs, routing weights), over the weight stacks gu / dn in
    turn. Reports us per step, the touched experts' weight bytes per second
    and f16 matrix-core TFLOP/s (2 * entries * n * k per product)."""
    import torch

    from swarmllm_amd._lib import X_F32, check, lib

    L = lib()
    size_m = tokens * topk
    y1 = torch.empty((size_m, 2 * inter), dtype=torch.float32, device="cuda")
    y2 = torch.empty((size_m, hidden), dtype=torch.float32, device="cuda")
    need = ctypes.c_size_t(0)
    check("qmm_moe_forward_prefill", L.qmm_moe_forward_prefill(
        qg, None, E, None, X_F32, hidden, None, None, None, topk, None, 2 * inter, None, 0, ctypes.byref(need), hidden,
        2 * inter, size_m, 0, 0))
    ws1 = torch.empty(need.value, dtype=torch.uint8, device="cuda")
    check("qmm_moe_forward_prefill", L.qmm_moe_forward_prefill(
        qd, None, E, None, X_F32, inter, None, None, ctypes.c_void_p(16), topk, None, hidden, None, 0,
        ctypes.byref(need), inter, hidden, size_m, 0, 0))
    ws2 = torch.empty(need.value, dtype=torch.uint8, device="cuda")
    before = L.qmm_moe_prefill_launches()

    def fn(s):
        for c in range(len(gu)):
            check("qmm_moe_forward_prefill", L.qmm_moe_forward_prefill(
                qg, gu[c].data_ptr(), E, x1.data_ptr(), X_F32, hidden, sids.data_ptr(), eids.data_ptr(), None, topk,
                y1.data_ptr(), 2 * inter, ws1.data_ptr(), ws1.numel(), ctypes.byref(need), hidden, 2 * inter, size_m,
                1, s))
            check("qmm_moe_forward_prefill", L.qmm_moe_forward_prefill(
                qd, dn[c].data_ptr(), E, x2.data_ptr(), X_F32, inter, sids.data_ptr(), eids.data_ptr(),
                topk_w.data_ptr(), topk, y2.data_ptr(), hidden, ws2.data_ptr(), ws2.numel(), ctypes.byref(need), inter,
                hidden, size_m, 1, s))

    g = capture(fn, stream)
    if L.qmm_moe_prefill_launches() < before + 2 * len(gu):
        raise RuntimeError("the prompt MoE step did not run the matrix-core grouped kernels")
    settle(g.replay, stream)
    ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
    us = ms * 1e3 / (reps * len(gu))
    wbytes = touched * (gu[0].numel() + dn[0].numel()) // E
    flops = 2.0 * size_m * (2 * inter * hidden + hidden * inter)
    r = {"tokens": tokens, "entries": size_m, "experts_touched": touched, "us_per_step": round(us, 3),
         "weight_bytes": wbytes, "weight_gbs": round(wbytes / (us * 1e-6) / 1e9, 1),
         "tflops_f16": round(flops / (us * 1e-6) / 1e12, 2)}
    log(f"prompt MoE (matrix cores), {tokens} tokens: {us:.2f} us per step, {r['weight_gbs']:.0f} GB/s of weights, "
        f"{r['tflops_f16']:.1f} TFLOP/s")
    return r


def moe_prompt_gpt_oss(stream, reps: int = 10, copies: int = 2, tokens: int = 512) -> dict:
    """BASELINE C4's experts (gpt-oss-20b: 32 MXFP4 experts, gate_up [5760,
    2880], down [2880, 2880], top-4) at a 512-token prompt through
    qmm_moe_forward_prefill."""
    import numpy as np
    import torch

    from swarmllm_amd import GgmlDType, QTensor, fill_normal

    E, topk, hidden, inter = 32, 4, 2880, 2880
    rng = np.random.default_rng(8)
    logits = rng.standard_normal((tokens, E)).astype(np.float32)
    choice = np.argsort(-logits, axis=1, kind="stable")[:, :topk]
    pairs = sorted((int(choice[t, j]), t * topk + j) for t in range(tokens) for j in range(topk))
    eids = torch.tensor([e for e, _ in pairs], dtype=torch.int32, device="cuda")
    sids = torch.tensor([p for _, p in pairs], dtype=torch.int32, device="cuda")
    sel = np.take_along_axis(logits, choice, axis=1).astype(np.float64)
    wts = np.exp(sel - sel.max(axis=1, keepdims=True))
    wts /= wts.sum(axis=1, keepdims=True)
    topk_w = torch.tensor(wts.reshape(-1), dtype=torch.float32, device="cuda")
    touched = len(set(e for e, _ in pairs))

    def stack(n, k, seed):
        parts = [QTensor.quantize(fill_normal(n * k, seed=(seed << 8) | i, std=0.02).reshape(n, k), GgmlDType(MXFP4))
                 for i in range(E)]
        return torch.cat([p.data_ for p in parts])

    gu = [stack(2 * inter, hidden, 80 + 2 * c) for c in range(copies)]
    dn = [stack(hidden, inter, 81 + 2 * c) for c in range(copies)]
    x1 = fill_normal(tokens * hidden, seed=(8 << 40) | 1).reshape(tokens, hidden)
    x2 = fill_normal(tokens * topk * inter, seed=(8 << 40) | 2).reshape(tokens * topk, inter)
    r = moe_prompt_step(stream, MXFP4, MXFP4, gu, dn, E, hidden, inter, topk, tokens, sids, eids, topk_w, x1, x2,
                        touched, reps)
    r["workload"] = ("gpt-oss-20b experts (BASELINE C4's weights: 32 MXFP4 experts, gate_up [5760, 2880], down "
                     "[2880, 2880], top-4) at a 512-token prompt, qmm_moe_forward_prefill")
    return r


def c1_q8_0(stream, reps: int = 50, copies: int = 16) -> dict:
    """BASELINE C1 (the reference's CPU-runnable case) on the device: Q8_0
    4096 x 4096 (N(0,0.02), seed 0) against one N(0,1) row, rotated over
    `copies` weights."""
    import torch

    from swarmllm_amd import GgmlDType, QTensor, fill_normal
    from swarmllm_amd._lib import check, lib

    L = lib()
    n = k = 4096
    ws = [QTensor.quantize(fill_normal(n * k, seed=c, std=0.02).reshape(n, k), GgmlDType(8)) for c in range(copies)]
    x = fill_normal(k, seed=1 << 32).reshape(1, k)
    y = torch.empty((1, n), dtype=torch.float32, device="cuda")
    need = ctypes.c_size_t(0)
    check("qmm_forward", L.qmm_forward(8, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, 1, 0, 0))
    buf = torch.empty(need.value, dtype=torch.uint8, device="cuda")

    def fn(s):
        for w in ws:
            check("qmm_forward", L.qmm_forward(8, w.data_.data_ptr(), x.data_ptr(), k, y.data_ptr(), n,
                                               buf.data_ptr(), buf.numel(), ctypes.byref(need), k, n, 1, 1, s))

    g = capture(fn, stream)
    settle(g.replay, stream)
    ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
    us = ms * 1e3 / (reps * copies)
    alg = n * (k // 32) * 34 + 4 * k + 4 * n
    gbs = alg / (us * 1e-6) / 1e9
    log(f"C1: {us:.2f} us per Q8_0 product (one launch, activation quantized in it), {gbs:.0f} GB/s")
    return {"workload": "C1: Q8_0 4096x4096 at M=1 (qmm_forward: one launch, the activation quantized in it)",
            "us_per_product": round(us, 3), "alg_bytes": alg, "gbs": round(gbs, 1),
            "percent_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}


def prefill_b32(stream, reps: int = 10, copies: int = 4) -> dict:
    """The 32-value block GEMM (Q8_0 and MXFP4, 4096 x 4096 at M = 512,
    activation quantized once to Q8_0 planes, then qmm_matmul alone), rotated
    over `copies` weights in one graph: no BASELINE config runs these types
    at prompt size; the line shows their matrix-core path's rate."""
    import torch

    from swarmllm_amd import GgmlDType, QTensor, fill_normal
    from swarmllm_amd._lib import check, lib

    L = lib()
    M, n, k = 512, 4096, 4096
    x = fill_normal(M * k, seed=(1 << 32) | 5).reshape(M, k)
    xq = torch.empty(L.qmm_act_bytes(1, k, M), dtype=torch.uint8, device="cuda")
    check("qmm_quantize_act", L.qmm_quantize_act(x.data_ptr(), xq.data_ptr(), 1, k, M, k,
                                                 torch.cuda.current_stream().cuda_stream))
    out = torch.empty((M, n), dtype=torch.float32, device="cuda")
    res = {}
    for t, name in ((8, "Q8_0"), (39, "MXFP4")):
        ws = [QTensor.quantize(fill_normal(n * k, seed=c, std=0.02).reshape(n, k), GgmlDType(t)) for c in range(copies)]

        def fn(s, ws=ws, t=t):
            for w in ws:
                check("qmm_matmul", L.qmm_matmul(t, w.data_.data_ptr(), xq.data_ptr(), out.data_ptr(), n, k, n, M, s))

        g = capture(fn, stream)
        settle(g.replay, stream)
        ms = time_gpu(lambda: [g.replay() for _ in range(reps)], stream)
        us = ms * 1e3 / (reps * copies)
        tops = 2.0 * M * n * k / (us * 1e-6) / 1e12
        log(f"{name} GEMM 4096x4096 at M=512: {us:.2f} us, {tops:.1f} TOP/s")
        res[name] = {"us_per_launch": round(us, 3), "tops": round(tops, 2)}
    return {"workload": "Q8_0 / MXFP4 4096x4096 at M=512, int8 MFMA GEMM (activation quantized once, Q8_0)", **res}


COPY_BYTES = 512 << 20  # the calibration copy: 512 MiB read + 512 MiB written


def profile_only(which: str, layers, outs, stream, reps: int) -> None:
    """Launch one kind of kernel alone, `reps` times, outside any graph, for
    rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE): the dominant decode
    launch rotating over the layer copies, a prefill GEMM (gate or down), or a plain
    device copy of COPY_BYTES whose counters calibrate the other two."""
    import torch

    from swarmllm_amd._lib import check, lib

    L = lib()
    s = stream.cuda_stream
    if which == "copy":
        src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for _ in range(reps):
                dst.copy_(src)
        torch.cuda.synchronize()
        log(f"profile copy: {reps} copies of {COPY_BYTES} bytes")
        return
    if which in ("read33", "read66"):
        sink = torch.empty(L.qmm_read_floor_sink_bytes(), dtype=torch.uint8, device="cuda")
        gate_bytes = 14336 * 16 * 144
        two = which == "read66"
        for i in range(reps):
            lay = layers[i % len(layers)]
            check("qmm_read_floor", L.qmm_read_floor(lay.w["gate"].data_.data_ptr(), gate_bytes,
                                                     lay.w["up"].data_.data_ptr() if two else None,
                                                     gate_bytes if two else 0, sink.data_ptr(), s))
        torch.cuda.synchronize()
        log(f"profile {which}: {reps} bare reads of {gate_bytes * (2 if two else 1)} bytes over {len(layers)} copies")
        return
    if which == "single":
        x, ws = layers[0].acts["ffn_in"]
        n, k = 14336, 4096
        need = ctypes.c_size_t(0)
        out = torch.empty((1, n), dtype=torch.float32, device="cuda")
        for i in range(reps):
            lay = layers[i % len(layers)]
            check("qmm_forward", L.qmm_forward(Q4K, lay.w["gate"].data_.data_ptr(), x.data_ptr(), k, out.data_ptr(),
                                               n, ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, 1, 1, s))
        torch.cuda.synchronize()
        log(f"profile single: {reps} Q4_K 14336x4096 M=1 launches over {len(layers)} copies")
        return
    if which == "dominant":
        x, ws = layers[0].acts["ffn_in"]
        n, k = 14336, 4096
        need = ctypes.c_size_t(0)
        ns = (ctypes.c_int64 * 2)(n, n)
        dp = (ctypes.c_void_p * 2)(outs["gate"].data_ptr(), outs["up"].data_ptr())
        for i in range(reps):
            lay = layers[i % len(layers)]
            wp = (ctypes.c_void_p * 2)(lay.w["gate"].data_.data_ptr(), lay.w["up"].data_.data_ptr())
            check("qmm_forward_shared", L.qmm_forward_shared(Q4K, 2, wp, ns, dp, ns, x.data_ptr(), k, ws.data_ptr(),
                                                             ws.numel(), ctypes.byref(need), k, 1, 1, s))
        torch.cuda.synchronize()
        log(f"profile dominant: {reps} gate+up launches over {len(layers)} copies")
        return
    name = "down" if which in ("prefill_down", "prefill_down_forward") else "gate"
    t, n, k = {nm: (tt, nn, kk) for nm, tt, nn, kk in LAYER}[name]
    M = 512
    xq, out = prefill_inputs(M, n, k)
    if which in ("prefill_forward", "prefill_down_forward"):
        # the product as the C3 layer runs it: qmm_forward with its planned
        # workspace (quantizer, the GEMM, cut along K where planned, the slot sum)
        from swarmllm_amd import fill_normal

        x = fill_normal(M * k, seed=(3 << 40) | 0xB1).reshape(M, k)
        need = ctypes.c_size_t(0)
        check("qmm_forward", L.qmm_forward(t, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, M, 0, 0))
        ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device="cuda")
        for i in range(reps):
            lay = layers[i % len(layers)]
            check("qmm_forward", L.qmm_forward(t, lay.w[name].data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n,
                                               ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, M, 1, s))
        torch.cuda.synchronize()
        log(f"profile {which}: {reps} qmm_forward products over {len(layers)} copies")
        return
    for i in range(reps):
        lay = layers[i % len(layers)]
        check("qmm_matmul", L.qmm_matmul(t, lay.w[name].data_.data_ptr(), xq.data_ptr(), out.data_ptr(), n, k,
                                         n, M, s))
    torch.cuda.synchronize()
    log(f"profile {which}: {reps} GEMM launches over {len(layers)} copies")


def measured_traffic(kernel_key: str):
    """HBM bytes per launch of a kernel from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration), or
    None when the summary is absent. Rows read `traffic <key> <bytes>`."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel_key:
                    return int(parts[2])
    except OSError:
        pass
    return None


def physical_cores(usable: int) -> int:
    """Physical cores among the CPUs this process may run on: distinct
    (package, core) pairs of /proc/cpuinfo over the affinity set, or the
    usable count when the file does not say."""
    try:
        allowed = os.sched_getaffinity(0)
        cores, cur = set(), {}
        with open("/proc/cpuinfo") as f:
            for line in list(f) + [""]:
                if not line.strip():
                    if cur.get("processor") is not None and int(cur["processor"]) in allowed and "core id" in cur:
                        cores.add((cur.get("physical id", "0"), cur["core id"]))
                    cur = {}
                    continue
                key, _, val = line.partition(":")
                cur[key.strip()] = val.strip()
        return max(1, min(len(cores), usable)) if cores else usable
    except (OSError, ValueError):
        return usable


def cpu_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=8, help="layer copies rotated (8 x 138 MB)")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extra", action="store_true", help="skip the C1 / C4 / C5 sections")
    ap.add_argument("--profile", choices=["single", "dominant", "read33", "read66", "prefill", "prefill_forward",
                                          "prefill_down", "prefill_down_forward", "copy", "c4"],
                    help="launch only this kernel --steps times (for rocprofv3 counter passes), print no JSON")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs its path on ONE GPU; --gpus {args.gpus} (WORLD_SIZE {world}) is not "
              "supported. The path shards by weight rows with no exchange (see the sharding design); run with "
              "--gpus 1.", file=sys.stderr)
        return 2

    import torch

    from swarmllm_amd._lib import lib

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    L = lib()
    if L.qmm_available() != 1:
        print("bench.py: libqmm kernels do not run on this device (gfx950 required)", file=sys.stderr)
        return 1
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} ({getattr(props, 'gcnArchName', '?')}), {props.multi_processor_count} CUs")
    # every timed product is captured into a graph before it first runs, so
    # the types are prepared first, as a runtime that captures before any
    # eager product does (qmm_prepare; the reference's
    # mmq_prepare_few_rows_once): else captured products of up to 8 rows
    # stay on the decode kernels
    for t in (8, 12, 14, 20, 39):
        if L.qmm_prepare(t) != 0:
            print(f"bench.py: qmm_prepare({t}) failed", file=sys.stderr)
            return 1

    stream = torch.cuda.Stream()  # default priority
    acts, outs = make_acts()
    t0 = time.perf_counter()
    layers = [Layer(c, acts) for c in range(args.copies)]
    lb = layer_bytes()
    log(f"{args.copies} layer copies quantized on the device in {time.perf_counter() - t0:.1f} s "
        f"({args.copies * lb['weights'] / 2**30:.2f} GiB of weights)")

    if args.profile == "c4":
        c4_moe(stream, profile_reps=args.steps)
        return 0
    if args.profile:
        profile_only(args.profile, layers, outs, stream, args.steps)
        return 0

    rep = Replayer(layers, outs, stream)
    rep.prepare(args.warmup)
    rep.prepare(args.steps)
    rep.prepare(len(layers))
    # the GPU's clock settles first (untimed replays of whole rotations),
    # then the W warmup steps, then exactly K timed steps
    settle(lambda: rep.run(len(layers)), stream)
    with torch.cuda.stream(stream):
        rep.run(args.warmup)
    torch.cuda.synchronize()
    log(f"clock settled ({SETTLE_MS:.0f} ms of untimed replays), warmup {args.warmup} steps done "
        f"(graphs for {sorted(rep.graphs)} steps captured before timing)")

    wall0 = time.perf_counter()
    ms = time_gpu(lambda: rep.run(args.steps), stream)
    wall = time.perf_counter() - wall0
    ms_per_step = ms / args.steps
    value = lb["total"] / (ms_per_step * 1e-3) / 1e9
    log(f"timed {args.steps} steps: {ms_per_step * 1e3:.2f} us/step "
        f"(host wall clock around the timed region {wall * 1e6 / args.steps:.2f} us/step)")

    dk = single_matvec(layers, stream, args.kernel_reps)
    log(f"roofline kernel (one Q4_K 14336x4096 matvec): {dk['us']:.3f} us/launch, {dk['gbs']:.1f} GB/s")
    gu = dominant_kernel(layers, outs, stream, args.kernel_reps)
    log(f"gate+up launch: {gu['us']:.3f} us/launch, {gu['gbs']:.1f} GB/s")
    gl = gate_up_glu(layers, stream, args.kernel_reps)
    log(f"gate+up+GLU launch: {gl['us_per_launch']:.3f} us/launch, {gl['gbs']:.1f} GB/s")
    rf = read_floor(layers, stream, args.kernel_reps)
    log(f"bare read floor: 33 MB {rf['bytes_33mb']['us_per_launch']:.3f} us, "
        f"66 MB {rf['bytes_66mb']['us_per_launch']:.3f} us a launch")

    pre = prefill_gemm(layers, stream, max(2, args.kernel_reps // 5))
    log(f"prefill GEMM (gate): {pre['us_per_launch']:.2f} us/launch, {pre['tops']:.1f} TOP/s; "
        f"through qmm_forward {pre['forward']['us']:.2f} us")
    pre_down = prefill_gemm(layers, stream, max(2, args.kernel_reps // 5), name="down")
    log(f"prefill GEMM (down): {pre_down['us_per_launch']:.2f} us/launch, {pre_down['tops']:.1f} TOP/s; "
        f"through qmm_forward {pre_down['forward']['us']:.2f} us")
    pre_layer = prefill_layer(layers, stream, max(2, args.kernel_reps // 10))
    log(f"prefill layer: {pre_layer['us_per_layer']:.2f} us/layer, {pre_layer['tops']:.1f} TOP/s")

    extra = {}
    if not args.no_extra:
        extra["c1"] = c1_q8_0(stream)
        extra["c4"] = c4_moe(stream)
        extra["moe_kquant"] = moe_kquant(stream)
        extra["moe_prompt_gpt_oss"] = moe_prompt_gpt_oss(stream)
        extra["c5"] = c5_shard(stream)
        extra["prefill_b32"] = prefill_b32(stream)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(layers, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['cpu']})")

    line = {
        "metric": "Q4_K matvec HBM GB/s (% of 8 TB/s) at M=1; prefill int8 MFMA TOPS at M=512",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: weights N(0,0.02) quantized on device (bit-exact from_float), activations N(0,1)",
        "config": {"workload": "C2: Llama-3-8B decode layer, 7 products at M=1 (q/k/v/o/gate/up Q4_K, down Q6_K)",
                   "rows": 1, "layer_bytes": lb["total"], "weight_copies": args.copies,
                   "percent_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(dk["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dk["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic("gate"),
                     "kernel": dk["kernel"], "us_per_launch": round(dk["us"], 4),
                     "alg_bytes_per_launch": dk["alg_bytes"]},
        "gate_up": {"kernel": gu["kernel"], "us_per_launch": round(gu["us"], 4), "alg_bytes_per_launch": gu["alg_bytes"],
                    "gbs": round(gu["gbs"], 2), "frac": round(gu["gbs"] / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic("gate_up")},
        "gate_up_glu": gl,
        "read_floor": rf,
        "cpu_baseline": cpu,
        "prefill": pre,
        "prefill_down": pre_down,
        "prefill_layer": pre_layer,
        **extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
