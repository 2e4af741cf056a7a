#!/usr/bin/env python3
"""bench.py — flashrt's MoE-layer hot path on one MI355X.

Headline: a 48-layer stack of the Q2_0 512-expert top-10 MoE layer
(hidden 2048, expert ff 512, shared expert ff 512), all experts resident in HBM, decode at bs=1.
A step is one token through the 48 layers (x_{l+1} = x_l + moe_l(rms_norm(x_l)), the pre-MoE
RMS norm without weight keeping the chained residual stream bounded); each step's input is a
fresh N(0,1) vector; router logits carry a per-layer Zipf(s=1.1) prior over a random permutation of
the experts. The 48 layers of one step are captured once as a HIP graph and replayed per step.

Also measured in the same run:
  - per-kernel durations (hipEvents on the launch stream, eager run) and the roofline of the
    dominant kernel: algorithmic expert bytes per launch / its average duration vs 8 TB/s;
  - one layer, 2048-token prefill (bf16 inputs, Zipf(1.2) prior): tokens/s and the
    grouped GEMM kernels' MFMA utilisation against the 2.5 PFLOP/s dense fp16 peak;
  - cpu_baseline: the reference's own CPU MoE (moe_cpu over its CpuPool, AVX-512 VNNI; built from
    its sources into oracle/_ref) on a bounded sample of the same workload on this host.

Prints ONE JSON line. `--gpus N` with N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-stack tokens/s (decode bs1, prefill 2K); achieved HBM TB/s & MFMA % of peak"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
N, FF, E, K, LAYERS = 2048, 512, 512, 10, 48
ZIPF_STACK, ZIPF_PREFILL, PREFILL_ALPHA = 1.1, 1.2, 0.4
SPIN_CYCLES = 100_000_000   # torch.cuda._sleep ahead of an eager timing pass (tens of ms)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_times(F, fn):
    """Runs fn() with the library's per-kernel hipEvent timing on; returns {kernel: (ms, launches)}."""
    import ctypes as C
    L = F.lib()
    L.frt_timing_begin()
    fn()
    names = C.create_string_buffer(64 * 32)
    ms = (C.c_double * 32)()
    cnt = (C.c_int * 32)()
    n = L.frt_timing_end(names, 32, ms, cnt, 32)
    out = {}
    for i in range(n):
        nm = names.raw[i * 32:(i + 1) * 32].split(b"\0")[0].decode()
        out[nm] = (float(ms[i]), int(cnt[i]))
    return out


# ---------------------------------------------------------------- config 2: decode stack

def build_stack(F, torch, layers):
    eb = F.expert_bytes(N, FF)
    arena = F.arena_alloc(layers, E, eb)
    g = F.gen
    for l in range(layers):
        g.experts(arena.blob(l, 0), arena.stride, 2, l, 0, E, N, FF)
    shared = torch.empty((layers, arena.stride), dtype=torch.uint8, device="cuda")
    router = torch.empty((layers, E, N), dtype=torch.float32, device="cuda")
    gate = torch.empty((layers, N), dtype=torch.float32, device="cuda")
    bias = torch.empty((layers, E), dtype=torch.float32, device="cuda")
    for l in range(layers):
        g.experts(shared[l], arena.stride, 2, l, 0, 1, N, FF, tensor_base=g.SHARED_TENSOR)
        g.normal(router[l], 2, l, g.ROUTER_TENSOR, 0.02)
        g.normal(gate[l], 2, l, g.GATE_TENSOR, 0.02)
        bias[l] = torch.from_numpy(g.zipf_bias(2, l, E, ZIPF_STACK))
    mls = [F.MoeLayer(arena.blob(l, 0), arena.stride, E, shared[l].data_ptr(), router[l], gate[l], N, FF, K,
                      router_bias=bias[l], norm_input=True) for l in range(layers)]
    if not os.environ.get("FRT_NO_ROUTER_WARM"):
        for l in range(layers):   # the call after layer l reads layer l + 1's router (layer 0's after the last)
            mls[l].set_next_router(router[(l + 1) % layers])
    torch.cuda.synchronize()
    return arena, shared, router, gate, bias, mls


def run_stack(args, F, torch):
    layers = args.layers
    arena, shared, router, gate, bias, mls = build_stack(F, torch, layers)
    total_steps = args.warmup + args.steps
    xs = torch.empty((total_steps, N), dtype=torch.float32, device="cuda")
    F.gen.normal(xs, 2, 0, F.gen.X_TENSOR, 1.0)
    ws = torch.empty(mls[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")
    xin = torch.empty((1, N), dtype=torch.float32, device="cuda")
    buf = [torch.empty((1, N), dtype=torch.float32, device="cuda") for _ in range(2)]
    ids = torch.empty((layers, K), dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()

    stack = F.MoeStack(mls) if args.decode_path == "stack" else None
    if stack is not None:
        ws = torch.empty(stack.workspace_bytes(), dtype=torch.uint8, device="cuda")

    def step_body():
        if stack is not None:   # x_{l+1} = x_l + moe_l(x_l) for the 48 layers in one call
            stack.forward(xin, buf[1], ids=ids, ws=ws)
            return
        cur = xin
        for l, ml in enumerate(mls):
            nxt = buf[l % 2]
            ml.forward(cur, nxt, T=1, resid=cur, ids=ids[l], ws=ws)
            cur = nxt

    with torch.cuda.stream(stream):
        xin.copy_(xs[0:1])
        step_body()                      # eager once (sets up everything outside capture)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step_body()
    with torch.cuda.stream(stream):
        for s in range(args.warmup):
            xin.copy_(xs[s:s + 1])
            graph.replay()
    stream.synchronize()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for s in range(args.warmup, total_steps):
            xin.copy_(xs[s:s + 1])
            graph.replay()
        e1.record(stream)
    stream.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    ms_per_step = gpu_ms / args.steps
    log(f"stack: {args.steps} steps x {layers} layers: {gpu_ms:.2f} ms on the stream ({wall * 1e3:.2f} ms wall), "
        f"{ms_per_step * 1e3:.1f} us/token")
    # the launch as the timed loop runs it: events right around each graph replay, in a pass of its own
    # after the input copy (the interval also holds the graph launch's start-up, which rocprof's
    # kernel time leaves out)
    n_ev = min(64, args.steps)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_ev)]
    with torch.cuda.stream(stream):
        for s, (a, b) in enumerate(evs):
            xin.copy_(xs[s:s + 1])
            a.record(stream)
            graph.replay()
            b.record(stream)
    stream.synchronize()
    replay_us = float(np.mean([a.elapsed_time(b) for a, b in evs])) * 1e3

    # per-kernel durations: eager launches on the same stream, queued behind a spin kernel so that
    # the host has enqueued them all before the GPU reaches them (the event deltas then measure the
    # GPU, not the host's launch rate)
    def eager(n_steps):
        with torch.cuda.stream(stream):
            torch.cuda._sleep(SPIN_CYCLES)
            for s in range(n_steps):
                xin.copy_(xs[s:s + 1])
                step_body()
    eager(1)
    stream.synchronize()
    kt = kernel_times(F, lambda: eager(args.timing_steps))
    del graph
    sync_err = F.layer_sync_error(ws)   # a persistent call that ran out of time would void the run
    res = dict(ms_per_step=ms_per_step, wall_s=wall, kernels=kt, sync_error=sync_err, replay_us=replay_us)
    res["_keep"] = (arena, shared, router, gate, bias, mls, xs, ws)
    return res


# ---------------------------------------------------------------- config 3: 2K prefill

def build_layer(F, torch, cfg, bias_np=None):
    """One layer of BASELINE configs[cfg]: its own arena (E experts), shared expert, router, gate."""
    eb = F.expert_bytes(N, FF)
    stride = (eb + 4095) // 4096 * 4096
    g = F.gen
    arena = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    g.experts(arena, stride, cfg, 0, 0, E, N, FF)
    shared = torch.empty(eb, dtype=torch.uint8, device="cuda")
    g.experts(shared, eb, cfg, 0, 0, 1, N, FF, tensor_base=g.SHARED_TENSOR)
    router = torch.empty((E, N), dtype=torch.float32, device="cuda")
    g.normal(router, cfg, 0, g.ROUTER_TENSOR, 0.02)
    gate = torch.empty(N, dtype=torch.float32, device="cuda")
    g.normal(gate, cfg, 0, g.GATE_TENSOR, 0.02)
    bias = None if bias_np is None else torch.from_numpy(np.ascontiguousarray(bias_np, np.float32)).cuda()
    ml = F.MoeLayer(arena.data_ptr(), stride, E, shared.data_ptr(), router, gate, N, FF, K, router_bias=bias)
    ml._bench_keep = (arena, shared, router, gate, bias)
    return ml


def time_prefill_layer(F, torch, ml, x, reps):
    """ms per call of a prefill-size layer call (event-timed on its stream after 3 warm calls: the median
    of 5 rounds of reps calls), the per-kernel durations and the grouped GEMMs' MFMA utilisation."""
    from types import SimpleNamespace
    T = x.shape[0]
    out = torch.empty((T, N), dtype=torch.float32, device="cuda")
    ws = ml.workspace(T)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for _ in range(3):
            ml.forward(x, out, T=T, ws=ws)
    stream.synchronize()
    per_round = []   # the median of 5 timed rounds of `reps` calls (box clocks drift within a run)
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for _ in range(reps):
                ml.forward(x, out, T=T, ws=ws)
            e1.record(stream)
        stream.synchronize()
        per_round.append(e0.elapsed_time(e1) / reps)
    ms = float(np.median(per_round))

    def eager():
        with torch.cuda.stream(stream):
            torch.cuda._sleep(SPIN_CYCLES)
            for _ in range(reps):
                ml.forward(x, out, T=T, ws=ws)
    kt = kernel_times(F, eager)
    S = T * K + T
    gu_flops = 2.0 * S * 2 * N * FF
    dn_flops = 2.0 * S * N * FF
    util = {}
    # gate/up runs as two kernels per layer (tiles of 2-4 token columns, then those of one)
    for name, parts, fl in (("pf_gateup", ("pf_gateup", "pf_gateup1"), gu_flops), ("pf_down", ("pf_down", "pf_down1"), dn_flops)):
        if all(p in kt for p in parts):
            avg_ms = sum(kt[p][0] / kt[p][1] for p in parts)
            util[name] = dict(avg_us=avg_ms * 1e3, tflops=fl / (avg_ms * 1e-3) / 1e12,
                              mfma_frac=fl / (avg_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS,
                              kernels=list(parts))
    flops = gu_flops + dn_flops
    return SimpleNamespace(ms=ms, tokens_per_s=T / ms * 1e3, kernels=kt, util=util, flops=flops)


def run_prefill(args, F, torch):
    """one layer, 2048 bf16 tokens, Zipf(1.2) popularity."""
    ml = build_layer(F, torch, 3, F.gen.zipf_bias(3, 0, E, ZIPF_PREFILL, PREFILL_ALPHA))
    x = torch.empty((2048, N), dtype=torch.float32, device="cuda")
    F.gen.normal(x, 3, 0, F.gen.X_TENSOR, 1.0, round_bf16=True)
    r = time_prefill_layer(F, torch, ml, x, args.prefill_reps)
    log(f"prefill 2K: {r.ms:.3f} ms/layer, {r.tokens_per_s:.0f} tok/s, experts {r.flops / 1e9:.1f} GFLOP")
    return r


def run_mixed(args, F, torch):
    """one launch of 8192 bf16 prefill tokens plus 16 uncorrelated fp32 decode tokens;
    +2.8 on the logits of 16 seeded hot experts puts about 90% of the selections on them."""
    hot = np.random.default_rng(4).permutation(E)[:16]
    bias = np.zeros(E, np.float32)
    bias[hot] = 2.8
    ml = build_layer(F, torch, 4, bias)
    x = torch.empty((8192 + 16, N), dtype=torch.float32, device="cuda")
    F.gen.normal(x[:8192], 4, 0, F.gen.X_TENSOR, 1.0, round_bf16=True)
    F.gen.normal(x[8192:], 4, 0, F.gen.X_TENSOR + 1, 1.0)
    r = time_prefill_layer(F, torch, ml, x, max(2, args.prefill_reps // 4))
    log(f"mixed 8192+16: {r.ms:.3f} ms/layer, {r.tokens_per_s:.0f} tok/s")
    return r


def run_windows(args, F, torch, st):
    """configs[0] (T = 1) and configs[1] (T = 3, pairwise cosine 0.8) as single-layer calls, and the
    other verify-window sizes T = 2, 5, 8: configs[0]-shaped layers (no prior, no input norm) over
    the 48 layers of the stack's arena, one call per layer captured as a graph and replayed, so that
    every call streams its experts from HBM as a lone layer call would. Per T: us per call and the
    HBM rate on the bytes the call must read (its distinct routed experts + shared + router)."""
    arena, shared, router, gate, bias, mls, _, _ = st["_keep"]
    layers = len(mls)
    eb = F.expert_bytes(N, FF)
    lay = [F.MoeLayer(arena.blob(l, 0), arena.stride, E, shared[l].data_ptr(), router[l], gate[l], N, FF, K)
           for l in range(layers)]
    stream = torch.cuda.Stream()
    res = {}
    reps = max(2, args.window_reps)
    for T in (1, 2, 3, 5, 8):
        x = torch.empty((layers, T, N), dtype=torch.float32, device="cuda")
        for l in range(layers):
            if T == 3:
                F.gen.correlated(x[l], 1, l, F.gen.X_TENSOR, 3, N, 0.8)
            else:
                F.gen.normal(x[l], 0, l, F.gen.X_TENSOR + T, 1.0)
        out = torch.empty((layers, T, N), dtype=torch.float32, device="cuda")
        ids = torch.empty((layers, T, K), dtype=torch.int32, device="cuda")
        ws = torch.empty(lay[0].workspace_bytes(T), dtype=torch.uint8, device="cuda")

        def body():
            for l in range(layers):
                lay[l].forward(x[l], out[l], T=T, ids=ids[l], ws=ws)
        with torch.cuda.stream(stream):
            body()
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            body()
        with torch.cuda.stream(stream):
            g.replay()
        stream.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
        stream.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * layers)
        idh = ids.cpu().numpy()
        distinct = float(np.mean([len(np.unique(idh[l])) for l in range(layers)]))
        need = (distinct + 1) * eb + E * N * 4 + N * 4
        # T <= 4: the grouped decode kernels; 5 .. 8: router + top-k + one moe_hits launch + combine
        path = "decode" if T * K <= 63 and T < args.window_min_t else ("window" if T <= 8 else "prefill")
        res[f"T{T}"] = dict(us_per_call=round(us, 2), tokens_per_s=round(T / us * 1e6, 1), path=path,
                            distinct_experts=round(distinct, 2), GBps=round(need / (us * 1e-6) / 1e9, 1))
        if T > 1:   # per-kernel averages over an eager pass of the 48 calls, queued behind a spin kernel
            def eager():
                with torch.cuda.stream(stream):
                    torch.cuda._sleep(SPIN_CYCLES)
                    body()
            kt = kernel_times(F, eager)
            stream.synchronize()
            res[f"T{T}"]["kernels_us"] = {k: round(v[0] * 1e3 / max(v[1], 1), 2) for k, v in kt.items()}
        del g
        log(f"window T={T}: {us:.2f} us/call ({path}), {distinct:.2f} distinct experts")
    return res


# ---------------------------------------------------------------- CPU baseline

def _host_cpus():
    """(CPUs in this process's affinity mask, one logical CPU per physical core among them, the
    CPU model name)."""
    cpus = sorted(os.sched_getaffinity(0))
    cores = {}
    for c in cpus:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/thread_siblings_list") as f:
                key = f.read().strip()
        except OSError:
            key = str(c)
        cores.setdefault(key, c)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return len(cpus), sorted(cores.values()), model


def cpu_baseline(args, F, torch, stack):
    """The reference's moe_cpu (oracle/_ref: its own CPU sources compiled here, AVX-512 VNNI on its
    CpuPool) or, when that was not built, the oracle's restatement, on a sample of config 2: the
    first `cpu_layers` layers' experts copied to host RAM, tokens chained through them with routing
    done on the host (numpy fp32 router GEMV + top-10 + softmax); the per-layer time is scaled to 48
    layers. Run with one worker per physical core of this process's CPUs (the reported value) and
    again with 8 workers."""
    from oracle import oracle as O
    arena, shared, router, gate, bias, mls, _, _ = stack["_keep"]
    nl = args.cpu_layers
    host = torch.empty((nl, E, arena.stride), dtype=torch.uint8)
    import ctypes as C
    for l in range(nl):
        t = torch.empty(E * arena.stride, dtype=torch.uint8, device="cuda")
        _copy_arena_layer(arena, l, t)
        host[l] = t.view(E, arena.stride).cpu()
        del t
    torch.cuda.synchronize()
    sh_h = shared[:nl].cpu().numpy()
    rw = router[:nl].cpu().numpy()
    gw = gate[:nl].cpu().numpy()
    bh = bias[:nl].cpu().numpy()
    host_np = host.numpy()
    n_aff, phys, model = _host_cpus()
    n_phys = len(phys)
    kind = "reference" if O.have_ref() else "port"
    R = O.ref() if O.have_ref() else None
    rng_x = O.gen_normal(2, 0, O.X_TENSOR, 64 * N).reshape(64, N)
    blobs = (C.c_void_p * 11)()
    try:
        from threadpoolctl import threadpool_limits
    except Exception:
        threadpool_limits = None

    def sample(workers, seconds):
        # the pool pinned to one logical CPU per physical core, as the reference's bench pins it
        # (to the cores this process may use); the caller thread is pinned too and restored after
        saved_aff = os.sched_getaffinity(0)
        pin = (C.c_int * len(phys))(*phys)
        pool = R.ref_pool_create_cpus(workers, pin, len(phys)) if R else None
        # numpy's BLAS threads stay at one: idle BLAS workers spinning beside the pool's would steal its cores
        limiter = threadpool_limits(1) if threadpool_limits else None
        route_times, moe_times = [], []
        t_end = time.perf_counter() + seconds
        steps = 0
        try:
            while time.perf_counter() < t_end and steps < 64:
                x = rng_x[steps].copy()
                for l in range(nl):
                    t0 = time.perf_counter()
                    u = (x / np.sqrt(np.float32((x.astype(np.float64) ** 2).mean()) + np.float32(1e-6))).astype(np.float32)
                    lg = rw[l] @ u + bh[l]
                    top = np.argsort(-lg, kind="stable")[:K]
                    p = np.exp((lg - lg.max()).astype(np.float64))
                    p /= p.sum()
                    w = (p[top] / p[top].sum()).astype(np.float32)
                    gl = float(gw[l] @ u)
                    order = np.argsort(top)
                    for i, k in enumerate(order):
                        blobs[i] = host_np[l, top[k]].ctypes.data
                    blobs[10] = sh_h[l].ctypes.data
                    ntok = np.ones(11, np.int32)
                    tok = np.zeros(44, np.int32)
                    wv = np.zeros(44, np.float32)
                    wv[0:40:4] = w[order]
                    wv[40] = 1.0 / (1.0 + np.exp(-np.clip(gl, -80.0, 80.0)))
                    out = np.zeros(N, np.float32)
                    t1 = time.perf_counter()
                    if R:
                        prep = R.ref_moe_prepare(pool, N, FF, C.cast(blobs, C.c_void_p), ntok, tok, wv, 11, u, 1)
                        R.ref_moe_run(pool, prep, out, N)
                        R.ref_moe_free(prep)
                    else:
                        qs, d = O.quantize_q8(u)
                        O.lib().orc_moe_cpu(N, FF, C.cast(blobs, C.c_void_p), ntok, tok, wv, 11, qs, d, 1, out, N,
                                            workers, 1)
                    t2 = time.perf_counter()
                    route_times.append(t1 - t0)
                    moe_times.append(t2 - t1)
                    x = x + out
                steps += 1
        finally:
            if limiter is not None and hasattr(limiter, "unregister"):
                limiter.unregister()
            if pool:
                R.ref_pool_destroy(pool)
            os.sched_setaffinity(0, saved_aff)
        t_layer = float(np.median([a + b for a, b in zip(route_times, moe_times)]))
        return dict(workers=workers, tokens=steps, us_per_layer=round(t_layer * 1e6, 1),
                    route_us=round(float(np.median(route_times)) * 1e6, 1),
                    moe_cpu_us=round(float(np.median(moe_times)) * 1e6, 1),
                    moe_cpu_GBps=round(11 * F.expert_bytes(N, FF) / float(np.median(moe_times)) / 1e9, 2),
                    tokens_per_s=round(1.0 / (LAYERS * t_layer), 2),
                    moe_cpu_tokens_per_s=round(1.0 / (LAYERS * float(np.median(moe_times))), 2))

    full = sample(n_phys, args.cpu_seconds)
    eight = sample(8, args.cpu_seconds / 2)
    what = "the reference moe_cpu (AVX-512 VNNI) on its CpuPool" if R else "the oracle's moe_cpu restatement"
    return dict(value=full["tokens_per_s"], unit="tokens/s", cores=n_phys, kind=kind, cpu_model=model,
                moe_cpu_only_tokens_per_s=full["moe_cpu_tokens_per_s"], pinned=bool(R),
                sample=(f"{full['tokens']} tokens x {nl} of {LAYERS} layers of configs[2] on the host CPU "
                        f"({model}; {n_aff} CPUs in this process's affinity mask, {n_phys} physical cores): RMS norm "
                        f"+ numpy fp32 router + top-10 on one thread (median {full['route_us']:.0f} us), then {what} with "
                        f"{n_phys} workers pinned one per physical core over the 10 routed + shared experts (median "
                        f"{full['moe_cpu_us']:.0f} us); median {full['us_per_layer']:.0f} us/layer x {LAYERS} layers; "
                        f"moe_cpu alone {full['moe_cpu_tokens_per_s']:.1f} tokens/s"),
                all_cores=full, workers_8=eight)


def _copy_arena_layer(arena, l, dst):
    """Device-to-device hipMemcpy of layer l's E blobs (one contiguous range of the arena) into dst."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    rc = hip.hipMemcpy(C.c_void_p(dst.data_ptr()), C.c_void_p(arena.blob(l, 0)), E * arena.stride, 3)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy failed: {rc}")


# ---------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=384)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--prefill-reps", type=int, default=10)
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="first run 3 plain device copies of MIB MiB (scales the HBM byte counters of a profile)")
    ap.add_argument("--timing-steps", type=int, default=3, help="decode steps in the per-kernel timing pass")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-windows", action="store_true", help="skip configs[0]/[1] and the other window sizes")
    ap.add_argument("--window-reps", type=int, default=8, help="replays of the 48-call graph per window size")
    ap.add_argument("--no-mixed", action="store_true", help="skip configs[4]")
    ap.add_argument("--decode-grid", type=int, default=0, help="workgroups of a persistent decode call (0: one per CU)")
    ap.add_argument("--decode-xcd", type=int, default=0,
                    help="1: persistent single-token calls split each layer by XCD (decode2.hip) where the shape "
                         "fits; 0: the single-grid persistent kernel (decode1.hip)")
    ap.add_argument("--decode-path", choices=["stack", "fused", "three"], default="stack",
                    help="the 48 layers as one persistent launch (stack, default), one persistent launch per layer "
                         "(fused), or three kernels per layer (three)")
    ap.add_argument("--window-min-t", type=int, default=2,
                    help="windows of at least this many tokens (2..8) take the window path (router, top-k and "
                         "grouping in one workgroup, one moe_hits launch, combine); 9: none")
    ap.add_argument("--route-waves", type=int, default=1, choices=[1, 8],
                    help="waves of a persistent decode workgroup that route the token (8: all, 1: one)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        sys.exit("bench.py: this build measures one MI355X; multi-GPU (expert-parallel) runs are not part of it "
                 "(see DESIGN.md, 'How the path would shard')")
    import torch
    import flashrt_amd as F
    F.lib()
    torch.cuda.set_device(0)
    if args.calib_copy:
        src = torch.ones(args.calib_copy << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    F.set_option("decode_fused", 0 if args.decode_path == "three" else 1)
    F.set_option("window_min_t", args.window_min_t)
    F.set_option("decode_grid", args.decode_grid)
    F.set_option("decode_xcd", args.decode_xcd)
    F.set_option("route_waves", args.route_waves)
    st = run_stack(args, F, torch)
    if st["sync_error"]:
        sys.exit("bench.py: a persistent decode call ran out of time waiting for another workgroup")
    ms = st["ms_per_step"]
    tok_s = 1e3 / ms
    expert_bytes_tok = args.layers * (K + 1) * F.expert_bytes(N, FF)
    router_bytes_tok = args.layers * (E * N * 4 + N * 4)
    stack_tbs = expert_bytes_tok / (ms * 1e-3) / 1e12

    # roofline of the dominant decode kernel
    kt = st["kernels"]
    # algorithmic bytes per launch: the expert weights each launch reads once ((K + 1) blobs per
    # token and layer); the router matrices are reported beside them (frac_with_router), not in them
    router_layer = E * N * 4 + N * 4
    per_launch_bytes = {
        "dec1_stack": args.layers * (K + 1) * F.expert_bytes(N, FF),
        "dec2_stack": args.layers * (K + 1) * F.expert_bytes(N, FF),
        "dec1_layer": (K + 1) * F.expert_bytes(N, FF),
        "dec2_layer": (K + 1) * F.expert_bytes(N, FF),
        "dec_route_gateup": (K + 1) * 2 * F.lib().frt_q2_mat_bytes(FF, N),
        "dec_down": (K + 1) * F.lib().frt_q2_mat_bytes(N, FF),
        "router_quant": 0,
    }
    router_bytes = {"dec1_stack": args.layers * router_layer, "dec2_stack": args.layers * router_layer,
                    "dec1_layer": router_layer, "dec2_layer": router_layer, "router_quant": router_layer}
    dom = max(kt, key=lambda k: kt[k][0])
    dom_avg_ms = kt[dom][0] / kt[dom][1]
    eager_avg_us = dom_avg_ms * 1e3
    if dom.endswith("_stack") and st.get("replay_us"):
        dom_avg_ms = st["replay_us"] * 1e-3   # the launch as the timed loop runs it (graph replays)
    dom_bytes = per_launch_bytes.get(dom)
    achieved = dom_bytes / (dom_avg_ms * 1e-3) / 1e9 if dom_bytes else None
    achieved_wr = (dom_bytes + router_bytes.get(dom, 0)) / (dom_avg_ms * 1e-3) / 1e9 if dom_bytes else None
    kernels = {k: dict(avg_us=round(v[0] / v[1] * 1e3, 2), launches=v[1],
                       share=round(v[0] / sum(x[0] for x in kt.values()), 3)) for k, v in kt.items()}
    for k, b in per_launch_bytes.items():
        if k in kt:
            kernels[k]["algo_bytes"] = int(b)
            kernels[k]["GBps"] = round(b / (kt[k][0] / kt[k][1] * 1e-3) / 1e9, 1)

    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            traffic = (json.load(f).get("kernels", {}).get(dom) or {}).get("bytes")   # HBM bytes per launch, rocprofv3 PMC

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded device generator: uniform 2-bit codes, fp16 |N(0,1)|*0.02 scales, fp32 N(0,0.02) "
                "router, N(0,1) inputs, per-layer Zipf(1.1) logit prior)",
        "config": {"workload": f"configs[2]: {args.layers}-layer Q2_0 MoE stack, decode bs=1, {args.steps} steps",
                   "hidden": N, "experts": E, "top_k": K, "expert_ff": FF, "shared_ff": FF, "layers": args.layers,
                   "global_batch": 1, "seq_len": 1, "parallelism": "none (one GPU)"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1) if achieved else None,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None, "traffic": traffic,
                     "algo_bytes": dom_bytes, "avg_us": round(dom_avg_ms * 1e3, 2),
                     "avg_from": "events around 64 graph replays" if dom.endswith("_stack") else "eager launch events",
                     "eager_avg_us": round(eager_avg_us, 2),
                     "frac_with_router": round(achieved_wr / HBM_PEAK_GBS, 4) if achieved_wr else None},
        "stack": {"expert_bytes_per_token": expert_bytes_tok, "router_bytes_per_token": router_bytes_tok,
                  "expert_TBps": round(stack_tbs, 3), "expert_hbm_frac": round(stack_tbs * 1e3 / HBM_PEAK_GBS, 4),
                  "expert_plus_router_hbm_frac": round((expert_bytes_tok + router_bytes_tok) / (ms * 1e-3) / 1e9
                                                       / HBM_PEAK_GBS, 4),
                  "kernels": kernels},
    }
    def pf_entry(pf):
        return {"tokens_per_s": round(pf.tokens_per_s, 1), "ms_per_layer": round(pf.ms, 4),
                "expert_gflop": round(pf.flops / 1e9, 2),
                "mfma_frac_layer": round(pf.flops / (pf.ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                "kernels": {k: dict(avg_us=round(v[0] / v[1] * 1e3, 2), launches=v[1]) for k, v in pf.kernels.items()},
                "mfma": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                         for k, v in pf.util.items()}}
    if not args.no_prefill:
        pf = run_prefill(args, F, torch)
        line["prefill_2k"] = pf_entry(pf)
        # the prefill roofline: expert flops over the grouped GEMM kernels' summed average durations
        parts = [p for p in ("pf_gateup", "pf_gateup1", "pf_down", "pf_down1") if p in pf.kernels]
        if parts:
            gemm_ms = sum(pf.kernels[p][0] / pf.kernels[p][1] for p in parts)
            tf = pf.flops / (gemm_ms * 1e-3) / 1e12
            line["roofline_prefill"] = {"bound": "mfma", "kernels": parts, "achieved": round(tf, 1),
                                        "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                        "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "avg_us": round(gemm_ms * 1e3, 2),
                                        "flops": pf.flops, "frac_layer": round(pf.flops / (pf.ms * 1e-3) / 1e12
                                                                               / MFMA_F16_PEAK_TFLOPS, 4)}
    if not args.no_mixed:
        line["mixed_cfg4"] = pf_entry(run_mixed(args, F, torch))
    if not args.no_windows:
        win = run_windows(args, F, torch, st)
        line["decode_cfg0"] = win["T1"]
        line["decode_cfg1"] = win["T3"]
        line["decode_windows"] = win
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args, F, torch, st)
    print(json.dumps(line), flush=True)
    st.clear()
    torch.cuda.synchronize()
    sys.stderr.flush()


if __name__ == "__main__":
    main()
