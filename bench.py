#!/usr/bin/env python3
"""Decode-attention benchmark of the MI355X attention block (one GPU).

Default workload: one decode step of the Llama-3-8B attention block at an
8K context -- H32 / HK8 / D128, 8192 cached rows per layer in an fp32 KV
cache, RoPE theta 5e5, new token at position 8192 -- over all 32 layers back
to back, each layer with its own cache (2.15 GB in HBM).  A "step" is those
32 layer calls of pkh_attn_decode_async, each doing RoPE on q/k, the KV
append and GQA attention over 8193 rows.

Prints one JSON line.  `value` is whole-job KV throughput in GB/s from the
algorithmic bytes per layer-step
    2*(ctx+1)*HK*D*s_kv + 2*H*D*4 + 2*HK*D*(4 + s_kv)
(KV stream, q in, o out, new k/v in, appended row out) over the timed wall
time.  `roofline.achieved` is the same bytes over the average duration of one
layer call measured with HIP events on the launch stream.  `cpu_baseline` is
the reference's own attention (its sources compiled with its AVX-512 code
and OpenMP, oracle/_ref) timed on this host's cores over a bounded sample of
the same workload; the oracle's vectorised build where the reference has no
counterpart (fp16 ragged batches) or is not built.

Inputs are synthetic: N(0,1) from torch's CUDA generator seeded with the
workload's seed, already resident in HBM when timing starts.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn KV GB/s (% HBM peak) + µs/layer-step, Llama-3-8B shape ctx 8K"
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    "llama3-8b-decode-ctx8192": dict(H=32, HK=8, D=128, ctx=8192, theta=5e5, layers=32,
                                     kv="f32", seed=3),
    "tinyllama-decode-ctx2048": dict(H=32, HK=4, D=64, ctx=2048, theta=1e4, layers=1,
                                     kv="f32", seed=2),
    "tinyllama-decode-ctx2048-rotating64": dict(H=32, HK=4, D=64, ctx=2048, theta=1e4,
                                                layers=64, kv="f32", seed=2),
}

# Causal prefill of a 2048-token prompt from position 0 through the 32
# attention layers of the Llama-3-8B shape (fp32 cache, fp16 MFMA operands).
PREFILL_WORKLOADS = {
    "llama3-8b-prefill-2048": dict(H=32, HK=8, D=128, S=2048, pos0=0, theta=5e5, layers=32,
                                   kv="f32", seed=4),
    # A 128-token prompt chunk after 8192 cached rows (chunked prefill of a
    # long prompt, the layer-major forward's unit): the cache rows [0, 8192)
    # are N(0,1) from the same generator.
    "llama3-8b-prefill-chunk128-ctx8192": dict(H=32, HK=8, D=128, S=128, pos0=8192, theta=5e5,
                                               layers=32, kv="f32", seed=6),
}
# One decode step of 16 sequences with contexts drawn from U[4096, 32768]
# (numpy default_rng(5)) over the 32 layers of the Llama-3-8B shape, fp16 KV.
RAGGED_WORKLOADS = {
    "llama3-8b-ragged16-fp16": dict(H=32, HK=8, D=128, n_seqs=16, ctx_lo=4096, ctx_hi=32768,
                                    ctx_seed=5, theta=5e5, layers=32, kv="f16", seed=5),
}
RAGGED_METRIC = "ragged-decode KV GB/s (% HBM peak), 16 sequences 4K-32K, Llama-3-8B shape, fp16 KV"

PREFILL_METRIC = "prefill-attn TFLOP/s (causal, useful FLOPs), Llama-3-8B shape, 2048 tokens"
MFMA_F16_PEAK_TFLOPS = 2500.0
PREFILL_TOL = 2e-3


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def decode_bytes(ctx: int, H: int, HK: int, D: int, s_kv: int) -> int:
    return 2 * (ctx + 1) * HK * D * s_kv + 2 * H * D * 4 + 2 * HK * D * (4 + s_kv)


def traffic_from_profiles(workload: str):
    """HBM bytes per launch measured with rocprofv3 PMC counters (FETCH_SIZE,
    WRITE_SIZE) and scaled by a plain copy kernel's reading, if recorded."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        t = json.load(open(path)).get(workload)
        return None if t is None else float(t["bytes_per_launch"])
    except (ValueError, KeyError, TypeError):
        return None


def cpu_model() -> str:
    """The host CPU's model name, as /proc/cpuinfo gives it."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def reference_available() -> bool:
    from oracle import pyref
    return pyref.available()


class _TimingModel:
    """The compiled reference (oracle/_ref) loaded with a synthetic Llama of
    the workload's attention shape and a hidden size of 64, so that its
    forward pass is almost all attention; see oracle/gguf.py."""

    def __init__(self, cfg, layers, ctx, tmpdir):
        from oracle import gguf, pyref
        self.pyref = pyref
        path = os.path.join(tmpdir, f"timing_{cfg['H']}_{cfg['HK']}_{cfg['D']}_{layers}_{ctx}.gguf")
        gguf.write_timing_model(path, n_layers=layers, n_heads=cfg["H"], n_kv_heads=cfg["HK"],
                                head_dim=cfg["D"], ctx=ctx, theta=cfg["theta"])
        self.m = pyref.RefModel(path)

    def threads(self, n):
        self.pyref.lib().ref_set_threads(n)

    def fill(self, K, V, rows):
        """Cache rows [0, rows) of every layer from host arrays [rows][HK][D]."""
        for layer in range(self.m.n_layers):
            self.m.kv_write(0, layer, 0, K)
            self.m.kv_write(1, layer, 0, V)

    def step(self, pos) -> float:
        """Seconds for one token through the reference's pickle_fast_forward at
        position pos (attending rows [0, pos])."""
        self.m.pos = pos
        t0 = time.perf_counter()
        self.m.forward1(1)
        return time.perf_counter() - t0

    def prefill(self, n) -> float:
        """Seconds for the reference's prefill of n tokens from position 0: one
        pickle_fast_forward call, which loops over the tokens."""
        self.m.pos = 0
        toks = np.ones(n, np.int32)
        logits = np.zeros(self.m.vocab_size, np.float32)
        t0 = time.perf_counter()
        rc = self.pyref.lib().ref_forward_n(self.m.h, toks.ctypes.data, n, logits.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"pickle_fast_forward rc={rc}")
        return time.perf_counter() - t0

    def close(self):
        self.m.close()


def cpu_baseline_decode_reference(K, V, cfg, layers, threads):
    """The reference's own attention (pickle_fast_forward of oracle/_ref, the
    reference's sources compiled with its AVX-512 intrinsics and OpenMP over
    heads, src/pickle_fast.c:1946-2094) at the workload's shape: one decode
    step over `layers` layers at the workload's position, less the same
    step at position 0 (the model's projections, RMSNorm and logits, about
    2% of it); then one layer on one thread.  Returns seconds per
    layer-step for `threads` threads and for one thread."""
    import tempfile
    ctx = cfg["ctx"]
    kh = K[0].contiguous().cpu().numpy()[:ctx]
    vh = V[0].contiguous().cpu().numpy()[:ctx]
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        for n_layers, n_threads in ((layers, threads), (1, 1)):
            tm = _TimingModel(cfg, n_layers, ctx + 1, tmp)
            try:
                tm.fill(kh, vh, ctx)
                tm.threads(n_threads)
                tm.step(ctx)                          # warm-up (tables, pages)
                full = tm.step(ctx)
                tm.step(0)
                base = tm.step(0)
                out[n_threads] = max(full - base, 1e-9) / n_layers
            finally:
                tm.close()
    return out[threads], out[1]


def cpu_baseline_decode_port(K, V, q, k, v, cfg, layers, threads):
    """The oracle's restatement of the reference's OpenMP attention, built at
    -O3 with 512-bit vectors (oracle/liboracle_avx512.so, bit-identical to
    the -O2 oracle), on host copies of `layers` layers: one warm-up layer
    call, then one timed decode step over those layers.  Used where the
    compiled reference is not present."""
    from oracle import pyoracle as po
    H, HK, D, ctx = cfg["H"], cfg["HK"], cfg["D"], cfg["ctx"]
    prev = po.use_build("avx512")
    try:
        _, sin, cos = po.rope_tables(D, cfg["theta"], ctx + 1)
        host = [(K[L].contiguous().cpu().numpy(), V[L].contiguous().cpu().numpy(),
                 q[L].cpu().numpy(), k[L].cpu().numpy(), v[L].cpu().numpy()) for L in range(layers)]
        kc, vc, qq, kk, vv = host[0]
        po.decode_step(kc, vc, ctx, qq, kk, vv, sin, cos, threads)     # warm-up
        t0 = time.perf_counter()
        for kc, vc, qq, kk, vv in host:
            po.decode_step(kc, vc, ctx, qq, kk, vv, sin, cos, threads)
        return (time.perf_counter() - t0) / layers
    finally:
        po.use_build(prev)


def run_decode(args, cfg):
    import torch
    import lestramanika_amd as pk
    from oracle import pyoracle as po

    torch.cuda.set_device(0)
    lib = pk.load()
    pk.check(lib.pkh_init(0), "pkh_init")
    H, HK, D, ctx, L = cfg["H"], cfg["HK"], cfg["D"], cfg["ctx"], cfg["layers"]
    max_seq = ctx + 1
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg["seed"])
    log(f"bench: allocating {L} layers x {HK} heads x {max_seq} rows x (K {D} | V {D}) fp32")
    # The cache in the library's default device layout (each layer
    # [kv_head][pos][K row | V row]); pkh_kv_t is caller-owned, as
    # pickle_fast_kv_t is, so it can point at torch's buffer.
    KV = torch.zeros((L, HK, max_seq, 2, D), dtype=torch.float32, device=dev)
    for layer in range(L):
        KV[layer, :, :ctx].normal_(generator=gen)
    K = KV[:, :, :, 0, :].permute(0, 2, 1, 3)       # [L][pos][HK][D] views
    V = KV[:, :, :, 1, :].permute(0, 2, 1, 3)
    q = torch.randn((L, H, D), generator=gen, device=dev)
    k = torch.randn((L, HK, D), generator=gen, device=dev)
    v = torch.randn((L, HK, D), generator=gen, device=dev)
    ao = torch.zeros((L, H, D), device=dev)

    kv = pk.KV()
    kv.n_layers, kv.n_kv_heads, kv.head_dim, kv.max_seq = L, HK, D, max_seq
    kv.k_stride_layer = kv.v_stride_layer = HK * max_seq * 2 * D
    kv.k, kv.v = KV.data_ptr(), KV.data_ptr() + D * 4
    kv.dtype, kv.device = pk.PKH_KV_F32, 0
    kv.stride_pos, kv.stride_head = 2 * D, max_seq * 2 * D

    half = min(D // 2, 64)
    sin = np.zeros((max_seq, half), np.float32)
    cos = np.zeros((max_seq, half), np.float32)
    lib.pkh_rope_host_tables(D, cfg["theta"], 0, ctx, None, sin.ctypes.data, cos.ctypes.data)
    rope = pk.Rope()
    pk.check(lib.pkh_rope_alloc(max_seq, half, ctypes.byref(rope)), "pkh_rope_alloc")
    pk.check(lib.pkh_rope_upload(ctypes.byref(rope), sin.ctypes.data, cos.ctypes.data, max_seq),
             "pkh_rope_upload")

    kvp, rp = ctypes.byref(kv), ctypes.byref(rope)
    qp = [q[i].data_ptr() for i in range(L)]
    kp = [k[i].data_ptr() for i in range(L)]
    vp = [v[i].data_ptr() for i in range(L)]
    op = [ao[i].data_ptr() for i in range(L)]
    call = lib.pkh_attn_decode_async

    def step(stream):
        sp = ctypes.c_void_p(stream.cuda_stream)
        for layer in range(L):
            rc = call(kvp, rp, layer, ctx, H, qp[layer], kp[layer], vp[layer], op[layer], sp)
            if rc != 0:
                raise pk.PkhError(rc, "pkh_attn_decode_async")

    stream = torch.cuda.current_stream()
    log(f"bench: warmup {args.warmup} eager steps")
    for _ in range(args.warmup):
        step(stream)
    torch.cuda.synchronize()

    # Eager launches: one host call per layer (reported beside the graph).
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(stream)
    torch.cuda.synchronize()
    eager_wall = time.perf_counter() - t0

    # The 32-layer step captured once as a HIP graph and replayed: what a
    # decode loop runs, without per-kernel host launch cost.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(torch.cuda.current_stream())
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()

    # Timed region: exactly K replays, bracketed by synchronize, with HIP
    # events on the replay stream around each replay.
    log(f"bench: timing {args.steps} graph replays x {L} layers")
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record(stream)
        graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    durs = np.array([e0.elapsed_time(e1) for e0, e1 in evs]) * 1e-3 / L   # s per layer-step

    s_kv = 4
    bpl = decode_bytes(ctx, H, HK, D, s_kv)
    n_launch = args.steps * L
    value = bpl * n_launch / wall / 1e9
    avg_launch = float(durs.mean())
    achieved = bpl / avg_launch / 1e9

    # The floor under one layer call on this box: the same replay of a
    # graph of L dependent launches of a one-element kernel, per launch.
    x1 = torch.zeros(1, device=dev)
    floor_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(floor_graph):
        for _ in range(L):
            x1.add_(1.0)
    for _ in range(args.warmup):
        floor_graph.replay()
    torch.cuda.synchronize()
    fevs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(args.steps)]
    for e0, e1 in fevs:
        e0.record(stream)
        floor_graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    node_us = float(np.mean([e0.elapsed_time(e1) for e0, e1 in fevs])) * 1e3 / L
    log(f"bench: graph node floor {node_us:.3f} us (one-element kernel, {L} nodes per graph)")

    # The host-pointer entry the seam binding uses (pkh_attn_decode with q, k,
    # v and ao in pageable host memory, as the reference's state buffers
    # are): one packed upload, the kernel, one download per layer call.  PCIe
    # included; reported beside the device-resident figure, never in value.
    hq = [np.ascontiguousarray(q[i].cpu().numpy()) for i in range(L)]
    hk = [np.ascontiguousarray(k[i].cpu().numpy()) for i in range(L)]
    hv = [np.ascontiguousarray(v[i].cpu().numpy()) for i in range(L)]
    hao = np.zeros((H, D), np.float32)
    host_steps = max(2, args.steps // 4)
    for layer in range(L):
        pk.check(lib.pkh_attn_decode(kvp, rp, layer, ctx, H, hq[layer].ctypes.data, hk[layer].ctypes.data,
                                     hv[layer].ctypes.data, hao.ctypes.data), "pkh_attn_decode")
    t0 = time.perf_counter()
    for _ in range(host_steps):
        for layer in range(L):
            lib.pkh_attn_decode(kvp, rp, layer, ctx, H, hq[layer].ctypes.data, hk[layer].ctypes.data,
                                hv[layer].ctypes.data, hao.ctypes.data)
    host_us = (time.perf_counter() - t0) / (host_steps * L) * 1e6
    log(f"bench: host-pointer entry {host_us:.2f} us/layer-step (PCIe both ways included)")

    # Parity of the benchmarked outputs (first and last layer) against the oracle.
    _, osin, ocos = po.rope_tables(D, cfg["theta"], max_seq)
    errs = []
    for layer in sorted({0, L - 1}):
        ref, _, _ = po.decode_step(K[layer].contiguous().cpu().numpy(),
                                   V[layer].contiguous().cpu().numpy(), ctx,
                                   q[layer].cpu().numpy(), k[layer].cpu().numpy(),
                                   v[layer].cpu().numpy(), osin, ocos, n_threads=16)
        errs.append(float(np.max(np.abs(ao[layer].cpu().numpy() - ref))))
    log(f"bench: max-abs err vs oracle (layers 0, {L - 1}): {max(errs):.3e}")

    cpu = None
    if not args.no_cpu_baseline:
        threads = min(16, os.cpu_count() or 1)
        sample_layers = min(L, args.cpu_layers)
        if reference_available():
            log(f"bench: CPU baseline (the compiled reference, {threads} threads, "
                f"{sample_layers} layers; then 1 thread, 1 layer)")
            t_cpu, t_one = cpu_baseline_decode_reference(K, V, cfg, sample_layers, threads)
            kind, build = "reference", ("the reference's src/pickle_fast.c compiled from its own "
                                        "sources (oracle/Makefile: -O3 -march=x86-64-v4 -fopenmp, "
                                        "its AVX-512 score and PV loops)")
            sample = (f"pickle_fast_forward of that build, one decode step over {sample_layers} "
                      f"layer(s) at position {ctx} of a synthetic Llama with this attention shape "
                      f"and hidden size 64 (oracle/gguf.py), cache rows N(0,1), less the same "
                      f"step at position 0 (its projections, ~2%)")
        else:
            log(f"bench: CPU baseline (oracle AVX-512 build, {threads} threads, {sample_layers} layers)")
            t_cpu = cpu_baseline_decode_port(K, V, q, k, v, cfg, sample_layers, threads)
            t_one = cpu_baseline_decode_port(K, V, q, k, v, cfg, 1, 1)
            kind, build = "port", ("oracle/pk_oracle.c at -O3 -march=x86-64-v4 "
                                   "-mprefer-vector-width=512, bit-identical to the -O2 oracle")
            sample = (f"one decode step over {sample_layers} layer(s) of the same workload "
                      f"({ctx} cached rows each)")
        cpu = {"value": round(bpl / t_cpu / 1e9, 3), "unit": "GB/s", "cores": threads,
               "kind": kind, "build": build, "sample": sample,
               "us_per_layer_step": round(t_cpu * 1e6, 2),
               "cpu_model": cpu_model(),
               "one_thread": {"value": round(bpl / t_one / 1e9, 3), "unit": "GB/s",
                              "us_per_layer_step": round(t_one * 1e6, 2),
                              "sample": "one layer of the same step on one thread"}}

    lib.pkh_rope_free(rp)
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: N(0,1) from torch's CUDA generator, seeded per workload",
        "config": {"workload": args.workload, "n_heads": H, "n_kv_heads": HK, "head_dim": D,
                   "context": ctx, "layers": L, "kv_dtype": cfg["kv"],
                   "rope_theta": cfg["theta"], "new_token_pos": ctx},
        "us_per_layer_step": round(wall / n_launch * 1e6, 3),
        "eager_us_per_layer_step": round(eager_wall / n_launch * 1e6, 3),
        "graph_node_floor_us": round(node_us, 3),
        "host_entry_us_per_layer_step": round(host_us, 2),
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "bytes_per_layer_step": bpl,
        "max_abs_err_vs_oracle": max(errs),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(args.workload),
                     "us_per_launch": round(avg_launch * 1e6, 3)},
        "cpu_baseline": cpu,
    }
    return result


def prefill_flops(H: int, D: int, S: int, pos0: int = 0) -> int:
    """Useful causal FLOPs: QK^T and PV over the n*(n+1)/2 (plus context)
    query-key pairs, 2 FLOPs per multiply-add, exp not counted."""
    pairs = S * pos0 + S * (S + 1) // 2
    return 4 * D * H * pairs


def oracle_prefill(q, k, v, cfg, threads):
    """The oracle's token loop (one restated decode step per prompt token) on
    one layer of the workload: the parity reference for the GPU outputs."""
    from oracle import pyoracle as po
    H, HK, D, S = cfg["H"], cfg["HK"], cfg["D"], cfg["S"]
    _, sin, cos = po.rope_tables(D, cfg["theta"], S)
    qq, kk, vv = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    kc = np.zeros((S, HK, D), np.float32)
    vc = np.zeros_like(kc)
    t0 = time.perf_counter()
    ao = po.prefill(kc, vc, 0, qq, kk, vv, sin, cos, threads)
    return time.perf_counter() - t0, ao


def cpu_baseline_prefill_reference(cfg, threads):
    """The reference's prefill (pickle_fast_forward over the prompt: one
    decode step per token through every layer, src/pickle_fast.c:1881-1898)
    of oracle/_ref on a one-layer synthetic model of the workload's attention
    shape, less that model's per-token cost outside attention (the same
    forward at position 0, times the prompt length).  Seconds per layer."""
    import tempfile
    S = cfg["S"]
    with tempfile.TemporaryDirectory() as tmp:
        tm = _TimingModel(cfg, 1, S, tmp)
        try:
            tm.threads(threads)
            tm.prefill(min(S, 64))                   # warm-up
            total = tm.prefill(S)
            tm.step(0)
            base = min(tm.step(0) for _ in range(5))
        finally:
            tm.close()
    return max(total - S * base, 1e-9), total


def run_prefill(args, cfg, name):
    import torch
    import lestramanika_amd as pk
    from oracle import pyoracle as po

    torch.cuda.set_device(0)
    lib = pk.load()
    pk.check(lib.pkh_init(0), "pkh_init")
    H, HK, D, S, L = cfg["H"], cfg["HK"], cfg["D"], cfg["S"], cfg["layers"]
    pos0 = cfg["pos0"]
    M = pos0 + S                                    # cache rows
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg["seed"])
    log(f"bench: prefill {name}: {L} layers, {S} tokens from position {pos0}, H{H} HK{HK} D{D}")
    KV = torch.zeros((L, HK, M, 2, D), dtype=torch.float32, device=dev)
    if pos0 > 0:
        for layer in range(L):
            KV[layer, :, :pos0].normal_(generator=gen)
    q = torch.randn((L, S, H, D), generator=gen, device=dev)
    k = torch.randn((L, S, HK, D), generator=gen, device=dev)
    v = torch.randn((L, S, HK, D), generator=gen, device=dev)
    ao = torch.zeros((L, S, H, D), device=dev)

    kv = pk.KV()
    kv.n_layers, kv.n_kv_heads, kv.head_dim, kv.max_seq = L, HK, D, M
    kv.k_stride_layer = kv.v_stride_layer = HK * M * 2 * D
    kv.k, kv.v = KV.data_ptr(), KV.data_ptr() + D * 4
    kv.dtype, kv.device = pk.PKH_KV_F32, 0
    kv.stride_pos, kv.stride_head = 2 * D, M * 2 * D
    half = min(D // 2, 64)
    sin = np.zeros((M, half), np.float32)
    cos = np.zeros((M, half), np.float32)
    lib.pkh_rope_host_tables(D, cfg["theta"], 0, M - 1, None, sin.ctypes.data, cos.ctypes.data)
    rope = pk.Rope()
    pk.check(lib.pkh_rope_alloc(M, half, ctypes.byref(rope)), "pkh_rope_alloc")
    pk.check(lib.pkh_rope_upload(ctypes.byref(rope), sin.ctypes.data, cos.ctypes.data, M),
             "pkh_rope_upload")
    kvp, rp = ctypes.byref(kv), ctypes.byref(rope)
    call = lib.pkh_attn_prefill_async

    def step(stream):
        sp = ctypes.c_void_p(stream.cuda_stream)
        for layer in range(L):
            rc = call(kvp, rp, layer, pos0, S, H, q[layer].data_ptr(),
                      k[layer].data_ptr(), v[layer].data_ptr(), ao[layer].data_ptr(), sp)
            if rc != 0:
                raise pk.PkhError(rc, "pkh_attn_prefill_async")

    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        step(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(torch.cuda.current_stream())
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    steps = max(1, args.steps // 4)
    log(f"bench: timing {steps} graph replays x {L} layer prefills")
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record(stream)
        graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    durs = np.array([e0.elapsed_time(e1) for e0, e1 in evs]) * 1e-3 / L
    fl = prefill_flops(H, D, S, pos0)
    value = fl * steps * L / wall / 1e12
    avg_launch = float(durs.mean())
    achieved = fl / avg_launch / 1e12

    cpu = None
    errs = []
    threads = min(16, os.cpu_count() or 1)
    if not args.no_cpu_baseline and pos0 == 0:
        if reference_available():
            log(f"bench: CPU baseline (the compiled reference's token loop, {threads} threads, 1 layer)")
            t_cpu, t_total = cpu_baseline_prefill_reference(cfg, threads)
            cpu = {"value": round(fl / t_cpu / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
                   "kind": "reference",
                   "build": ("the reference's src/pickle_fast.c compiled from its own sources "
                             "(oracle/Makefile: -O3 -march=x86-64-v4 -fopenmp)"),
                   "sample": (f"pickle_fast_forward of that build over a {S}-token prompt from "
                              f"position 0 (its token loop) on a one-layer synthetic Llama with "
                              f"this attention shape and hidden size 64, less {S} times the "
                              f"model's one-token cost at position 0 (its projections)"),
                   "us_per_layer": round(t_cpu * 1e6, 1),
                   "us_per_layer_with_projections": round(t_total * 1e6, 1),
                   "cpu_model": cpu_model()}
        else:
            log(f"bench: CPU baseline (oracle token loop, AVX-512 build, {threads} threads, 1 layer)")
            from oracle import pyoracle as po
            prev = po.use_build("avx512")
            try:
                t_cpu, _ = oracle_prefill(q[0], k[0], v[0], cfg, threads)
            finally:
                po.use_build(prev)
            cpu = {"value": round(fl / t_cpu / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
                   "kind": "port",
                   "build": ("oracle/pk_oracle.c at -O3 -march=x86-64-v4 "
                             "-mprefer-vector-width=512, bit-identical to the -O2 oracle"),
                   "sample": (f"one layer's {S}-token causal prefill of the same workload with "
                              f"the oracle's token loop (one restated reference decode step "
                              f"per token)"),
                   "us_per_layer": round(t_cpu * 1e6, 1)}
    _, osin, ocos = po.rope_tables(D, cfg["theta"], M)
    for layer in sorted({0, L - 1}):
        kc = np.zeros((M, HK, D), np.float32)
        vc = np.zeros_like(kc)
        kc[:pos0] = KV[layer, :, :pos0, 0].permute(1, 0, 2).cpu().numpy()
        vc[:pos0] = KV[layer, :, :pos0, 1].permute(1, 0, 2).cpu().numpy()
        ref = po.prefill(kc, vc, pos0, q[layer].cpu().numpy(), k[layer].cpu().numpy(),
                         v[layer].cpu().numpy(), osin, ocos, threads)
        errs.append(float(np.max(np.abs(ao[layer].cpu().numpy() - ref))))
    log(f"bench: prefill max-abs err vs oracle: {max(errs):.3e} (tolerance {PREFILL_TOL})")
    lib.pkh_rope_free(rp)
    metric = PREFILL_METRIC if pos0 == 0 else (
        f"prefill-attn TFLOP/s (causal, useful FLOPs), Llama-3-8B shape, {S} tokens after "
        f"{pos0} cached rows")
    return {
        "metric": metric,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA operands, f32 accumulate/softmax/cache",
        "data": "synthetic: N(0,1) from torch's CUDA generator, seeded per workload",
        "config": {"workload": name, "n_heads": H, "n_kv_heads": HK, "head_dim": D,
                   "tokens": S, "pos0": cfg["pos0"], "layers": L, "kv_dtype": cfg["kv"],
                   "rope_theta": cfg["theta"]},
        "us_per_layer": round(wall / (steps * L) * 1e6, 3),
        "flops_per_layer": fl,
        "pct_mfma_peak": round(100.0 * value / MFMA_F16_PEAK_TFLOPS, 2),
        "max_abs_err_vs_oracle": max(errs),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": traffic_from_profiles(name),
                     "us_per_launch": round(avg_launch * 1e6, 3)},
        "cpu_baseline": cpu,
    }


def cpu_baseline_ragged(KV, ctx, slot0, q, k, v, cfg, threads):
    """The oracle's single-sequence fp16 decode step, looped over the
    sequences (the reference has no batch API), on host copies of layer 0."""
    from oracle import pyoracle as po
    H, HK, D = cfg["H"], cfg["HK"], cfg["D"]
    _, sin, cos = po.rope_tables(D, cfg["theta"], max(ctx) + 1)
    lay = KV[0].cpu().numpy().view(np.uint16)          # [HK][slots][2][D]
    host = []
    for s, c in enumerate(ctx):
        rows = lay[:, slot0[s]:slot0[s] + c + 1]       # [HK][c+1][2][D]
        kc = np.ascontiguousarray(rows[:, :, 0].transpose(1, 0, 2))
        vc = np.ascontiguousarray(rows[:, :, 1].transpose(1, 0, 2))
        host.append((kc, vc))
    qq, kk, vv = q[0].cpu().numpy(), k[0].cpu().numpy(), v[0].cpu().numpy()
    outs = []
    t0 = time.perf_counter()
    for s, c in enumerate(ctx):
        kc, vc = host[s]
        outs.append(po.decode_step_f16(kc, vc, c, qq[s], kk[s], vv[s], sin, cos, threads))
    return time.perf_counter() - t0, np.stack(outs)


def run_ragged(args, cfg, name):
    import torch
    import lestramanika_amd as pk

    torch.cuda.set_device(0)
    lib = pk.load()
    pk.check(lib.pkh_init(0), "pkh_init")
    H, HK, D, L, n = cfg["H"], cfg["HK"], cfg["D"], cfg["layers"], cfg["n_seqs"]
    ctx = np.random.default_rng(cfg["ctx_seed"]).integers(
        cfg["ctx_lo"], cfg["ctx_hi"], size=n, endpoint=True).tolist()
    slot0 = np.zeros(n + 1, np.int64)
    slot0[1:] = np.cumsum([c + 1 for c in ctx])
    slots = int(slot0[-1])
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg["seed"])
    log(f"bench: ragged {name}: {n} sequences, sum(ctx) = {sum(ctx)}, {L} layers, fp16 KV "
        f"({L * HK * slots * 2 * D * 2 / 1e9:.1f} GB)")
    # Caller-owned pkh_kv_batch_t over torch's buffer, in the library's
    # layout: each layer [kv_head][slot][K row | V row].
    KV = torch.empty((L, HK, slots, 2, D), dtype=torch.float16, device=dev)
    for layer in range(L):
        KV[layer].normal_(generator=gen)
    q = torch.randn((L, n, H, D), generator=gen, device=dev)
    k = torch.randn((L, n, HK, D), generator=gen, device=dev)
    v = torch.randn((L, n, HK, D), generator=gen, device=dev)
    ao = torch.zeros((L, n, H, D), device=dev)
    d_slot0 = torch.from_numpy(slot0).to(dev)
    h_slot0 = (ctypes.c_int64 * (n + 1))(*slot0.tolist())
    h_max = (ctypes.c_int * n)(*[c + 1 for c in ctx])
    kvb = pk.KVBatch()
    kvb.n_layers, kvb.n_kv_heads, kvb.head_dim, kvb.n_seqs = L, HK, D, n
    kvb.dtype, kvb.device = pk.PKH_KV_F16, 0
    kvb.layer_stride = HK * slots * 2 * D
    kvb.slot0 = ctypes.cast(h_slot0, ctypes.POINTER(ctypes.c_int64))
    kvb.max_seq = ctypes.cast(h_max, ctypes.POINTER(ctypes.c_int))
    kvb.k, kvb.v = KV.data_ptr(), KV.data_ptr() + D * 2
    kvb.d_slot0 = d_slot0.data_ptr()
    kvb.stride_pos, kvb.stride_head = 2 * D, slots * 2 * D

    max_seq = max(ctx) + 1
    half = min(D // 2, 64)
    sin = np.zeros((max_seq, half), np.float32)
    cos = np.zeros((max_seq, half), np.float32)
    lib.pkh_rope_host_tables(D, cfg["theta"], 0, max_seq - 1, None, sin.ctypes.data,
                             cos.ctypes.data)
    rope = pk.Rope()
    pk.check(lib.pkh_rope_alloc(max_seq, half, ctypes.byref(rope)), "pkh_rope_alloc")
    pk.check(lib.pkh_rope_upload(ctypes.byref(rope), sin.ctypes.data, cos.ctypes.data,
                                 max_seq), "pkh_rope_upload")
    plan = ctypes.c_void_p()
    pk.check(lib.pkh_plan_create(ctypes.byref(kvb), (ctypes.c_int * n)(*ctx), H,
                                 ctypes.byref(plan)), "pkh_plan_create")
    kvp, rp = ctypes.byref(kvb), ctypes.byref(rope)
    call = lib.pkh_attn_decode_batch_async

    def step(stream):
        sp = ctypes.c_void_p(stream.cuda_stream)
        for layer in range(L):
            rc = call(kvp, rp, plan, layer, q[layer].data_ptr(), k[layer].data_ptr(),
                      v[layer].data_ptr(), ao[layer].data_ptr(), sp)
            if rc != 0:
                raise pk.PkhError(rc, "pkh_attn_decode_batch_async")

    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        step(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(torch.cuda.current_stream())
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    steps = max(1, args.steps // 2)
    log(f"bench: timing {steps} graph replays x {L} layers")
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record(stream)
        graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    durs = np.array([e0.elapsed_time(e1) for e0, e1 in evs]) * 1e-3 / L
    bpl = sum(decode_bytes(c, H, HK, D, 2) for c in ctx)
    value = bpl * steps * L / wall / 1e9
    avg_launch = float(durs.mean())
    achieved = bpl / avg_launch / 1e9

    threads = min(16, os.cpu_count() or 1)
    log(f"bench: ragged parity + CPU baseline (oracle AVX-512 build, {threads} threads, layer 0)")
    from oracle import pyoracle as po
    prev = po.use_build("avx512")
    try:
        t_cpu, ref = cpu_baseline_ragged(KV, ctx, slot0, q, k, v, cfg, threads)
    finally:
        po.use_build(prev)
    err = float(np.max(np.abs(ao[0].cpu().numpy() - ref)))
    log(f"bench: ragged max-abs err vs oracle: {err:.3e}")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = {"value": round(bpl / t_cpu / 1e9, 3), "unit": "GB/s", "cores": threads,
               "kind": "port",
               "build": ("oracle/pk_oracle.c at -O3 -march=x86-64-v4 -mprefer-vector-width=512, "
                         "bit-identical to the -O2 oracle (the reference has no fp16 cache and "
                         "no batch API, so there is no reference build to time)"),
               "sample": (f"one layer of the same step: the oracle's fp16-KV decode step "
                          f"looped over the {n} sequences"),
               "us_per_layer_step": round(t_cpu * 1e6, 1),
               "cpu_model": cpu_model()}
    lib.pkh_plan_free(plan)
    lib.pkh_rope_free(rp)
    return {
        "metric": RAGGED_METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV, f32 arithmetic",
        "data": "synthetic: N(0,1) from torch's CUDA generator, seeded per workload",
        "config": {"workload": name, "n_heads": H, "n_kv_heads": HK, "head_dim": D,
                   "n_seqs": n, "contexts": ctx, "layers": L, "kv_dtype": cfg["kv"],
                   "rope_theta": cfg["theta"]},
        "us_per_layer_step": round(wall / (steps * L) * 1e6, 3),
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "bytes_per_layer_step": bpl,
        "max_abs_err_vs_oracle": err,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(name),
                     "us_per_launch": round(avg_launch * 1e6, 3)},
        "cpu_baseline": cpu,
    }


def run_copy_calibration(args):
    """A plain device copy of known size, for scaling the PMC byte counters."""
    import torch
    n = 256 << 20   # 1 GiB of fp32
    a = torch.randn(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(args.warmup + args.steps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4,
                      "launches": args.warmup + args.steps}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="llama3-8b-decode-ctx8192",
                    choices=sorted(WORKLOADS) + sorted(PREFILL_WORKLOADS) + sorted(RAGGED_WORKLOADS)
                    + ["copy-calibration"])
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the prefill, chunked-prefill and ragged measurements appended to "
                         "the decode line")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=32,
                    help="layers in the CPU-baseline sample")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the library has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "copy-calibration":
        run_copy_calibration(args)
        return
    if args.workload in PREFILL_WORKLOADS:
        res = run_prefill(args, PREFILL_WORKLOADS[args.workload], args.workload)
    elif args.workload in RAGGED_WORKLOADS:
        res = run_ragged(args, RAGGED_WORKLOADS[args.workload], args.workload)
    else:
        res = run_decode(args, WORKLOADS[args.workload])
        if not args.no_secondary and args.workload == "llama3-8b-decode-ctx8192":
            import torch
            keep = ("metric", "value", "unit", "pct_mfma_peak", "pct_hbm_peak", "us_per_layer",
                    "us_per_layer_step", "max_abs_err_vs_oracle", "roofline", "cpu_baseline",
                    "config", "dtype")
            res["secondary"] = {}
            for name, fn, table in (("llama3-8b-prefill-2048", run_prefill, PREFILL_WORKLOADS),
                                    ("llama3-8b-prefill-chunk128-ctx8192", run_prefill, PREFILL_WORKLOADS),
                                    ("llama3-8b-ragged16-fp16", run_ragged, RAGGED_WORKLOADS)):
                torch.cuda.empty_cache()
                sec = fn(args, table[name], name)
                res["secondary"][name] = {k: sec[k] for k in keep if k in sec}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
