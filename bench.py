#!/usr/bin/env python3
"""Benchmark of the fused per-layer kernel set on one MI355X.

One step = one pass of the memory-bound kernels of a decoder layer at
Mistral-7B prefill shapes (T=4096, hidden 4096, intermediate 14336, Q 32x128,
K 8x128, theta 1e6, fp16), in the order of the reference's fused fp16 layer
(gpu/engine/layer.cu:958-1059): RMSNorm, RoPE Q, RoPE K, residual add +
RMSNorm, SwiGLU, residual add. Inputs are synthetic (numpy PCG64 seed 0) and
resident in HBM before timing. Buffers rotate over several sets whose total
exceeds the 256 MB Infinity Cache, so every kernel reads its inputs from HBM.

Printed JSON line: value = layer algorithmic bytes / wall time per step
(GB/s); us_per_layer = sum of the six kernels' event-timed durations;
per-kernel GB/s and %-of-8 TB/s; extra kernels (gather per forward, fused
RMSNorm+int8, int8 dequant, decode T=64 layer); roofline of the dominant
kernel (SwiGLU); and the CPU oracle timed on the host cores on a bounded
token sample of the same layer.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-extra]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from neurogrid_amd import _lib  # noqa: E402
from neurogrid_amd import workloads as W  # noqa: E402
from neurogrid_amd.device import DeviceBuffer as DB  # noqa: E402

PEAK_GBPS = 8000.0  # MI355X HBM3E, AMD published
METRIC = "fused-kernel HBM GB/s (% of peak) + µs/layer at Mistral-7B shapes"
ROTATE_BYTES = 1536 << 20  # rotating working set, > 6x the 256 MB MALL


class Hip:
    """The few HIP runtime calls the benchmark needs (events and a stream)."""

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")
        self.h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipEventSynchronize.argtypes = [C.c_void_p]
        self.h.hipEventDestroy.argtypes = [C.c_void_p]

    def check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def stream(self):
        s = C.c_void_p()
        self.check(self.h.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s

    def events(self, n):
        out = []
        for _ in range(n):
            e = C.c_void_p()
            self.check(self.h.hipEventCreate(C.byref(e)), "hipEventCreate")
            out.append(e)
        return out

    def record(self, ev, stream):
        self.check(self.h.hipEventRecord(ev, stream), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.check(self.h.hipEventSynchronize(b), "hipEventSynchronize")
        ms = C.c_float()
        self.check(self.h.hipEventElapsedTime(C.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def sync(self):
        self.check(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------------------------- layer kernel set

class LayerSet:
    """Device buffers of one rotating set for one decoder layer's kernels."""

    def __init__(self, d, cfg, shared):
        self.x = DB.from_array(d["x"])               # rmsnorm input
        self.normed = DB(d["x"].nbytes)              # rmsnorm output
        self.q = DB.from_array(d["q"])               # rope q (in place, as the engine calls it)
        self.k = DB.from_array(d["k"])               # rope k (in place)
        self.attn = DB.from_array(d["x"])            # o-proj output -> add+rmsnorm input
        self.res = DB.from_array(d["residual"])      # residual in
        self.res_out = DB(d["x"].nbytes)             # residual out
        self.h2 = DB(d["x"].nbytes)                  # add+rmsnorm normed out
        self.gate = DB.from_array(d["gate"])
        self.up = DB.from_array(d["up"])
        self.act = DB(d["gate"].nbytes)              # swiglu out
        self.down = DB.from_array(d["x"])            # down-proj output -> final add
        self.out = DB(d["x"].nbytes)
        self.shared = shared

    @staticmethod
    def nbytes(cfg):
        T, H, I, e = cfg.T, cfg.H, cfg.I, cfg.e
        return e * (T * H * 9 + T * I * 3 + T * (cfg.nq + cfg.nkv) * cfg.D)


def layer_launches(L, cfg, s):
    """The six kernels of one step as (name, thunk) pairs."""
    T, H, I, D = cfg.T, cfg.H, cfg.I, cfg.D
    sh = s.shared
    eps, theta = C.c_float(cfg.eps), C.c_float(cfg.theta)
    bf = cfg.dtype == "bf16"
    rms = L.cuda_bf16_rmsnorm if bf else L.cuda_rmsnorm
    rope = L.cuda_bf16_rope_with_theta if bf else L.cuda_rope_with_theta
    addn = L.ng_bf16_add_rmsnorm if bf else L.cuda_add_rmsnorm
    swig = L.ng_bf16_silu_mul if bf else L.cuda_silu_mul
    add = L.cuda_bf16_add if bf else L.cuda_add
    return [
        ("rmsnorm", lambda: rms(s.normed.vp, s.x.vp, sh["w_attn"].vp, T, H, eps)),
        ("rope_q", lambda: rope(s.q.vp, s.q.vp, sh["pos"].ip, 1, T, cfg.nq, D, 0, theta)),
        ("rope_k", lambda: rope(s.k.vp, s.k.vp, sh["pos"].ip, 1, T, cfg.nkv, D, 0, theta)),
        ("add_rmsnorm", lambda: addn(s.h2.vp, s.res_out.vp, s.attn.vp, s.res.vp, sh["w_ffn"].vp, T, H, eps)),
        ("silu_mul", lambda: swig(s.act.vp, s.gate.vp, s.up.vp, T * I)),
        ("add", lambda: add(s.out.vp, s.down.vp, s.res_out.vp, T * H)),
    ]


def run_layer(L, hip, stream, cfg, steps, warmup, nsets=None):
    """Time `steps` layer steps (after `warmup`) with per-kernel events on the launch stream."""
    d = W.make_layer_inputs(cfg, seed=0, with_table=False)
    shared = {"w_attn": DB.from_array(d["w_attn"]), "w_ffn": DB.from_array(d["w_ffn"]),
              "pos": DB.from_array(d["pos"])}
    if nsets is None:
        nsets = max(2, -(-ROTATE_BYTES // LayerSet.nbytes(cfg)))
    sets = [LayerSet(d, cfg, shared) for _ in range(nsets)]
    del d
    launches = [layer_launches(L, cfg, s) for s in sets]
    names = [n for n, _ in launches[0]]
    nk = len(names)
    evs = hip.events((nk + 1) * steps)

    def step(i, timed):
        for j, (name, fn) in enumerate(launches[i % nsets]):
            if timed:
                hip.record(evs[(i - warmup) * (nk + 1) + j], stream)
            rc = fn()
            if rc != 0:
                raise RuntimeError(f"{name} returned {rc}")
        if timed:
            hip.record(evs[(i - warmup) * (nk + 1) + nk], stream)

    for i in range(warmup):
        step(i, False)
    hip.sync()
    t0 = time.perf_counter()
    for i in range(warmup, warmup + steps):
        step(i, True)
    hip.sync()
    wall = time.perf_counter() - t0
    per = {n: [] for n in names}
    for s_ in range(steps):
        base = s_ * (nk + 1)
        for j, n in enumerate(names):
            per[n].append(hip.elapsed_ms(evs[base + j], evs[base + j + 1]) * 1e3)
    for e in evs:
        hip.h.hipEventDestroy(e)
    for s in sets:
        for b in vars(s).values():
            if isinstance(b, DB):
                b.free()
    return wall, per, nsets


# ----------------------------------------------------------------------------- other kernels

def time_kernel(hip, stream, fns, reps, warmup=3):
    """Average event time (us) of fns[i % len(fns)]() over reps launches."""
    for i in range(warmup):
        fns[i % len(fns)]()
    evs = hip.events(2 * reps)
    for i in range(reps):
        hip.record(evs[2 * i], stream)
        rc = fns[i % len(fns)]()
        if rc != 0:
            raise RuntimeError(f"kernel returned {rc}")
        hip.record(evs[2 * i + 1], stream)
    ts = [hip.elapsed_ms(evs[2 * i], evs[2 * i + 1]) * 1e3 for i in range(reps)]
    for e in evs:
        hip.h.hipEventDestroy(e)
    return float(np.mean(ts)), float(np.median(ts))


def extra_kernels(L, hip, stream, reps):
    out = {}
    # embedding gather at Mistral-7B prefill (per forward pass)
    cfg = W.CONFIGS["mistral7b_prefill"]
    rng = np.random.Generator(np.random.PCG64(0))
    table = W.round_to(rng.standard_normal((cfg.vocab, cfg.H), dtype=np.float32) * np.float32(0.02), "f16")
    tb = DB.from_array(table)
    del table
    nb = 4
    ids = [DB.from_array(rng.integers(0, cfg.vocab, cfg.T).astype(np.int32)) for _ in range(nb)]
    outs = [DB(2 * cfg.T * cfg.H) for _ in range(nb)]
    fns = [lambda i=i: L.cuda_gather_embeddings(outs[i].vp, tb.vp, ids[i].ip, cfg.H, cfg.T) for i in range(nb)]
    us, med = time_kernel(hip, stream, fns, reps)
    b = W.layer_bytes(cfg)["gather"]
    out["gather_mistral7b_prefill"] = {"us": us, "GBps": b / us / 1e3, "bytes": b,
                                       "note": "table 262 MB stays partly cache-resident; rows random"}
    for x in ids + outs + [tb]:
        x.free()

    # fused RMSNorm + per-token int8, and int8 weight dequant (quant config)
    q = W.make_quant_inputs(seed=0)
    qb = W.quant_bytes()
    nb = 8
    xs = [DB.from_array(q["x"]) for _ in range(nb)]
    wb = DB.from_array(q["w"])
    codes = [DB(q["x"].size) for _ in range(nb)]
    scl = [DB(4 * W.QUANT_T) for _ in range(nb)]
    fns = [lambda i=i: L.ng_rmsnorm_quant_int8(codes[i].vp, scl[i].vp, xs[i].vp, wb.vp, W.QUANT_T, W.QUANT_H,
                                               C.c_float(1e-5)) for i in range(nb)]
    us, _ = time_kernel(hip, stream, fns, reps)
    out["rmsnorm_quant_int8"] = {"us": us, "GBps": qb["rmsnorm_quant"] / us / 1e3, "bytes": qb["rmsnorm_quant"]}
    for x in xs + codes + scl:
        x.free()
    nb = 3
    wq = [DB.from_array(q["wq"]) for _ in range(nb)]
    ws = DB.from_array(q["wscale"])
    wo = [DB(2 * q["wq"].size) for _ in range(nb)]
    fns = [lambda i=i: L.cuda_dequantize_weights(wo[i].vp, wq[i].vp, ws.vp, W.QUANT_WN, W.QUANT_WK, 1)
           for i in range(nb)]
    us, _ = time_kernel(hip, stream, fns, reps)
    out["dequant_int8_weights"] = {"us": us, "GBps": qb["dequant"] / us / 1e3, "bytes": qb["dequant"]}
    for x in wq + wo:
        x.free()
    return out


# ----------------------------------------------------------------------------- CPU baseline

def cpu_baseline(cfg, budget_s=10.0):
    """The CPU oracle (a C restatement of the reference semantics) running the
    same layer kernel set on a token sample, all host cores, OpenMP."""
    from oracle import oracle as O

    sample_T = 256
    sub = W.LayerConfig(**{**cfg.__dict__, "T": sample_T, "key": cfg.key + "_cpu_sample"})
    d = W.make_layer_inputs(sub, seed=0, with_table=False)
    nbytes = sum(W.layer_bytes(sub)[k] for k in W.LAYER_KERNELS)
    cores = os.cpu_count() or 1
    O.set_threads(cores)

    def one():
        O.rmsnorm(d["x"], d["w_attn"], sub.eps, sub.dtype)
        O.rope(d["q"], d["pos"], 0, sub.theta, sub.dtype)
        O.rope(d["k"], d["pos"], 0, sub.theta, sub.dtype)
        O.add_rmsnorm(d["x"], d["residual"], d["w_ffn"], sub.eps, sub.dtype)
        O.elementwise("silu_mul", d["gate"], d["up"], dtype=sub.dtype)
        O.elementwise("add", d["x"], d["residual"], dtype=sub.dtype)

    one()
    ts = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(ts) < 3:
        t = time.perf_counter()
        one()
        ts.append(time.perf_counter() - t)
    med = float(np.median(ts))
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "us_per_layer_sample": med * 1e6,
            "sample": f"{cfg.key} layer kernel set on T={sample_T} tokens (of {cfg.T}), median of {len(ts)} "
                      f"reps in {budget_s:.0f} s, OpenMP over {cores} host threads"}


# ----------------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="mistral7b_prefill")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: every kernel shards over tokens with no exchange, "
                                   "so N>1 is N independent copies of the N=1 run; run with --gpus 1"}))
        sys.exit(2)

    L = _lib.load()
    if L.cuda_init(0) != 0:
        raise RuntimeError("cuda_init(0) failed")
    hip = Hip()
    stream = hip.stream()
    L.ng_set_stream(stream)

    cfg = W.CONFIGS[args.config]
    log(f"layer {cfg.key}: {args.warmup} warmup + {args.steps} timed steps")
    wall, per, nsets = run_layer(L, hip, stream, cfg, args.steps, args.warmup)
    lb = W.layer_bytes(cfg)
    layer_bytes = sum(lb[k] for k in W.LAYER_KERNELS)
    ms_per_step = wall / args.steps * 1e3
    kernels = {}
    for k in W.LAYER_KERNELS:
        us = float(np.mean(per[k]))
        kernels[k] = {"us": us, "us_median": float(np.median(per[k])), "GBps": lb[k] / us / 1e3,
                      "frac": lb[k] / us / 1e3 / PEAK_GBPS, "bytes": lb[k]}
    us_layer = sum(kernels[k]["us"] for k in W.LAYER_KERNELS)
    log(f"layer done: {us_layer:.1f} us kernel time, {ms_per_step * 1e3:.1f} us wall per step")

    extra = {}
    if not args.no_extra:
        for key in ("mistral7b_decode", "llama2_13b_prefill", "mistral_nemo_bf16"):
            log(f"layer {key}")
            c2 = W.CONFIGS[key]
            _, p2, _ = run_layer(L, hip, stream, c2, 10, 3)
            lb2 = W.layer_bytes(c2)
            k2 = {k: float(np.mean(p2[k])) for k in W.LAYER_KERNELS}
            extra[key] = {"us_per_layer": sum(k2.values()),
                          "GBps": sum(lb2[k] for k in W.LAYER_KERNELS) / sum(k2.values()) / 1e3,
                          "per_kernel_us": k2}
        log("gather / rmsnorm+int8 / dequant")
        extra.update(extra_kernels(L, hip, stream, 30))

    dom = "silu_mul"
    roof = {"kernel": "cuda_silu_mul (ew_vec_kernel<f16, SILU_MUL>)", "bound": "hbm",
            "achieved": kernels[dom]["GBps"], "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": kernels[dom]["GBps"] / PEAK_GBPS, "traffic": None,
            "algorithmic_bytes_per_launch": lb[dom], "avg_launch_us": kernels[dom]["us"]}

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(cfg, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": layer_bytes / (ms_per_step * 1e-3) / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic: numpy PCG64 seed 0, N(0,1) activations, N(0,4) residual, N(1,0.02) weights",
        "config": {"workload": f"{cfg.model} prefill decoder-layer kernel set (rmsnorm, rope_q, rope_k, "
                               f"add_rmsnorm, silu_mul, add)", "T": cfg.T, "hidden": cfg.H,
                   "intermediate": cfg.I, "q_heads": cfg.nq, "kv_heads": cfg.nkv, "head_dim": cfg.D,
                   "rope_theta": cfg.theta, "eps": cfg.eps, "rotating_sets": nsets},
        "us_per_layer": us_layer,
        "pct_of_peak": layer_bytes / us_layer / 1e3 / PEAK_GBPS * 100,
        "layer_bytes": layer_bytes,
        "per_kernel": kernels,
        "extra": extra,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
