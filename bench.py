#!/usr/bin/env python3
"""Benchmark of the fused per-layer kernel set on one MI355X.

One step = one pass of the memory-bound kernels of a decoder layer at
Mistral-7B prefill shapes (T=4096, hidden 4096, intermediate 14336, Q 32x128,
K 8x128, theta 1e6, fp16), in the order of the reference's fused fp16 layer
(gpu/engine/layer.cu:958-1059): RMSNorm, RoPE Q, RoPE K, residual add +
RMSNorm, SwiGLU, residual add. Inputs are synthetic (numpy PCG64 seed 0) and
resident in HBM before timing. Buffers rotate over several sets whose total
exceeds the 256 MB Infinity Cache, so every kernel reads its inputs from HBM.

Launches go through the library's C ABI on the stream set with
ng_set_stream. The host side is Python (ctypes), which issues launches more
slowly than a short kernel runs, so every timed sequence is captured once
into a HIP graph and replayed: the GPU then never waits for the host.
  * step time: one graph holding exactly K layer steps (6 K launches, the
    steps cycling over the rotating sets), replayed once between two HIP
    events on the launch stream, after a W-step warm-up graph;
  * per-kernel time: one graph per kernel holding R back-to-back launches of
    that kernel over the rotating sets; the event time of a replay / R is the
    kernel's average launch duration (it includes the short dispatch gap
    between consecutive graph nodes, so it is a slight over-estimate).

Printed JSON line: value = layer algorithmic bytes / step time (GB/s);
us_per_layer = sum of the six kernels' average durations; per-kernel GB/s
and fraction of 8 TB/s; extra layer configurations (decode T=64, Llama-2-13B,
Mistral-Nemo bf16) and kernels (gather per forward, fused RMSNorm+int8, int8
dequant, QK LayerNorm + RoPE, cuda_gemm_int8 at Mistral-7B's INT8 projections);
the layer with this library's fused entry points; the roofline of the dominant
kernel (SwiGLU); and the CPU oracle timed on the host cores on a bounded token
sample of the same layer.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--no-cpu] [--no-extra]
       python bench.py --profile-pass  (eager launches of every kernel for rocprofv3: the kernel trace and
                                        the --pmc FETCH_SIZE / WRITE_SIZE runs)
       python bench.py --gemm-only  (cuda_gemm_int8 timings only)
       python bench.py --decode-only  (the INT8 layer's fused decode entry points and the decode layer only)
       python bench.py --profile-decode  (eager launches of the decode steps, fused and unfused, for rocprofv3)
       python bench.py --floors-only  (the access-pattern floor kernels only)
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import statistics
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
ROTATE_BYTES = 1536 << 20  # layer-step rotation: > 6x the 256 MB Infinity Cache
POOL_BYTES = 1 << 30       # per-kernel pools: bytes touched between reuses of a buffer
TRAFFIC_FILE = ROOT / "profiles" / "memory_bound_kernels_hbm_traffic.json"


class Hip:
    """The HIP runtime calls the benchmark needs: a stream, events, graphs."""

    CAPTURE_RELAXED = 2

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")
        vp = C.c_void_p
        self.h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        self.h.hipEventRecord.argtypes = [vp, vp]
        self.h.hipEventSynchronize.argtypes = [vp]
        self.h.hipEventDestroy.argtypes = [vp]
        self.h.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        self.h.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        self.h.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
        self.h.hipGraphLaunch.argtypes = [vp, vp]
        self.h.hipGraphExecDestroy.argtypes = [vp]
        self.h.hipGraphDestroy.argtypes = [vp]
        self.h.hipMemcpyAsync.argtypes = [vp, vp, C.c_size_t, C.c_int, vp]
        self.h.hipStreamSynchronize.argtypes = [vp]

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

    def capture(self, stream, thunks):
        """Capture the launches made by `thunks` on `stream` into an executable graph."""
        self.check(self.h.hipStreamBeginCapture(stream, self.CAPTURE_RELAXED), "hipStreamBeginCapture")
        try:
            for name, fn in thunks:
                rc = fn()
                if rc != 0:
                    raise RuntimeError(f"{name} returned {rc} during capture")
        finally:
            g = C.c_void_p()
            rc_end = self.h.hipStreamEndCapture(stream, C.byref(g))
        self.check(rc_end, "hipStreamEndCapture")
        ex = C.c_void_p()
        self.check(self.h.hipGraphInstantiate(C.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return Graph(self, g, ex)


class Graph:
    def __init__(self, hip, g, ex):
        self.hip, self.g, self.ex = hip, g, ex

    def launch(self, stream):
        self.hip.check(self.hip.h.hipGraphLaunch(self.ex, stream), "hipGraphLaunch")

    def destroy(self):
        if self.ex is not None:
            self.hip.h.hipGraphExecDestroy(self.ex)
            self.hip.h.hipGraphDestroy(self.g)
            self.ex = None


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

    def free(self):
        for b in vars(self).values():
            if isinstance(b, DB):
                b.free()


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


def fused_launches(L, cfg, s):
    """A layer in steady state with this library's fused entry points, four
    launches: the residual add that ends the previous layer fused into this
    layer's RMSNorm (cuda_add_rmsnorm), Q and K rotated in one launch
    (ng_rope_qk_with_theta), add+RMSNorm, SwiGLU. Needs call-site changes in
    the engine (layer.cu:986-1057), so it is reported beside the headline."""
    T, H, I, D = cfg.T, cfg.H, cfg.I, cfg.D
    sh = s.shared
    eps, theta = C.c_float(cfg.eps), C.c_float(cfg.theta)
    bf = cfg.dtype == "bf16"
    addn = L.ng_bf16_add_rmsnorm if bf else L.cuda_add_rmsnorm
    rope_qk = L.ng_bf16_rope_qk_with_theta if bf else L.ng_rope_qk_with_theta
    swig = L.ng_bf16_silu_mul if bf else L.cuda_silu_mul
    return [
        ("add_rmsnorm_in", lambda: addn(s.normed.vp, s.res_out.vp, s.down.vp, s.res.vp, sh["w_attn"].vp, T, H, eps)),
        ("rope_qk", lambda: rope_qk(s.q.vp, s.q.vp, s.k.vp, s.k.vp, sh["pos"].ip, 1, T, cfg.nq, cfg.nkv, D, 0, theta)),
        ("add_rmsnorm", lambda: addn(s.h2.vp, s.out.vp, s.attn.vp, s.res_out.vp, sh["w_ffn"].vp, T, H, eps)),
        ("silu_mul", lambda: swig(s.act.vp, s.gate.vp, s.up.vp, T * I)),
    ]


def fused_bytes(cfg):
    lb = W.layer_bytes(cfg)
    return 2 * lb["add_rmsnorm"] + lb["rope_q"] + lb["rope_k"] - 4 * cfg.T + lb["silu_mul"]


def engine_bf16_launches(L, cfg, s, hip, stream):
    """The bf16 engine's own memory-bound sequence, unfused
    (gpu/engine/layer.cu:1497-1615): copy residual <- input, RMSNorm, RoPE Q,
    RoPE K, add, copy residual <- sum, RMSNorm in place, SiLU in place, mul in
    place, residual add. The copies are device-to-device hipMemcpyAsync on the
    launch stream, as the engine's cudaMemcpyAsync calls are."""
    T, H, I, D = cfg.T, cfg.H, cfg.I, cfg.D
    sh = s.shared
    eps, theta = C.c_float(cfg.eps), C.c_float(cfg.theta)
    nb = T * H * 2

    def copy(dst, src):
        return hip.h.hipMemcpyAsync(dst.vp, src.vp, nb, 3, stream)

    return [
        ("copy_residual", lambda: copy(s.res, s.x)),
        ("rmsnorm", lambda: L.cuda_bf16_rmsnorm(s.normed.vp, s.x.vp, sh["w_attn"].vp, T, H, eps)),
        ("rope_q", lambda: L.cuda_bf16_rope_with_theta(s.q.vp, s.q.vp, sh["pos"].ip, 1, T, cfg.nq, D, 0, theta)),
        ("rope_k", lambda: L.cuda_bf16_rope_with_theta(s.k.vp, s.k.vp, sh["pos"].ip, 1, T, cfg.nkv, D, 0, theta)),
        ("add", lambda: L.cuda_bf16_add(s.attn.vp, s.attn.vp, s.res.vp, T * H)),
        ("copy_residual2", lambda: copy(s.res_out, s.attn)),
        ("rmsnorm2", lambda: L.cuda_bf16_rmsnorm(s.attn.vp, s.attn.vp, sh["w_ffn"].vp, T, H, eps)),
        ("silu", lambda: L.cuda_bf16_silu(s.gate.vp, s.gate.vp, T * I)),
        ("mul", lambda: L.cuda_bf16_mul(s.gate.vp, s.gate.vp, s.up.vp, T * I)),
        ("add_out", lambda: L.cuda_bf16_add(s.out.vp, s.down.vp, s.res_out.vp, T * H)),
    ]


def engine_int8_launches(L, cfg, s, hip, stream):
    """The fp16 INT8 engine layer's own memory-bound sequence, unfused
    (gpu/engine/layer.cu:458-598, cuda_layer_forward): copy residual <- input,
    RMSNorm, RoPE Q and K in place, add in place (o-proj output + residual),
    copy residual <- sum, RMSNorm in place, SiLU in place, mul in place,
    residual add. The copies are device-to-device hipMemcpyAsync on the launch
    stream, as the engine's cudaMemcpy calls are (stream-ordered here)."""
    T, H, I, D = cfg.T, cfg.H, cfg.I, cfg.D
    sh = s.shared
    eps, theta = C.c_float(cfg.eps), C.c_float(cfg.theta)
    nb = T * H * 2

    def copy(dst, src):
        return hip.h.hipMemcpyAsync(dst.vp, src.vp, nb, 3, stream)

    return [
        ("copy_residual", lambda: copy(s.res, s.x)),
        ("rmsnorm", lambda: L.cuda_rmsnorm(s.normed.vp, s.x.vp, sh["w_attn"].vp, T, H, eps)),
        ("rope_q", lambda: L.cuda_rope_with_theta(s.q.vp, s.q.vp, sh["pos"].ip, 1, T, cfg.nq, D, 0, theta)),
        ("rope_k", lambda: L.cuda_rope_with_theta(s.k.vp, s.k.vp, sh["pos"].ip, 1, T, cfg.nkv, D, 0, theta)),
        ("add", lambda: L.cuda_add(s.attn.vp, s.attn.vp, s.res.vp, T * H)),
        ("copy_residual2", lambda: copy(s.res_out, s.attn)),
        ("rmsnorm2", lambda: L.cuda_rmsnorm(s.attn.vp, s.attn.vp, sh["w_ffn"].vp, T, H, eps)),
        ("silu", lambda: L.cuda_silu(s.gate.vp, s.gate.vp, T * I)),
        ("mul", lambda: L.cuda_mul(s.gate.vp, s.gate.vp, s.up.vp, T * I)),
        ("add_out", lambda: L.cuda_add(s.out.vp, s.down.vp, s.res_out.vp, T * H)),
    ]


def engine_int8_fused_launches(L, cfg, s):
    """The same layer with the call-site change for the INT8 layer: the first
    copy dropped (the layer input is the residual), add + copy + RMSNorm as one
    cuda_add_rmsnorm writing the residual and the normed sum (normed in place
    over the o-proj output), SiLU + mul as one cuda_silu_mul in place; six
    launches."""
    T, H, I, D = cfg.T, cfg.H, cfg.I, cfg.D
    sh = s.shared
    eps, theta = C.c_float(cfg.eps), C.c_float(cfg.theta)
    return [
        ("rmsnorm", lambda: L.cuda_rmsnorm(s.normed.vp, s.x.vp, sh["w_attn"].vp, T, H, eps)),
        ("rope_q", lambda: L.cuda_rope_with_theta(s.q.vp, s.q.vp, sh["pos"].ip, 1, T, cfg.nq, D, 0, theta)),
        ("rope_k", lambda: L.cuda_rope_with_theta(s.k.vp, s.k.vp, sh["pos"].ip, 1, T, cfg.nkv, D, 0, theta)),
        ("add_rmsnorm", lambda: L.cuda_add_rmsnorm(s.attn.vp, s.res_out.vp, s.attn.vp, s.x.vp, sh["w_ffn"].vp, T, H,
                                                   eps)),
        ("silu_mul", lambda: L.cuda_silu_mul(s.gate.vp, s.gate.vp, s.up.vp, T * I)),
        ("add_out", lambda: L.cuda_add(s.out.vp, s.down.vp, s.res_out.vp, T * H)),
    ]


def engine_bf16_bytes(cfg):
    T, H, I, e = cfg.T, cfg.H, cfg.I, cfg.e
    lb = W.layer_bytes(cfg)
    return (2 * 2 * T * H * e + 2 * lb["rmsnorm"] + lb["rope_q"] + lb["rope_k"] + 2 * lb["add"]
            + 2 * T * I * e + 3 * T * I * e)


class Pool:
    """`n` copies of one buffer in one device allocation (slot j at offset
    j * slot bytes), all holding the same initial data, so that a kernel can be
    launched over many distinct buffers."""

    def __init__(self, hip, slot_bytes, n, init=None):
        self.slot = -(-int(slot_bytes) // 256) * 256
        self.n = n
        self.buf = DB(self.slot * n)
        if init is not None:
            self.buf.upload(init)
            for j in range(1, n):
                hip.check(hip.h.hipMemcpyAsync(self.at(j), self.at(0), int(slot_bytes), 3, None), "hipMemcpyAsync")
            hip.sync()

    def at(self, j):
        return self.buf.offset((j % self.n) * self.slot)

    def free(self):
        self.buf.free()


class GroupPool:
    """Pool slots that each hold several weight tensors one after another, as
    an engine allocates a layer's weights in sequence: member(p).at(j) is
    tensor p of slot j. One split-kernel launch over two such tensors (gate
    and up) runs up to 20% faster or slower with their distance in memory,
    and separate pools would leave that distance to the allocator."""

    class _Member:
        def __init__(self, group, p):
            self.group, self.p = group, p

        def at(self, j):
            return C.c_void_p(self.group.pool.at(j).value + self.group.offs[self.p])

        def free(self):
            pass

    def __init__(self, hip, arrays, n):
        self.offs, off = [], 0
        for a in arrays:
            self.offs.append(off)
            off += -(-a.nbytes // 256) * 256
        cat = np.zeros(off, np.uint8)
        for a, o in zip(arrays, self.offs):
            cat[o:o + a.nbytes] = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        self.pool = Pool(hip, off, n, cat)

    def member(self, p):
        return GroupPool._Member(self, p)

    def free(self):
        self.pool.free()


def pool_slots(footprint_bytes, min_slots=3, max_slots=64):
    """Slots so that at least POOL_BYTES of other buffers are touched between
    two launches on the same slot (the Infinity Cache is 256 MB)."""
    return int(min(max_slots, max(min_slots, -(-POOL_BYTES // int(footprint_bytes)) + 1)))


def kernel_pools_for(L, hip, cfg, d, shared):
    """Yield (name, make) per layer kernel; make() allocates that kernel's
    buffer pools and returns (thunks, pools), one thunk per pool slot."""
    T, H, I, D, e = cfg.T, cfg.H, cfg.I, cfg.D, cfg.e
    eps, theta = C.c_float(cfg.eps), C.c_float(cfg.theta)
    bf = cfg.dtype == "bf16"
    rms = L.cuda_bf16_rmsnorm if bf else L.cuda_rmsnorm
    rope = L.cuda_bf16_rope_with_theta if bf else L.cuda_rope_with_theta
    addn = L.ng_bf16_add_rmsnorm if bf else L.cuda_add_rmsnorm
    swig = L.ng_bf16_silu_mul if bf else L.cuda_silu_mul
    add = L.cuda_bf16_add if bf else L.cuda_add
    rope_qk = L.ng_bf16_rope_qk_with_theta if bf else L.ng_rope_qk_with_theta
    th = T * H * e
    tq, tk, ti = T * cfg.nq * D * e, T * cfg.nkv * D * e, T * I * e

    def mk(name, footprint, specs, launch):
        def make():
            n = pool_slots(footprint)
            pools = [Pool(hip, nbytes, n, init) for nbytes, init in specs]
            thunks = [(name, (lambda j=j: launch(*[p.at(j) for p in pools]))) for j in range(n)]
            return thunks, pools
        return name, make

    yield mk("rmsnorm", 2 * th, [(th, d["x"]), (th, None)],
             lambda x, y: rms(y, x, shared["w_attn"].vp, T, H, eps))
    yield mk("rope_q", tq, [(tq, d["q"])], lambda q: rope(q, q, shared["pos"].ip, 1, T, cfg.nq, D, 0, theta))
    yield mk("rope_k", tk, [(tk, d["k"])], lambda k: rope(k, k, shared["pos"].ip, 1, T, cfg.nkv, D, 0, theta))
    yield mk("add_rmsnorm", 4 * th, [(th, d["x"]), (th, d["residual"]), (th, None), (th, None)],
             lambda x, r, ro, y: addn(y, ro, x, r, shared["w_ffn"].vp, T, H, eps))
    yield mk("silu_mul", 3 * ti, [(ti, d["gate"]), (ti, d["up"]), (ti, None)],
             lambda g, u, o: swig(o, g, u, T * I))
    yield mk("add", 3 * th, [(th, d["x"]), (th, d["residual"]), (th, None)],
             lambda a, b, o: add(o, a, b, T * H))
    # not in the engine's sequence: Q and K in one launch (ng_rope_qk_with_theta)
    yield mk("rope_qk", tq + tk, [(tq, d["q"]), (tk, d["k"])],
             lambda q, k: rope_qk(q, q, k, k, shared["pos"].ip, 1, T, cfg.nq, cfg.nkv, D, 0, theta))


def time_graph(hip, stream, graphs, reps, warmup=2):
    """Average event time (ms) of one replay of graphs[i % len(graphs)] over reps replays."""
    for i in range(warmup):
        graphs[i % len(graphs)].launch(stream)
    hip.sync()
    e0, e1 = hip.events(2)
    hip.record(e0, stream)
    for i in range(reps):
        graphs[i % len(graphs)].launch(stream)
    hip.record(e1, stream)
    ms = hip.elapsed_ms(e0, e1)
    hip.h.hipEventDestroy(e0)
    hip.h.hipEventDestroy(e1)
    return ms / reps


def kernel_graph(hip, stream, thunks_per_set, launches):
    """A graph of `launches` back-to-back launches cycling over the rotating sets."""
    seq = [thunks_per_set[i % len(thunks_per_set)] for i in range(launches)]
    return hip.capture(stream, seq)


def run_layer(L, hip, stream, cfg, steps, warmup, kernel_launches=24, kernel_reps=4, nsets=None):
    """Step time over `steps` replays of the per-set layer graphs, and the
    average duration of each kernel from its own back-to-back graph."""
    d = W.make_layer_inputs(cfg, seed=0, with_table=False)
    shared = {"w_attn": DB.from_array(d["w_attn"]), "w_ffn": DB.from_array(d["w_ffn"]),
              "pos": DB.from_array(d["pos"])}
    if nsets is None:
        nsets = min(32, max(2, -(-ROTATE_BYTES // LayerSet.nbytes(cfg))))
    sets = [LayerSet(d, cfg, shared) for _ in range(nsets)]
    del d
    step_ms, wall_ms = time_steps(hip, stream, [layer_launches(L, cfg, s) for s in sets], steps, warmup)
    seq = {"fused_step_ms": time_steps(hip, stream, [fused_launches(L, cfg, s) for s in sets], steps, warmup)[0]}
    if cfg.dtype == "bf16":
        seq["engine_bf16_step_ms"] = time_steps(
            hip, stream, [engine_bf16_launches(L, cfg, s, hip, stream) for s in sets], steps, warmup)[0]
    else:
        seq["engine_int8_step_ms"] = time_steps(
            hip, stream, [engine_int8_launches(L, cfg, s, hip, stream) for s in sets], steps, warmup)[0]
        seq["engine_int8_fused_step_ms"] = time_steps(
            hip, stream, [engine_int8_fused_launches(L, cfg, s) for s in sets], steps, warmup)[0]

    for s in sets:
        s.free()

    # Per-kernel: each kernel over its own pool of buffers (see Pool).
    d = W.make_layer_inputs(cfg, seed=0, with_table=False)
    per, slots = {}, {}
    for name, make in kernel_pools_for(L, hip, cfg, d, shared):
        thunks, pools = make()
        for t_name, fn in thunks:
            if fn() != 0:
                raise RuntimeError(f"{t_name} failed")
        hip.sync()
        n = max(kernel_launches, len(thunks))
        g = kernel_graph(hip, stream, thunks, n)
        per[name] = time_graph(hip, stream, [g], kernel_reps, 1) * 1e3 / n
        slots[name] = len(thunks)
        g.destroy()
        for p in pools:
            p.free()
    eng = {}
    for name, make in engine_unfused_pools_for(L, hip, cfg, d, shared, stream):
        thunks, pools = make()
        eng[name] = time_pool_kernel(hip, stream, thunks, kernel_launches, kernel_reps)
        for p in pools:
            p.free()
    seq["engine_bf16_kernels_us" if cfg.dtype == "bf16" else "engine_int8_kernels_us"] = eng
    del d
    for b in shared.values():
        b.free()
    return step_ms, wall_ms, per, nsets, slots, seq


def copy_times(hip, stream, byte_counts, launches=24, reps=4):
    """Average duration (us) of a plain device-to-device hipMemcpyAsync that
    moves b bytes (reads b / 2, writes b / 2), for each b in byte_counts,
    timed as the kernels are: back-to-back in one graph over a pool of
    buffers. The HBM rate a streaming kernel of that size can reach."""
    out = {}
    for b in sorted(set(int(x) for x in byte_counts)):
        half = b // 2
        n = pool_slots(b)
        src, dst = Pool(hip, half, n), Pool(hip, half, n)
        thunks = [("copy", (lambda j=j: hip.h.hipMemcpyAsync(dst.at(j), src.at(j), half, 3, stream)))
                  for j in range(n)]
        out[b] = time_pool_kernel(hip, stream, thunks, launches, reps)
        src.free()
        dst.free()
    return out


def fused_layer_report(cfg, per, seq):
    """The four-launch steady state (fused_launches): its graph step time,
    and the sum of its kernels' per-kernel averages."""
    b = fused_bytes(cfg)
    us = seq["fused_step_ms"] * 1e3
    us_sum = 2 * per["add_rmsnorm"] + per["rope_qk"] + per["silu_mul"]
    return {"kernels": ["add_rmsnorm (residual add of the previous layer + RMSNorm)", "rope_qk", "add_rmsnorm",
                        "silu_mul"],
            "us_per_step": us, "us_per_layer": us_sum, "layer_bytes": b, "GBps": b / us / 1e3,
            "frac": b / us / 1e3 / PEAK_GBPS,
            "note": "us_per_step: graph replay of the four launches per step; us_per_layer: the sum of their "
                    "per-kernel averages; the engine's six-kernel sequence is the headline"}


def time_steps(hip, stream, launches, steps, warmup):
    """Step time of a sequence: one graph of `warmup` steps replayed once
    untimed, then one graph of exactly `steps` steps (cycling over the
    rotating sets' launch lists) replayed once between two events. An eager
    pass first makes argument errors surface outside any capture."""
    for lset in launches:
        for name, fn in lset:
            if fn() != 0:
                raise RuntimeError(f"{name} failed")
    hip.sync()
    n = len(launches)
    warm_graph = hip.capture(stream, [t for i in range(max(warmup, 1)) for t in launches[i % n]])
    timed_graph = hip.capture(stream, [t for i in range(warmup, warmup + steps) for t in launches[i % n]])
    warm_graph.launch(stream)
    hip.sync()
    t0 = time.perf_counter()
    step_ms = time_graph(hip, stream, [timed_graph], 1, 0) / steps
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    warm_graph.destroy()
    timed_graph.destroy()
    return step_ms, wall_ms


# ----------------------------------------------------------------------------- other kernels

def time_kernel(hip, stream, fns, launches=24, reps=4):
    """Average duration (us) of fns cycled back-to-back inside one graph."""
    for f in fns:
        if f() != 0:
            raise RuntimeError("kernel failed")
    hip.sync()
    g = kernel_graph(hip, stream, [("k", f) for f in fns], launches)
    us = time_graph(hip, stream, [g], reps, 1) * 1e3 / launches
    g.destroy()
    return us


def time_pool_kernel(hip, stream, thunks, launches=24, reps=4):
    """Average duration (us) of `thunks` (one per buffer slot) cycled back-to-back in one graph."""
    for _, f in thunks:
        if f() != 0:
            raise RuntimeError("kernel failed")
    hip.sync()
    n = max(launches, len(thunks))
    g = kernel_graph(hip, stream, thunks, n)
    us = time_graph(hip, stream, [g], reps, 1) * 1e3 / n
    g.destroy()
    return us


def time_rotating(hip, stream, variants, rounds=3, launches=24, timer=None):
    """Median duration (us) of each variant (what `timer` takes: by default
    time_pool_kernel's thunks, one per buffer slot), timed over `rounds` rounds
    with the order rotated each round: the first variant timed in a run comes
    out slower on this GPU, by up to 5-10% (15% for the prefill GEMMs)."""
    timer = timer or time_pool_kernel
    names = list(variants)
    times = {nm: [] for nm in names}
    for r in range(rounds):
        for nm in names[r % len(names):] + names[:r % len(names)]:
            times[nm].append(timer(hip, stream, variants[nm], launches=launches))
    return {nm: statistics.median(v) for nm, v in times.items()}


def extra_kernels(L, hip, stream):
    out = {}
    # Embedding gather at Mistral-7B prefill (per forward pass): 8 copies of
    # the [32000, 4096] fp16 table (262 MB each) and a distinct id vector per
    # launch, so rows come from HBM rather than the Infinity Cache.
    cfg = W.CONFIGS["mistral7b_prefill"]
    rng = np.random.Generator(np.random.PCG64(0))
    table = W.round_to(rng.standard_normal((cfg.vocab, cfg.H), dtype=np.float32) * np.float32(0.02), "f16")
    ntab, nids = 8, 24
    tabs = Pool(hip, table.nbytes, ntab, table)
    del table
    ids = Pool(hip, 4 * cfg.T, nids)
    assert ids.slot == 4 * cfg.T  # slots are contiguous, so one upload fills every slot
    ids.buf.upload(np.stack([rng.integers(0, cfg.vocab, cfg.T).astype(np.int32) for _ in range(nids)]))
    outs = Pool(hip, 2 * cfg.T * cfg.H, 8)
    ipt = lambda j: C.cast(ids.at(j), C.POINTER(C.c_int))
    thunks = [("gather", (lambda j=j: L.cuda_gather_embeddings(outs.at(j), tabs.at(j), ipt(j), cfg.H, cfg.T)))
              for j in range(nids)]
    us = time_pool_kernel(hip, stream, thunks)
    b = W.layer_bytes(cfg)["gather"]
    out["gather_mistral7b_prefill"] = {"us": us, "GBps": b / us / 1e3, "frac": b / us / 1e3 / PEAK_GBPS,
                                       "bytes": b, "buffer_sets": f"{ntab} tables, {nids} id vectors",
                                       "note": "table [32000,4096] fp16 (262 MB), uniform ids"}
    for p in (tabs, ids, outs):
        p.free()

    # Embedding gather at Mistral-Nemo (bf16, T = 2048): Zipf(1.1) ids over a
    # [131072, 5120] table (1.34 GB); 4 table copies and 24 id vectors, so a
    # launch finds no row of the previous one in the caches. Zipf ids repeat,
    # so the hot rows come from the caches within a launch: FETCH_SIZE (the
    # traffic summary) is below the algorithmic bytes.
    nm = W.CONFIGS["mistral_nemo_bf16"]
    rng = np.random.Generator(np.random.PCG64(1))
    ntab, nids = 4, 24
    tabs = Pool(hip, 2 * nm.vocab * nm.H, ntab)
    for r0 in range(0, nm.vocab, 16384):            # fill slot 0 in pieces, then copy it
        piece = W.round_to(rng.standard_normal((min(16384, nm.vocab - r0), nm.H), dtype=np.float32)
                           * np.float32(0.02), "bf16")
        hip.check(L.cuda_copy_int8_to_device(tabs.buf.offset(2 * r0 * nm.H), piece.ctypes.data, piece.nbytes),
                  "upload")
    del piece
    for j in range(1, ntab):
        hip.check(hip.h.hipMemcpyAsync(tabs.at(j), tabs.at(0), 2 * nm.vocab * nm.H, 3, None), "hipMemcpyAsync")
    hip.sync()
    ids = Pool(hip, 4 * nm.T, nids)
    assert ids.slot == 4 * nm.T
    zipf = np.stack([W.zipf_ids(rng, nm.T, nm.vocab, 1.1) for _ in range(nids)])
    ids.buf.upload(zipf)
    outs = Pool(hip, 2 * nm.T * nm.H, 8)
    thunks = [("gather_zipf", (lambda j=j: L.cuda_gather_embeddings(outs.at(j), tabs.at(j), ipt(j), nm.H, nm.T)))
              for j in range(nids)]
    us = time_pool_kernel(hip, stream, thunks)
    b = W.layer_bytes(nm)["gather"]
    distinct = float(np.mean([np.unique(z).size for z in zipf]))
    out["gather_mistral_nemo_bf16_zipf"] = {
        "us": us, "GBps": b / us / 1e3, "frac": b / us / 1e3 / PEAK_GBPS, "bytes": b,
        "buffer_sets": f"{ntab} tables, {nids} id vectors",
        "distinct_rows_per_launch": distinct,
        "note": "table [131072,5120] bf16 (1.34 GB), Zipf(1.1) ids; GBps counts every row read once per token "
                "(algorithmic bytes), though repeated ids are served from the caches"}
    for p in (tabs, ids, outs):
        p.free()

    # Fused RMSNorm + per-token int8, and int8 weight dequant (quant config).
    q = W.make_quant_inputs(seed=0)
    qb = W.quant_bytes()
    eps = C.c_float(1e-5)
    b = qb["rmsnorm_quant"]
    n = pool_slots(b)
    xs, codes, scl = Pool(hip, q["x"].nbytes, n, q["x"]), Pool(hip, q["x"].size, n), Pool(hip, 4 * W.QUANT_T, n)
    wb = DB.from_array(q["w"])
    thunks = [("rmsnorm_quant", (lambda j=j: L.ng_rmsnorm_quant_int8(codes.at(j), scl.at(j), xs.at(j), wb.vp,
                                                                     W.QUANT_T, W.QUANT_H, eps))) for j in range(n)]
    us = time_pool_kernel(hip, stream, thunks)
    out["rmsnorm_quant_int8"] = {"us": us, "GBps": b / us / 1e3, "frac": b / us / 1e3 / PEAK_GBPS, "bytes": b,
                                 "buffer_sets": n}
    # Per-token int8 alone (cuda_quantize_weights_per_row with the tokens as
    # rows), on the same activations.
    b = qb["quant_per_token"]
    thunks = [("quant_per_token", (lambda j=j: L.cuda_quantize_weights_per_row(codes.at(j), scl.at(j), xs.at(j),
                                                                               W.QUANT_T, W.QUANT_H)))
              for j in range(n)]
    us = time_pool_kernel(hip, stream, thunks)
    out["quantize_per_token_int8"] = {"us": us, "GBps": b / us / 1e3, "frac": b / us / 1e3 / PEAK_GBPS, "bytes": b,
                                      "buffer_sets": n}
    for p in (xs, codes, scl):
        p.free()
    wb.free()
    b = qb["dequant"]
    n = pool_slots(b)
    wq, wo = Pool(hip, q["wq"].nbytes, n, q["wq"]), Pool(hip, 2 * q["wq"].size, n)
    ws = DB.from_array(q["wscale"])
    thunks = [("dequant", (lambda j=j: L.cuda_dequantize_weights(wo.at(j), wq.at(j), ws.vp, W.QUANT_WN, W.QUANT_WK,
                                                                1))) for j in range(n)]
    us = time_pool_kernel(hip, stream, thunks)
    out["dequant_int8_weights"] = {"us": us, "GBps": b / us / 1e3, "frac": b / us / 1e3 / PEAK_GBPS, "bytes": b,
                                   "buffer_sets": n}
    for p in (wq, wo):
        p.free()
    ws.free()

    # QK LayerNorm + RoPE at Mistral-7B prefill shapes (not part of the Mistral
    # layer; the engine runs it for models with per-head norms, layer.cu:998-1018):
    # the fused entry point vs the four launches it replaces.
    d = W.make_layer_inputs(cfg, seed=0, with_table=False)
    T, D, nq, nkv = cfg.T, cfg.D, cfg.nq, cfg.nkv
    tq, tk = T * nq * D * 2, T * nkv * D * 2
    n = pool_slots(2 * (tq + tk))
    qp, kp = Pool(hip, tq, n, d["q"]), Pool(hip, tk, n, d["k"])
    wq, wk, pos = DB.from_array(d["w_attn"][:D]), DB.from_array(d["w_ffn"][:D]), DB.from_array(d["pos"])
    eps, th = C.c_float(1e-5), C.c_float(cfg.theta)
    fused = [("qkn_rope", (lambda j=j: L.ng_qk_rmsnorm_rope_with_theta(
        qp.at(j), qp.at(j), kp.at(j), kp.at(j), wq.vp, wk.vp, pos.ip, 1, T, nq, nkv, D, eps, 0, th)))
        for j in range(n)]
    us_f = time_pool_kernel(hip, stream, fused)

    def composed(j):
        for rc in (L.ng_per_head_rmsnorm(qp.at(j), qp.at(j), wq.vp, T, nq, D, eps),
                   L.ng_per_head_rmsnorm(kp.at(j), kp.at(j), wk.vp, T, nkv, D, eps),
                   L.cuda_rope_with_theta(qp.at(j), qp.at(j), pos.ip, 1, T, nq, D, 0, th),
                   L.cuda_rope_with_theta(kp.at(j), kp.at(j), pos.ip, 1, T, nkv, D, 0, th)):
            if rc != 0:
                return rc
        return 0

    us_c = time_pool_kernel(hip, stream, [("qkn_composed", (lambda j=j: composed(j))) for j in range(n)])
    b = 2 * (tq + tk) + 4 * T + 4 * D
    out["qk_rmsnorm_rope_mistral7b_prefill"] = {
        "us": us_f, "GBps": b / us_f / 1e3, "frac": b / us_f / 1e3 / PEAK_GBPS, "bytes": b,
        "composed_us": us_c, "note": "fused ng_qk_rmsnorm_rope_with_theta vs ng_per_head_rmsnorm x2 + "
                                             "cuda_rope_with_theta x2 (composed_us: the four launches)"}
    for p in (qp, kp):
        p.free()
    for x in (wq, wk, pos):
        x.free()
    out["gemm_int8"] = gemm_extras(L, hip, stream)
    out["gemm_int8_shared_a"] = sh = shared_a_extras(L, hip, stream)
    out["norm_gemm_int8_shared_a"] = norm_shared_extras(L, hip, stream)
    out["gemm_int8_silu_mul"] = silu_mul_gemm_extras(L, hip, stream)
    out["gemm_int8_silu_mul_llama2_7b"] = silu_mul_gemm_extras(L, hip, stream, N=11008)
    out["gemm_int8_add"] = gemm_add_extras(L, hip, stream)
    out["int8_decode_layer"] = int8_decode_layer_extras(L, hip, stream)
    g = out["gemm_int8"]
    g["mistral7b_layer_M1"]["shared_a_us"] = (sh["qkv_M1"]["us"] + g["q_proj_M1"]["us"] + sh["gate_up_M1"]["us"]
                                              + g["down_proj_M1"]["us"])
    g["mistral7b_layer_M1"]["shared_a_note"] = ("q/k/v in one ng_gemm_int8_shared_a call, o, gate/up in one call, "
                                                "down")
    return out


PREFILL_M = (512, 1024, 2048, 4096)
# The composition through hipBLASLt is timed only at the row counts where it
# has run clean on MI355X; at 1024 and 2048 rows a run over it (and over a
# blocked variant) ended in a GPU memory fault whose cause was not found.
COMPOSED_M = (512, 4096)


def gemm_extras(L, hip, stream):
    """cuda_gemm_int8 at the INT8 projections of one Mistral-7B layer
    (layer.cu:487-501,551,575: B int8 [N, K] with per-row scales), for M = 1
    and 64 tokens, against the reference's composition without its cudaMalloc /
    cudaFree (cuda_dequantize_weights into an fp16 buffer, then
    cuda_gemm_fp16). Weight pools keep the codes cache-cold. Also every
    projection at prefill sizes (PREFILL_M tokens): cuda_gemm_int8 (the fused
    prefill MFMA kernel below 4096 tokens, the composition through its own
    buffers from 4096 on), the fused kernel alone (ng_gemm_int8_noalloc, the
    same kernel without allocation) and the composition (at COMPOSED_M)."""
    rng = np.random.Generator(np.random.PCG64(0))
    H, I = 4096, 14336
    shapes = {"q_proj": (H, H), "k_proj": (H, 1024), "gate_proj": (H, I), "down_proj": (I, H)}
    per_layer = {"q_proj": 2, "k_proj": 2, "gate_proj": 2, "down_proj": 1}   # q+o, k+v, gate+up, down
    out, layer, prefill = {}, {1: [0.0, 0.0], 64: [0.0, 0.0]}, {}
    for name, (K, N) in shapes.items():
        wq = rng.integers(-128, 128, (N, K)).astype(np.int8)
        n = pool_slots(N * K)
        wp = Pool(hip, wq.nbytes, n, wq)
        del wq
        sc = DB.from_array(rng.uniform(1e-3, 1e-2, N).astype(np.float32))
        deq = DB(2 * N * K)
        for M in (1, 64):
            ab = DB.from_array(W.round_to(rng.standard_normal((M, K), dtype=np.float32), "f16"))
            cp = Pool(hip, 2 * M * N, n)
            th = [("gemm_int8", (lambda j=j: L.cuda_gemm_int8(cp.at(j), ab.vp, wp.at(j), sc.vp, M, K, N, True)))
                  for j in range(n)]
            us = time_pool_kernel(hip, stream, th)

            def comp(j, M=M, ab=ab, cp=cp):
                rc = L.cuda_dequantize_weights(deq.vp, wp.at(j), sc.vp, N, K, 1)
                return rc or L.cuda_gemm_fp16(cp.at(j), ab.vp, deq.vp, M, K, N, False, True)

            usc = time_pool_kernel(hip, stream, [("composed", (lambda j=j: comp(j))) for j in range(n)])
            b = N * K + 2 * M * K + 2 * M * N + 4 * N
            out[f"{name}_M{M}"] = {"us": us, "GBps": b / us / 1e3, "frac": b / us / 1e3 / PEAK_GBPS, "bytes": b,
                                   "composed_us": usc, "buffer_sets": n}
            layer[M][0] += per_layer[name] * us
            layer[M][1] += per_layer[name] * usc
            cp.free()
            ab.free()
        for M in PREFILL_M:
            ab = DB.from_array(W.round_to(rng.standard_normal((M, K), dtype=np.float32), "f16"))
            cb = DB(2 * M * N)
            # The same kernel below 4096 tokens: timed in rotated order.
            tr = time_rotating(hip, stream, {
                "gemm": [lambda: L.cuda_gemm_int8(cb.vp, ab.vp, wp.at(0), sc.vp, M, K, N, True)],
                "noalloc": [lambda: L.ng_gemm_int8_noalloc(cb.vp, ab.vp, wp.at(0), sc.vp, M, K, N, True)]},
                launches=8, timer=lambda *a, **k: time_kernel(*a, reps=2, **k))
            us, usf = tr["gemm"], tr["noalloc"]

            def comp(M=M, ab=ab, cb=cb):
                rc = L.cuda_dequantize_weights(deq.vp, wp.at(0), sc.vp, N, K, 1)
                return rc or L.cuda_gemm_fp16(cb.vp, ab.vp, deq.vp, M, K, N, False, True)

            usc = None
            if M in COMPOSED_M:
                try:
                    usc = time_kernel(hip, stream, [comp], launches=8, reps=2)
                except RuntimeError as e:   # hipBLASLt refuses some shapes (status 6 at K = 14336)
                    print(f"[bench] composed {name} M={M}: {e}", file=sys.stderr, flush=True)
            out[f"{name}_M{M}"] = {"us": us, "TFLOPs": 2 * M * N * K / us / 1e6,
                                   "fused_us": usf, "fused_TFLOPs": 2 * M * N * K / usf / 1e6,
                                   "composed_us": usc, "composed_TFLOPs": usc and 2 * M * N * K / usc / 1e6,
                                   "note": "us: cuda_gemm_int8 (fused int8 prefill MFMA kernel below 4096 tokens, "
                                           "dequantize + hipBLASLt from 4096 on); fused: the prefill kernel "
                                           "(ng_gemm_int8_noalloc); composed: cuda_dequantize_weights + "
                                           "cuda_gemm_fp16"}
            prefill.setdefault(M, [0.0, 0.0, 0.0])
            prefill[M][0] += per_layer[name] * us
            prefill[M][1] += per_layer[name] * (usc or float("nan"))
            prefill[M][2] += per_layer[name] * usf
            ab.free()
            cb.free()
        wp.free()
        sc.free()
        deq.free()
    for M, (u, c, *f) in list(layer.items()) + list(prefill.items()):
        out[f"mistral7b_layer_M{M}"] = {"us": u, "composed_us": None if c != c else c,
                                        "note": "q, k, v, o, gate, up, down projections of one layer"}
        if f:
            out[f"mistral7b_layer_M{M}"]["fused_us"] = f[0]
    return out


def shared_a_extras(L, hip, stream):
    """ng_gemm_int8_shared_a against separate cuda_gemm_int8 calls for the
    projections of one Mistral-7B INT8 layer that read the same normed rows:
    q/k/v (layer.cu:487-501) and gate/up (layer.cu:575-583), at M = 1, 2, 8,
    32 and 64 decode tokens and 512 and 2048 prefill tokens. Both forms give
    the same bits; weight pools keep the codes cache-cold."""
    rng = np.random.Generator(np.random.PCG64(5))
    K = 4096
    sets = {"qkv": [4096, 1024, 1024], "gate_up": [14336, 14336]}
    out = {}
    for name, ns in sets.items():
        n = pool_slots(sum(ns) * K)
        wqs, scs = [], []
        for N in ns:
            wqs.append(rng.integers(-128, 128, (N, K)).astype(np.int8))
            scs.append(DB.from_array(rng.uniform(1e-3, 1e-2, N).astype(np.float32)))
        grp = GroupPool(hip, wqs, n)
        pools = [(N, grp.member(p), sc) for p, (N, sc) in enumerate(zip(ns, scs))]
        del wqs
        cnt = len(ns)
        for M in (1, 2, 8, 32, 64, 512, 2048):
            ab = DB.from_array(W.round_to(rng.standard_normal((M, K), dtype=np.float32), "f16"))
            cps = [Pool(hip, 2 * M * N, n) for N in ns]

            def sep(j, M=M, ab=ab, cps=cps):
                for (N, wp, sc), cp in zip(pools, cps):
                    rc = L.cuda_gemm_int8(cp.at(j), ab.vp, wp.at(j), sc.vp, M, K, N, True)
                    if rc:
                        return rc
                return 0

            args = [((C.c_void_p * cnt)(*[cp.at(j) for cp in cps]), (C.c_void_p * cnt)(*[wp.at(j) for _, wp, _ in pools]))
                    for j in range(n)]
            scv = (C.c_void_p * cnt)(*[sc.ptr for _, _, sc in pools])
            nv = (C.c_int * cnt)(*ns)
            tr = time_rotating(hip, stream, {
                "separate": [("separate", (lambda j=j: sep(j))) for j in range(n)],
                "shared": [("shared", (lambda j=j, M=M, ab=ab: L.ng_gemm_int8_shared_a(
                    cnt, args[j][0], ab.vp, args[j][1], scv, nv, M, K))) for j in range(n)]})
            us_sep, us_sh = tr["separate"], tr["shared"]
            b = sum(N * K + 2 * M * N + 4 * N for N in ns) + 2 * M * K
            out[f"{name}_M{M}"] = {"us": us_sh, "separate_us": us_sep, "GBps": b / us_sh / 1e3,
                                   "frac": b / us_sh / 1e3 / PEAK_GBPS, "bytes": b, "buffer_sets": n}
            for cp in cps:
                cp.free()
            ab.free()
        for _, wp, sc in pools:
            sc.free()
        grp.free()
    out["note"] = ("us: one ng_gemm_int8_shared_a call (one launch per group of products with the same launch "
                   "shape: the GEMV kernel at 1-2 tokens, the small-M MFMA kernel for q/k/v at 8, the split kernel "
                   "and its reduction up to 128 tokens (at 64 q alone and k/v together), the fused prefill kernel "
                   "and its reduction above); separate_us: one cuda_gemm_int8 call per projection")
    return out


def norm_shared_extras(L, hip, stream):
    """The decode steps norm -> projections of one Mistral-7B INT8 layer as one
    call against the two calls it replaces: RMSNorm then q/k/v
    (layer.cu:467,487-501); residual add + RMSNorm then q/k/v (the previous
    layer's last residual add folded into the attention norm); residual add +
    RMSNorm then gate/up (layer.cu:559-583); at M = 1, 2 and 4 tokens. us:
    ng_rmsnorm_gemm_int8_shared_a / ng_add_rmsnorm_gemm_int8_shared_a;
    two_calls_us: cuda_rmsnorm / cuda_add_rmsnorm, then ng_gemm_int8_shared_a.
    The call is one launch where the products take at most 1024 GEMV blocks
    (q/k/v at 1-2 tokens) and the two calls otherwise. Both give the same
    bits; weight pools keep the codes cache-cold."""
    rng = np.random.Generator(np.random.PCG64(6))
    K = 4096
    out = {}
    w = DB.from_array(W.round_to(1 + 0.05 * rng.standard_normal(K, dtype=np.float32), "f16"))
    for name, ns, add in (("rmsnorm_qkv", [4096, 1024, 1024], False), ("add_rmsnorm_qkv", [4096, 1024, 1024], True),
                          ("add_rmsnorm_gate_up", [14336, 14336], True)):
        n = pool_slots(sum(ns) * K)
        wqs, scs = [], []
        for N in ns:
            wqs.append(rng.integers(-128, 128, (N, K)).astype(np.int8))
            scs.append(DB.from_array(rng.uniform(1e-3, 1e-2, N).astype(np.float32)))
        grp = GroupPool(hip, wqs, n)
        pools = [(N, grp.member(p), sc) for p, (N, sc) in enumerate(zip(ns, scs))]
        del wqs
        cnt = len(ns)
        scv = (C.c_void_p * cnt)(*[sc.ptr for _, _, sc in pools])
        nv = (C.c_int * cnt)(*ns)
        for M in (1, 2, 4):
            xb = DB.from_array(W.round_to(rng.standard_normal((M, K), dtype=np.float32), "f16"))
            rb = DB.from_array(W.round_to(rng.standard_normal((M, K), dtype=np.float32), "f16"))
            yb, rob = DB(2 * M * K), DB(2 * M * K)
            cps = [Pool(hip, 2 * M * N, n) for N in ns]
            args = [((C.c_void_p * cnt)(*[cp.at(j) for cp in cps]), (C.c_void_p * cnt)(*[wp.at(j) for _, wp, _ in pools]))
                    for j in range(n)]
            eps = C.c_float(1e-5)

            def one(j, M=M, xb=xb, rb=rb, yb=yb, rob=rob):
                if add:
                    return L.ng_add_rmsnorm_gemm_int8_shared_a(cnt, yb.vp, rob.vp, args[j][0], xb.vp, rb.vp, w.vp, eps,
                                                               args[j][1], scv, nv, M, K)
                return L.ng_rmsnorm_gemm_int8_shared_a(cnt, yb.vp, args[j][0], xb.vp, w.vp, eps, args[j][1], scv, nv,
                                                       M, K)

            def two(j, M=M, xb=xb, rb=rb, yb=yb, rob=rob):
                rc = (L.cuda_add_rmsnorm(yb.vp, rob.vp, xb.vp, rb.vp, w.vp, M, K, eps) if add
                      else L.cuda_rmsnorm(yb.vp, xb.vp, w.vp, M, K, eps))
                return rc or L.ng_gemm_int8_shared_a(cnt, args[j][0], yb.vp, args[j][1], scv, nv, M, K)

            tr = time_rotating(hip, stream, {"two_calls": [("two_calls", (lambda j=j: two(j))) for j in range(n)],
                                             "fused": [("fused", (lambda j=j: one(j))) for j in range(n)]})
            us_two, us_one = tr["two_calls"], tr["fused"]
            rows = 2 * M * K * ((3 if add else 1) + (2 if add else 1)) + 2 * K   # x (+res) in, normed (+res_out) out, w
            b = sum(N * K + 2 * M * N + 4 * N for N in ns) + rows
            out[f"{name}_M{M}"] = {"us": us_one, "two_calls_us": us_two, "GBps": b / us_one / 1e3,
                                   "frac": b / us_one / 1e3 / PEAK_GBPS, "bytes": b, "buffer_sets": n}
            for cp in cps:
                cp.free()
            for x in (xb, rb, yb, rob):
                x.free()
        for _, wp, sc in pools:
            sc.free()
        grp.free()
    w.free()
    return out


def silu_mul_gemm_extras(L, hip, stream, K=4096, N=14336):
    """The gate/up projections and SwiGLU (layer.cu:575-588) at M = 1, 2, 4, 8
    and 64 tokens, Mistral-7B's by default (N = 11008: Llama-2-7B's). us:
    ng_gemm_int8_silu_mul (the GEMV kernel at M <= 2 here; from 3 rows the
    split kernel's SwiGLU form, or with K slices (N = 11008) one shared split
    launch and the reduction's SwiGLU form);
    two_calls_us: ng_gemm_int8_shared_a, then cuda_silu_mul. Both give the same bits; weight pools keep the codes
    cache-cold."""
    rng = np.random.Generator(np.random.PCG64(8))
    n = pool_slots(2 * N * K)
    wqs, scs = [], []
    for _ in range(2):
        wqs.append(rng.integers(-128, 128, (N, K)).astype(np.int8))
        scs.append(DB.from_array(rng.uniform(1e-3, 1e-2, N).astype(np.float32)))
    grp = GroupPool(hip, wqs, n)
    del wqs
    (gp, gs), (up_, us_) = (grp.member(0), scs[0]), (grp.member(1), scs[1])
    out = {}
    for M in (1, 2, 4, 8, 64):
        ab = DB.from_array(W.round_to(rng.standard_normal((M, K), dtype=np.float32), "f16"))
        gb, ub, ob = (Pool(hip, 2 * M * N, n) for _ in range(3))
        scv = (C.c_void_p * 2)(gs.ptr, us_.ptr)
        nv = (C.c_int * 2)(N, N)

        def one(j, M=M, ab=ab, gb=gb, ub=ub, ob=ob):
            return L.ng_gemm_int8_silu_mul(ob.at(j), gb.at(j), ub.at(j), ab.vp, gp.at(j), gs.vp, up_.at(j), us_.vp,
                                           M, K, N)

        def two(j, M=M, ab=ab, gb=gb, ub=ub, ob=ob):
            rc = L.ng_gemm_int8_shared_a(2, (C.c_void_p * 2)(gb.at(j), ub.at(j)), ab.vp,
                                         (C.c_void_p * 2)(gp.at(j), up_.at(j)), scv, nv, M, K)
            return rc or L.cuda_silu_mul(ob.at(j), gb.at(j), ub.at(j), M * N)

        tr = time_rotating(hip, stream, {"two_calls": [("two_calls", (lambda j=j: two(j))) for j in range(n)],
                                         "fused": [("fused", (lambda j=j: one(j))) for j in range(n)]})
        us_two, us_one = tr["two_calls"], tr["fused"]
        b = 2 * (N * K + 4 * N) + 2 * M * K + 3 * 2 * M * N
        out[f"gate_up_silu_mul_M{M}"] = {"us": us_one, "two_calls_us": us_two, "GBps": b / us_one / 1e3,
                                         "frac": b / us_one / 1e3 / PEAK_GBPS, "bytes": b, "buffer_sets": n}
        for x in (gb, ub, ob):
            x.free()
        ab.free()
    for s in scs:
        s.free()
    grp.free()
    return out


def gemm_add_extras(L, hip, stream, K=14336, N=4096):
    """Mistral-7B's down projection and the layer's final residual add
    (layer.cu:593-598) at M = 1, 2, 4, 8, 64, 512 and 2048 tokens. us:
    ng_gemm_int8_add (one launch on the GEMV kernel's shapes, M <= 2 here; from
    3 tokens the split kernel, and from 129 the prefill kernel, with the add in
    the reduction of their K slices); two_calls_us: cuda_gemm_int8, then
    cuda_add. Both give the same bits; weight pools keep
    the codes cache-cold."""
    rng = np.random.Generator(np.random.PCG64(9))
    n = pool_slots(N * K)
    wq = rng.integers(-128, 128, (N, K)).astype(np.int8)
    wp = Pool(hip, wq.nbytes, n, wq)
    del wq
    sc = DB.from_array(rng.uniform(1e-3, 1e-2, N).astype(np.float32))
    out = {}
    for M in (1, 2, 4, 8, 64, 512, 2048):
        ab = DB.from_array(W.round_to(rng.standard_normal((M, K), dtype=np.float32), "f16"))
        rb = DB.from_array(W.round_to(rng.standard_normal((M, N), dtype=np.float32), "f16"))
        cb, ob = Pool(hip, 2 * M * N, n), Pool(hip, 2 * M * N, n)

        def one(j, M=M, ab=ab, rb=rb, cb=cb, ob=ob):
            return L.ng_gemm_int8_add(ob.at(j), cb.at(j), ab.vp, wp.at(j), sc.vp, rb.vp, M, K, N)

        def two(j, M=M, ab=ab, rb=rb, cb=cb, ob=ob):
            return (L.cuda_gemm_int8(cb.at(j), ab.vp, wp.at(j), sc.vp, M, K, N, True)
                    or L.cuda_add(ob.at(j), cb.at(j), rb.vp, M * N))

        tr = time_rotating(hip, stream, {"two_calls": [("two_calls", (lambda j=j: two(j))) for j in range(n)],
                                         "fused": [("fused", (lambda j=j: one(j))) for j in range(n)]})
        us_two, us_one = tr["two_calls"], tr["fused"]
        b = N * K + 4 * N + 2 * M * K + 3 * 2 * M * N
        out[f"down_add_M{M}"] = {"us": us_one, "two_calls_us": us_two, "GBps": b / us_one / 1e3,
                                 "frac": b / us_one / 1e3 / PEAK_GBPS, "bytes": b, "buffer_sets": n}
        for x in (cb, ob):
            x.free()
        ab.free()
        rb.free()
    wp.free()
    sc.free()
    return out


def int8_decode_layer_extras(L, hip, stream):
    """One Mistral-7B INT8 layer at decode (M = 1, 2, 8 and 64 tokens), everything
    but attention, as one graph step on cache-cold weights (a pool of weight
    sets, 218 MB each). engine_us: the engine's own calls
    (gpu/engine/layer.cu:458-598) on this library, 17 launches: copy residual,
    RMSNorm, q, k, v, RoPE Q, RoPE K, o, add, copy residual, RMSNorm in place,
    gate, up, SiLU, mul, down, add. fused_us: the same layer through the fused
    entry points, 6 launches: ng_rmsnorm_gemm_int8_shared_a (q/k/v),
    ng_rope_qk_with_theta, o, cuda_add_rmsnorm (normed in place, the layer
    input as residual), ng_gemm_int8_silu_mul (in place on gate),
    ng_gemm_int8_add. fused_rope_us: the same with RMSNorm, q/k/v and RoPE in
    one launch (ng_rmsnorm_qkv_rope_int8), 5 launches. From M = 3 on the fused
    calls are their compositions (norm, then ng_gemm_int8_shared_a, ...), so
    only the shared-A products and the fused memory-bound entry points remain
    of the fusion. The attention output is a fixed buffer."""
    rng = np.random.Generator(np.random.PCG64(10))
    H, I, NQ, NKV, D = 4096, 14336, 32, 8, 128
    KV = NKV * D
    eps, theta = C.c_float(1e-5), C.c_float(1e6)
    shapes = {"q": (H, H), "k": (KV, H), "v": (KV, H), "o": (H, H), "gate": (I, H), "up": (I, H), "down": (H, I)}
    n = pool_slots(sum(a * b for a, b in shapes.values()))
    wqs, ws = [], {}
    for name, (N, K) in shapes.items():
        wqs.append(rng.integers(-128, 128, (N, K)).astype(np.int8))
        ws[name] = DB.from_array(rng.uniform(1e-3, 1e-2, N).astype(np.float32))
    grp = GroupPool(hip, wqs, n)   # the layer's weights one after another, as an engine loads them
    wp = {name: grp.member(p) for p, name in enumerate(shapes)}
    del wqs
    w_attn = DB.from_array(W.round_to(1 + 0.05 * rng.standard_normal(H, dtype=np.float32), "f16"))
    w_ffn = DB.from_array(W.round_to(1 + 0.05 * rng.standard_normal(H, dtype=np.float32), "f16"))
    out = {}
    for M in (1, 2, 8, 64):
        f16 = lambda *shape: DB.from_array(W.round_to(rng.standard_normal(shape, dtype=np.float32), "f16"))
        x, attn = f16(M, H), f16(M, H)
        pos = DB.from_array(np.arange(100, 100 + M, dtype=np.int32))
        normed, res, res2, q, o, out_b = (DB(2 * M * H) for _ in range(6))
        gate, up = DB(2 * M * I), DB(2 * M * I)
        k_b, v_b = DB(2 * M * KV), DB(2 * M * KV)
        nb = 2 * M * H

        def gemm(c, a, name, j, N, K):
            return L.cuda_gemm_int8(c.vp, a.vp, wp[name].at(j), ws[name].vp, M, K, N, True)

        def engine(j):
            steps = (
                lambda: hip.h.hipMemcpyAsync(res.vp, x.vp, nb, 3, stream),
                lambda: L.cuda_rmsnorm(normed.vp, x.vp, w_attn.vp, M, H, eps),
                lambda: gemm(q, normed, "q", j, H, H),
                lambda: gemm(k_b, normed, "k", j, KV, H),
                lambda: gemm(v_b, normed, "v", j, KV, H),
                lambda: L.cuda_rope_with_theta(q.vp, q.vp, pos.ip, 1, M, NQ, D, 0, theta),
                lambda: L.cuda_rope_with_theta(k_b.vp, k_b.vp, pos.ip, 1, M, NKV, D, 0, theta),
                lambda: gemm(normed, attn, "o", j, H, H),
                lambda: L.cuda_add(normed.vp, normed.vp, res.vp, M * H),
                lambda: hip.h.hipMemcpyAsync(res.vp, normed.vp, nb, 3, stream),
                lambda: L.cuda_rmsnorm(normed.vp, normed.vp, w_ffn.vp, M, H, eps),
                lambda: gemm(gate, normed, "gate", j, I, H),
                lambda: gemm(up, normed, "up", j, I, H),
                lambda: L.cuda_silu(gate.vp, gate.vp, M * I),
                lambda: L.cuda_mul(gate.vp, gate.vp, up.vp, M * I),
                lambda: gemm(normed, gate, "down", j, H, I),
                lambda: L.cuda_add(out_b.vp, normed.vp, res.vp, M * H),
            )
            for f in steps:
                rc = f()
                if rc:
                    return rc
            return 0

        qkv_n = (C.c_int * 3)(H, KV, KV)
        qkv_s = (C.c_void_p * 3)(ws["q"].ptr, ws["k"].ptr, ws["v"].ptr)
        qkv_c = (C.c_void_p * 3)(q.ptr, k_b.ptr, v_b.ptr)

        def fused(j, rope_in_qkv=False):
            qkv_w = (C.c_void_p * 3)(wp["q"].at(j), wp["k"].at(j), wp["v"].at(j))
            front = (
                (lambda: L.ng_rmsnorm_qkv_rope_int8(normed.vp, q.vp, k_b.vp, v_b.vp, x.vp, w_attn.vp, eps, qkv_w,
                                                    qkv_s, pos.ip, M, H, NQ, NKV, D, theta)),
            ) if rope_in_qkv else (
                lambda: L.ng_rmsnorm_gemm_int8_shared_a(3, normed.vp, qkv_c, x.vp, w_attn.vp, eps, qkv_w, qkv_s,
                                                        qkv_n, M, H),
                lambda: L.ng_rope_qk_with_theta(q.vp, q.vp, k_b.vp, k_b.vp, pos.ip, 1, M, NQ, NKV, D, 0, theta),
            )
            steps = front + (
                lambda: gemm(o, attn, "o", j, H, H),
                lambda: L.cuda_add_rmsnorm(normed.vp, res2.vp, o.vp, x.vp, w_ffn.vp, M, H, eps),
                lambda: L.ng_gemm_int8_silu_mul(gate.vp, gate.vp, up.vp, normed.vp, wp["gate"].at(j), ws["gate"].vp,
                                                wp["up"].at(j), ws["up"].vp, M, H, I),
                lambda: L.ng_gemm_int8_add(out_b.vp, normed.vp, gate.vp, wp["down"].at(j), ws["down"].vp, res2.vp,
                                           M, I, H),
            )
            for f in steps:
                rc = f()
                if rc:
                    return rc
            return 0

        tr = time_rotating(hip, stream, {
            "engine": [("engine", (lambda j=j: engine(j))) for j in range(n)],
            "fused": [("fused", (lambda j=j: fused(j))) for j in range(n)],
            "fused_rope": [("fused_rope", (lambda j=j: fused(j, True))) for j in range(n)]}, launches=12)
        us_e, us_f, us_r = tr["engine"], tr["fused"], tr["fused_rope"]
        wbytes = sum(a * b + 4 * a for a, b in shapes.values())
        out[f"M{M}"] = {"engine_us": us_e, "fused_us": us_f, "fused_rope_us": us_r, "weight_bytes": wbytes,
                        "fused_weight_GBps": wbytes / us_r / 1e3, "fused_frac": wbytes / us_r / 1e3 / PEAK_GBPS,
                        "launches": {"engine": 17, "fused": 6 if M <= 2 else None,
                                     "fused_rope": 5 if M <= 2 else None}, "buffer_sets": n}
        for b_ in (x, attn, pos, normed, res, res2, q, o, out_b, gate, up, k_b, v_b):
            b_.free()
    for name in shapes:
        ws[name].free()
    grp.free()
    w_attn.free()
    w_ffn.free()
    out["note"] = ("attention excluded (its output is a fixed buffer); engine = the reference's call sequence on this "
                   "library (its cuda_gemm_int8 calls take the fused GEMV kernels), fused = the six fused entry points")
    return out


# ----------------------------------------------------------------------------- access-pattern floors

# Hand-written kernels that move exactly the bytes of a library kernel, in its
# access pattern, with no arithmetic: the time that pattern costs on this GPU.
# They are measurement aids, not part of the library: compiled at run time
# with hipRTC from this source and launched through the module API.
FLOOR_SRC = r"""
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
// One row of 64 V 16-byte vectors per one-wave workgroup, all loads first
// (the row kernels' pattern). MODE 0: read only; 1: write 8 bytes per vector
// (int8 codes of an fp16 row, 8-byte stores); 2: the same, 16-byte stores
// after a lane-pair exchange; 3: write 16 bytes per vector (a 1:1 row copy);
// 4: write only, 8 bytes per vector.
template <int MODE, int V>
__device__ void rows(void* out, const u32x4* x, unsigned* sink) {
    const unsigned lane = threadIdx.x;
    const u32x4* r = x + (unsigned long long)blockIdx.x * (64 * V);
    u32x4 v[V];
    if (MODE != 4) {
#pragma unroll
        for (int k = 0; k < V; ++k) v[k] = __builtin_nontemporal_load(r + lane + 64 * k);
    } else {
#pragma unroll
        for (int k = 0; k < V; ++k) v[k] = u32x4{lane, (unsigned)k, blockIdx.x, 7u};
    }
    if (MODE == 0) {
        u32x4 a = v[0];
#pragma unroll
        for (int k = 1; k < V; ++k) a ^= v[k];
        if ((a[0] ^ a[1] ^ a[2] ^ a[3]) == 0x9e3779b9u) sink[0] = a[0];
    } else if (MODE == 1 || MODE == 4) {
        u32x2* q = (u32x2*)out + (unsigned long long)blockIdx.x * (64 * V);
#pragma unroll
        for (int k = 0; k < V; ++k) __builtin_nontemporal_store(u32x2{v[k][0] ^ v[k][1], v[k][2] ^ v[k][3]}, q + lane + 64 * k);
    } else if (MODE == 2) {
        char* q = (char*)out + (unsigned long long)blockIdx.x * (64 * V) * 8;
        const bool odd = lane & 1;
#pragma unroll
        for (int k = 0; k < V; k += 2) {
            const u32x2 c0 = {v[k][0] ^ v[k][1], v[k][2] ^ v[k][3]};
            const u32x2 c1 = {v[k + 1][0] ^ v[k + 1][1], v[k + 1][2] ^ v[k + 1][3]};
            const u32x2 send = odd ? c0 : c1;
            const u32x2 recv = {(unsigned)__builtin_amdgcn_update_dpp(0, (int)send[0], 0xB1, 0xf, 0xf, false),
                                (unsigned)__builtin_amdgcn_update_dpp(0, (int)send[1], 0xB1, 0xf, 0xf, false)};
            const u32x4 o = odd ? u32x4{recv[0], recv[1], c1[0], c1[1]} : u32x4{c0[0], c0[1], recv[0], recv[1]};
            const unsigned v0 = odd ? (lane - 1 + (k + 1) * 64) : (lane + k * 64);
            __builtin_nontemporal_store(o, (u32x4*)(q + v0 * 8));
        }
    } else {
        u32x4* y = (u32x4*)out + (unsigned long long)blockIdx.x * (64 * V);
#pragma unroll
        for (int k = 0; k < V; ++k) __builtin_nontemporal_store(v[k] ^ u32x4{1u, 2u, 3u, 4u}, y + lane + 64 * k);
    }
}
// The int8 row pattern with its scale stores (one word per row into `sink`,
// 4096 rows): R rows per one-wave workgroup, every load first; or a
// persistent grid striding over the rows, the next row's loads issued before
// the current row is stored.
template <int R>
__device__ void rows_code8_scales(void* out, const u32x4* x, unsigned* sink) {
    const unsigned lane = threadIdx.x;
    const unsigned row0 = blockIdx.x * R;
    u32x4 v[R][8];
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int k = 0; k < 8; ++k) v[j][k] = __builtin_nontemporal_load(x + (unsigned long long)(row0 + j) * 512 + lane + 64 * k);
#pragma unroll
    for (int j = 0; j < R; ++j) {
        unsigned m = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) m ^= v[j][k][0] ^ v[j][k][3];
        m ^= (unsigned)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xf, 0xf, false);
        u32x2* q = (u32x2*)out + (unsigned long long)(row0 + j) * 512;
#pragma unroll
        for (int k = 0; k < 8; ++k) __builtin_nontemporal_store(u32x2{v[j][k][0] ^ v[j][k][1], v[j][k][2] ^ v[j][k][3] ^ m}, q + lane + 64 * k);
        if (lane == 0) sink[row0 + j] = m;
    }
}
extern "C" __global__ __launch_bounds__(64) void floor_rows_code8_scales(void* o, const u32x4* x, unsigned* s) { rows_code8_scales<1>(o, x, s); }
extern "C" __global__ __launch_bounds__(64) void floor_rows4_code8_scales(void* o, const u32x4* x, unsigned* s) { rows_code8_scales<4>(o, x, s); }
extern "C" __global__ __launch_bounds__(64) void floor_persistent_code8_scales(void* o, const u32x4* x, unsigned* s) {
    const unsigned lane = threadIdx.x, G = gridDim.x;
    unsigned r = blockIdx.x;
    u32x4 a[8], b[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) a[k] = __builtin_nontemporal_load(x + (unsigned long long)r * 512 + lane + 64 * k);
    while (r < 4096u) {
        const unsigned rn = r + G < 4096u ? r + G : r;
#pragma unroll
        for (int k = 0; k < 8; ++k) b[k] = __builtin_nontemporal_load(x + (unsigned long long)rn * 512 + lane + 64 * k);
        __builtin_amdgcn_sched_barrier(0);
        unsigned m = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) m ^= a[k][0] ^ a[k][3];
        u32x2* q = (u32x2*)o + (unsigned long long)r * 512;
#pragma unroll
        for (int k = 0; k < 8; ++k) __builtin_nontemporal_store(u32x2{a[k][0] ^ a[k][1], a[k][2] ^ a[k][3] ^ m}, q + lane + 64 * k);
        if (lane == 0) s[r] = m;
        if (rn == r) break;
#pragma unroll
        for (int k = 0; k < 8; ++k) a[k] = b[k];
        r = rn;
    }
}
// A 1:1 row copy, four rows per one-wave workgroup, every load first.
extern "C" __global__ __launch_bounds__(64) void floor_rows4_copy(u32x4* y, const u32x4* x) {
    const unsigned lane = threadIdx.x;
    const unsigned long long row0 = (unsigned long long)blockIdx.x * 4;
    u32x4 v[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int k = 0; k < 8; ++k) v[j][k] = __builtin_nontemporal_load(x + (row0 + j) * 512 + lane + 64 * k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int k = 0; k < 8; ++k) __builtin_nontemporal_store(v[j][k] ^ u32x4{1u, 2u, 3u, 4u}, y + (row0 + j) * 512 + lane + 64 * k);
}
extern "C" __global__ __launch_bounds__(64) void floor_rows_read(void* o, const u32x4* x, unsigned* s) { rows<0, 8>(o, x, s); }
extern "C" __global__ __launch_bounds__(64) void floor_rows_code8(void* o, const u32x4* x, unsigned* s) { rows<1, 8>(o, x, s); }
extern "C" __global__ __launch_bounds__(64) void floor_rows_code16(void* o, const u32x4* x, unsigned* s) { rows<2, 8>(o, x, s); }
extern "C" __global__ __launch_bounds__(64) void floor_rows_copy(void* o, const u32x4* x, unsigned* s) { rows<3, 8>(o, x, s); }
extern "C" __global__ __launch_bounds__(64) void floor_rows_write8(void* o, const u32x4* x, unsigned* s) { rows<4, 8>(o, x, s); }
// Flat streams, one 16-byte vector per lane: a 1:1 copy, and 16 bytes in /
// 8 bytes out.
extern "C" __global__ __launch_bounds__(64) void floor_flat_copy(u32x4* y, const u32x4* x) {
    const unsigned long long i = (unsigned long long)blockIdx.x * 64 + threadIdx.x;
    __builtin_nontemporal_store(__builtin_nontemporal_load(x + i), y + i);
}
extern "C" __global__ __launch_bounds__(64) void floor_flat_code8(u32x2* q, const u32x4* x) {
    const unsigned long long i = (unsigned long long)blockIdx.x * 64 + threadIdx.x;
    const u32x4 v = __builtin_nontemporal_load(x + i);
    __builtin_nontemporal_store(u32x2{v[0] ^ v[1], v[2] ^ v[3]}, q + i);
}
extern "C" __global__ __launch_bounds__(64) void floor_empty(unsigned* s) {
    if (threadIdx.x == 1000u) s[0] = 1u;
}
"""


class FloorKernels:
    """FLOOR_SRC compiled for gfx950 with hipRTC and loaded as a module."""

    def __init__(self, hip):
        rtc = C.CDLL("libhiprtc.so")
        prog = C.c_void_p()
        if rtc.hiprtcCreateProgram(C.byref(prog), FLOOR_SRC.encode(), b"floors.hip", 0, None, None) != 0:
            raise RuntimeError("hiprtcCreateProgram failed")
        opts = [b"--offload-arch=gfx950", b"-O3"]
        arr = (C.c_char_p * len(opts))(*opts)
        rc = rtc.hiprtcCompileProgram(prog, len(opts), arr)
        if rc != 0:
            n = C.c_size_t()
            rtc.hiprtcGetProgramLogSize(prog, C.byref(n))
            log = C.create_string_buffer(n.value)
            rtc.hiprtcGetProgramLog(prog, log)
            raise RuntimeError(f"hiprtcCompileProgram failed: {log.value.decode(errors='replace')}")
        n = C.c_size_t()
        rtc.hiprtcGetCodeSize(prog, C.byref(n))
        self.code = C.create_string_buffer(n.value)
        rtc.hiprtcGetCode(prog, self.code)
        rtc.hiprtcDestroyProgram(C.byref(prog))
        self.hip = hip
        self.mod = C.c_void_p()
        hip.check(hip.h.hipModuleLoadData(C.byref(self.mod), self.code), "hipModuleLoadData")
        self.fns = {}
        hip.h.hipModuleLaunchKernel.argtypes = [C.c_void_p] + [C.c_uint] * 6 + [C.c_uint, C.c_void_p, C.c_void_p,
                                                                                 C.c_void_p]

    def fn(self, name):
        if name not in self.fns:
            f = C.c_void_p()
            self.hip.check(self.hip.h.hipModuleGetFunction(C.byref(f), self.mod, name.encode()),
                           "hipModuleGetFunction")
            self.fns[name] = f
        return self.fns[name]

    def launch(self, name, grid, stream, *ptrs):
        args = [C.c_void_p(p.value if isinstance(p, C.c_void_p) else p) for p in ptrs]
        params = (C.c_void_p * len(args))(*[C.cast(C.byref(a), C.c_void_p) for a in args])
        return self.hip.h.hipModuleLaunchKernel(self.fn(name), grid, 1, 1, 64, 1, 1, 0, stream, params, None)

    def unload(self):
        self.hip.h.hipModuleUnload(self.mod)


def floor_extras(hip, stream):
    """Each access pattern at Mistral-7B prefill sizes (T = H = 4096, fp16)
    next to the library kernel that has it, timed like the kernels (a graph of
    back-to-back launches over buffer pools touching more than 1 GB between
    reuses of a buffer): the 50.3 MB norm+int8 pattern (read 33.5 MB, write
    16.8 MB of codes) with 8- and 16-byte code stores and as a flat stream; the
    67.1 MB 1:1 pattern of RMSNorm, RoPE Q and the gather as rows and as a flat
    stream; the two halves alone; the int8 pattern with its scale stores, one
    and four rows per wave and as a persistent grid of 1024 waves; the 1:1
    pattern four rows per wave; empty grids of 1 to 16384 one-wave workgroups
    (the fixed cost of a launch); and flat copies at the sizes of RoPE K
    (16.8 MB) and of Llama-2-13B's RMSNorm (167.8 MB)."""
    fk = FloorKernels(hip)
    T, H = 4096, 4096
    xb, qb = 2 * T * H, T * H
    nv = T * H // 8
    sink = DB(4 * T)
    out = {}

    def pools(in_bytes, out_bytes):
        n = pool_slots(in_bytes + out_bytes)
        return Pool(hip, in_bytes, n), Pool(hip, max(out_bytes, 256), n), n

    def timed(name, grid, in_bytes, out_bytes, moved, extra_sink=True):
        src, dst, n = pools(in_bytes, out_bytes)
        hip.h.hipMemsetAsync.argtypes = [C.c_void_p, C.c_int, C.c_size_t, C.c_void_p]
        hip.check(hip.h.hipMemsetAsync(src.buf.offset(0), 0x11, src.slot * src.n, None), "hipMemsetAsync")
        hip.sync()
        args = (lambda j: (dst.at(j), src.at(j), sink.vp)) if extra_sink else (lambda j: (dst.at(j), src.at(j)))
        thunks = [(name, (lambda j=j: fk.launch(name, grid, stream, *args(j)))) for j in range(n)]
        us = time_pool_kernel(hip, stream, thunks)
        src.free()
        dst.free()
        return {"us": us, "bytes": moved, "GBps": moved / us / 1e3 if moved else None,
                "frac": moved / us / 1e3 / PEAK_GBPS if moved else None}

    out["rows_code8_50MB"] = timed("floor_rows_code8", T, xb, qb, xb + qb)
    out["rows_code8_scales_50MB"] = timed("floor_rows_code8_scales", T, xb, qb, xb + qb + 4 * T)
    out["rows4_code8_scales_50MB"] = timed("floor_rows4_code8_scales", T // 4, xb, qb, xb + qb + 4 * T)
    out["persistent1024_code8_scales_50MB"] = timed("floor_persistent_code8_scales", 1024, xb, qb, xb + qb + 4 * T)
    out["rows4_copy_67MB"] = timed("floor_rows4_copy", T // 4, xb, xb, 2 * xb, extra_sink=False)
    out["rows_code16_50MB"] = timed("floor_rows_code16", T, xb, qb, xb + qb)
    out["flat_code8_50MB"] = timed("floor_flat_code8", nv // 64, xb, qb, xb + qb, extra_sink=False)
    out["rows_copy_67MB"] = timed("floor_rows_copy", T, xb, xb, 2 * xb)
    out["flat_copy_67MB"] = timed("floor_flat_copy", nv // 64, xb, xb, 2 * xb, extra_sink=False)
    out["rows_read_33MB"] = timed("floor_rows_read", T, xb, 0, xb)
    out["rows_write8_17MB"] = timed("floor_rows_write8", T, 256, qb, qb)
    for label, b in (("flat_copy_17MB", 8 << 20), ("flat_copy_168MB", 2 * 8192 * 5120 * 2 // 2)):
        out[label] = timed("floor_flat_copy", b // 16 // 64, b, b, 2 * b, extra_sink=False)
    for grid in (1, 1024, 4096, 16384):
        thunks = [("floor_empty", (lambda grid=grid: hip.h.hipModuleLaunchKernel(
            fk.fn("floor_empty"), grid, 1, 1, 64, 1, 1, 0, stream,
            (C.c_void_p * 1)(C.cast(C.byref(C.c_void_p(sink.ptr)), C.c_void_p)), None)))]
        out[f"empty_{grid}_workgroups"] = {"us": time_pool_kernel(hip, stream, thunks)}
    sink.free()
    fk.unload()
    out["note"] = ("hand-written kernels with a library kernel's access pattern and bytes and no arithmetic "
                   "(compiled at run time by hipRTC from bench.py's FLOOR_SRC), timed as the kernels are")
    return out


# ----------------------------------------------------------------------------- CPU baseline

def cpu_baseline(cfg, budget_s=10.0, sample_1t=256):
    """The CPU oracle (oracle/ng_oracle.c, a C restatement of the reference
    semantics, built -O3 -march=x86-64-v3 with OpenMP) running the same layer
    kernel set on the same inputs: the full T on all host threads, and a
    sample of `sample_1t` tokens on one thread (the full T would take about 5 s
    per repetition there)."""
    from oracle import oracle as O

    def inputs(T):
        sub = W.LayerConfig(**{**cfg.__dict__, "T": T, "key": f"{cfg.key}_cpu_T{T}"})
        return sub, W.make_layer_inputs(sub, seed=0, with_table=False)

    def ops(sub, d):
        return [("rmsnorm", lambda: O.rmsnorm(d["x"], d["w_attn"], sub.eps, sub.dtype)),
                ("rope_q", lambda: O.rope(d["q"], d["pos"], 0, sub.theta, sub.dtype)),
                ("rope_k", lambda: O.rope(d["k"], d["pos"], 0, sub.theta, sub.dtype)),
                ("add_rmsnorm", lambda: O.add_rmsnorm(d["x"], d["residual"], d["w_ffn"], sub.eps, sub.dtype)),
                ("silu_mul", lambda: O.elementwise("silu_mul", d["gate"], d["up"], dtype=sub.dtype)),
                ("add", lambda: O.elementwise("add", d["x"], d["residual"], dtype=sub.dtype))]

    def measure(sub, d, seconds, min_reps=5):
        """Median layer time and per-kernel medians (s) over repetitions of the six."""
        steps = ops(sub, d)
        for _, f in steps:
            f()
        ts, per = [], {k: [] for k, _ in steps}
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(ts) < min_reps:
            t0 = time.perf_counter()
            for k, f in steps:
                t = time.perf_counter()
                f()
                per[k].append(time.perf_counter() - t)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)), len(ts), {k: float(np.median(v)) for k, v in per.items()}

    sub1, d1 = inputs(sample_1t)
    O.set_threads(1)
    med1, n1, _ = measure(sub1, d1, budget_s / 4, 3)
    b1 = sum(W.layer_bytes(sub1)[k] for k in W.LAYER_KERNELS)
    del d1
    sub, d = inputs(cfg.T)
    O.set_threads(os.cpu_count() or 1)
    cores = O.get_threads()
    med, n, per = measure(sub, d, budget_s)
    nbytes = sum(W.layer_bytes(sub)[k] for k in W.LAYER_KERNELS)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "us_per_layer": med * 1e6, "per_kernel_us": {k: v * 1e6 for k, v in per.items()},
            "value_1_thread": b1 / med1 / 1e9, "us_per_layer_sample_1_thread": med1 * 1e6,
            "build": "gcc -O3 -march=x86-64-v3 -fopenmp -ffp-contract=off (portable x86-64-v3, not -march=native: "
                     "the oracle is built in one container and run on the GPU box's host)",
            "sample": f"{cfg.key} layer kernel set (rmsnorm, rope q, rope k, add+rmsnorm, silu_mul, add) on the "
                      f"full T={cfg.T}: median of {n} reps on {cores} OpenMP threads; one thread on the first "
                      f"{sample_1t} tokens: median of {n1} reps"}


# ----------------------------------------------------------------------------- rocprofv3 profiling pass

PROFILE_LAUNCHES = 5
PROFILE_WARMUP = 20


def profile_pass(L, hip, stream):
    """The program the committed rocprofv3 summaries come from (--kernel-trace
    --stats, and --pmc FETCH_SIZE / WRITE_SIZE in runs of their own). Every
    launch is eager (no graph) and none uses hipBLASLt.

    Calibration: a 256 MiB device-to-device copy (reads and writes 256 MiB),
    and cuda_quantize_per_tensor over 128 Mi fp16 values, whose absmax kernel
    reads 256 MiB and writes one word. Then, for each layer configuration, each
    layer kernel (and ng_rope_qk_with_theta; for bf16 and for Mistral-7B
    prefill also the engine's unfused RMSNorm in place, add in place, SiLU and
    mul in place) PROFILE_LAUNCHES times, each
    launch on a buffer slot untouched for over 1 GB of other traffic; the
    embedding gathers (Mistral-7B uniform ids, Mistral-Nemo Zipf ids); fused
    RMSNorm + int8, residual add + RMSNorm + int8 and int8 dequant at the
    quant configuration; QK LayerNorm + RoPE. Before each group a line
    "[profile] <label> dispatches=<n>" goes to stderr: n is the number of this
    library's kernel dispatches in the group, in order, so a summary can name
    every dispatch of the trace."""

    def group(label, thunks, per_call=1, warm=PROFILE_WARMUP):
        # `warm` launches, then PROFILE_LAUNCHES measured ones, all enqueued
        # without waiting, cycling over the buffer slots: the GPU stays busy
        # (clocks up) and every launch finds a slot untouched since a full
        # cycle of the others.
        seq = [thunks[i % len(thunks)] for i in range(warm + PROFILE_LAUNCHES)]
        log_profile(label, PROFILE_LAUNCHES * per_call, warm * per_call)
        for fn in seq:
            if fn() != 0:
                raise RuntimeError(f"{label} failed")
        hip.sync()

    nbytes = 256 << 20
    src, dst = DB(nbytes), DB(nbytes)
    print("[profile] calib/copy_256MiB rocclr_copies=3", file=sys.stderr, flush=True)
    for _ in range(3):
        hip.check(hip.h.hipMemcpyAsync(dst.vp, src.vp, nbytes, 3, stream), "hipMemcpyAsync")
    hip.sync()
    sc = DB(4)
    # fill (1 thread), absmax (reads 256 MiB), quantise, finalise: 4 dispatches per call
    group("calib/quant_per_tensor_256MiB", [lambda: L.cuda_quantize_per_tensor(dst.vp, sc.vp, src.vp, nbytes // 2)],
          per_call=4, warm=0)
    for b in (src, dst, sc):
        b.free()

    for key in ("mistral7b_prefill", "mistral7b_decode", "llama2_13b_prefill", "mistral_nemo_bf16"):
        cfg = W.CONFIGS[key]
        d = W.make_layer_inputs(cfg, seed=0, with_table=False)
        shared = {"w_attn": DB.from_array(d["w_attn"]), "w_ffn": DB.from_array(d["w_ffn"]),
                  "pos": DB.from_array(d["pos"])}
        for name, make in kernel_pools_for(L, hip, cfg, d, shared):
            thunks, pools = make()
            group(f"{key}/{name}", [fn for _, fn in thunks])
            for p in pools:
                p.free()
        if cfg.dtype == "bf16" or key == "mistral7b_prefill":
            for name, make in engine_unfused_pools_for(L, hip, cfg, d, shared, stream):
                if name == "copy_residual":     # a runtime copy, not a kernel of this library
                    continue
                thunks, pools = make()
                group(f"{key}/engine_{name}", [fn for _, fn in thunks])
                for p in pools:
                    p.free()
        for b in shared.values():
            b.free()
        del d

    # embedding gathers
    for key, ntab in (("mistral7b_prefill", 8), ("mistral_nemo_bf16", 4)):
        cfg = W.CONFIGS[key]
        rng = np.random.Generator(np.random.PCG64(2))
        row_bytes = cfg.H * 2
        tabs = Pool(hip, row_bytes * cfg.vocab, ntab)
        for r0 in range(0, cfg.vocab, 16384):
            n = min(16384, cfg.vocab - r0)
            piece = W.round_to(rng.standard_normal((n, cfg.H), dtype=np.float32) * np.float32(0.02), cfg.dtype)
            hip.check(L.cuda_copy_int8_to_device(tabs.buf.offset(r0 * row_bytes), piece.ctypes.data, piece.nbytes),
                      "upload")
        for j in range(1, ntab):
            hip.check(hip.h.hipMemcpyAsync(tabs.at(j), tabs.at(0), row_bytes * cfg.vocab, 3, None), "hipMemcpyAsync")
        hip.sync()
        zipf = cfg.ids.startswith("zipf")
        ids = np.stack([W.zipf_ids(rng, cfg.T, cfg.vocab, 1.1) if zipf else
                        rng.integers(0, cfg.vocab, cfg.T).astype(np.int32) for _ in range(ntab)])
        idb = DB.from_array(ids)
        outs = Pool(hip, 2 * cfg.T * cfg.H, ntab)
        group(f"{key}/gather_{'zipf' if zipf else 'uniform'}",
              [(lambda j=j: L.cuda_gather_embeddings(outs.at(j), tabs.at(j), C.cast(idb.offset(4 * cfg.T * j),
                                                                                    C.POINTER(C.c_int)),
                                                     cfg.H, cfg.T)) for j in range(ntab)])
        for b in (tabs, outs, idb):
            b.free()

    # quant configuration
    q = W.make_quant_inputs(seed=0)
    T, H, eps = W.QUANT_T, W.QUANT_H, C.c_float(1e-5)
    n = pool_slots(W.quant_bytes()["rmsnorm_quant"])
    xs, res, ro = Pool(hip, q["x"].nbytes, n, q["x"]), Pool(hip, q["x"].nbytes, n, q["x"]), Pool(hip, q["x"].nbytes, n)
    codes, scl = Pool(hip, q["x"].size, n), Pool(hip, 4 * T, n)
    wb = DB.from_array(q["w"])
    group("quant/rmsnorm_quant", [(lambda j=j: L.ng_rmsnorm_quant_int8(codes.at(j), scl.at(j), xs.at(j), wb.vp, T, H,
                                                                       eps)) for j in range(n)])
    group("quant/add_rmsnorm_quant", [(lambda j=j: L.ng_add_rmsnorm_quant_int8(
        codes.at(j), scl.at(j), ro.at(j), xs.at(j), res.at(j), wb.vp, T, H, eps)) for j in range(n)])
    group("quant/quant_per_token", [(lambda j=j: L.cuda_quantize_weights_per_row(codes.at(j), scl.at(j), xs.at(j), T,
                                                                                 H)) for j in range(n)])
    for p in (xs, res, ro, codes, scl):
        p.free()
    wb.free()
    n = pool_slots(W.quant_bytes()["dequant"])
    wq, wo = Pool(hip, q["wq"].nbytes, n, q["wq"]), Pool(hip, 2 * q["wq"].size, n)
    ws = DB.from_array(q["wscale"])
    group("quant/dequant", [(lambda j=j: L.cuda_dequantize_weights(wo.at(j), wq.at(j), ws.vp, W.QUANT_WN, W.QUANT_WK,
                                                                   1)) for j in range(n)])
    for p in (wq, wo):
        p.free()
    ws.free()

    # QK LayerNorm + RoPE at Mistral-7B prefill shapes
    cfg = W.CONFIGS["mistral7b_prefill"]
    d = W.make_layer_inputs(cfg, seed=0, with_table=False)
    T, D, nq, nkv = cfg.T, cfg.D, cfg.nq, cfg.nkv
    n = pool_slots(2 * (d["q"].nbytes + d["k"].nbytes))
    qp, kp = Pool(hip, d["q"].nbytes, n, d["q"]), Pool(hip, d["k"].nbytes, n, d["k"])
    wq, wk, pos = DB.from_array(d["w_attn"][:D]), DB.from_array(d["w_ffn"][:D]), DB.from_array(d["pos"])
    group("mistral7b_prefill/qk_rmsnorm_rope", [(lambda j=j: L.ng_qk_rmsnorm_rope_with_theta(
        qp.at(j), qp.at(j), kp.at(j), kp.at(j), wq.vp, wk.vp, pos.ip, 1, T, nq, nkv, D, eps, 0,
        C.c_float(cfg.theta))) for j in range(n)])
    for p in (qp, kp):
        p.free()
    for b in (wq, wk, pos):
        b.free()
    log("profile pass done")


def profile_decode(L, hip, stream):
    """Eager launches (no graph, no device copies) of the INT8 layer's decode
    steps at Mistral-7B and one token, for a rocprofv3 kernel trace: the fused
    entry points (ng_rmsnorm_qkv_rope_int8, ng_gemm_int8_silu_mul,
    ng_gemm_int8_add; one dispatch per call) and the calls they replace
    (cuda_rmsnorm, ng_gemm_int8_shared_a on q/k/v, ng_rope_qk_with_theta,
    gate/up through ng_gemm_int8_shared_a, cuda_silu_mul, cuda_gemm_int8 on
    down, cuda_add), plus o (cuda_gemm_int8) and cuda_add_rmsnorm. Two weight
    sets, uploaded from the host (436 MB, above the 256 MB Infinity Cache),
    alternate between launches. Before each group a line "[profile] <label>
    warmup=<w> dispatches=<n>" goes to stderr."""
    rng = np.random.Generator(np.random.PCG64(11))
    H, I, NQ, NKV, D, M = 4096, 14336, 32, 8, 128, 1
    KV = NKV * D
    eps, theta = C.c_float(1e-5), C.c_float(1e6)
    shapes = {"q": (H, H), "k": (KV, H), "v": (KV, H), "o": (H, H), "gate": (I, H), "up": (I, H), "down": (H, I)}
    sets = []
    for _ in range(2):
        ws = {}
        for name, (N, K) in shapes.items():
            ws[name] = (DB.from_array(rng.integers(-128, 128, (N, K)).astype(np.int8)),
                        DB.from_array(rng.uniform(1e-3, 1e-2, N).astype(np.float32)))
        sets.append(ws)
    f16 = lambda *shape: DB.from_array(W.round_to(rng.standard_normal(shape, dtype=np.float32), "f16"))
    x, attn, res = f16(M, H), f16(M, H), f16(M, H)
    w_attn = DB.from_array(W.round_to(1 + 0.05 * rng.standard_normal(H, dtype=np.float32), "f16"))
    pos = DB.from_array(np.array([100], np.int32))
    normed, q, o, out, res2 = (DB(2 * M * H) for _ in range(5))
    kb, vb = DB(2 * M * KV), DB(2 * M * KV)
    gate, up, sw = DB(2 * M * I), DB(2 * M * I), DB(2 * M * I)
    qkv_c = (C.c_void_p * 3)(q.ptr, kb.ptr, vb.ptr)
    qkv_n = (C.c_int * 3)(H, KV, KV)
    gu_n = (C.c_int * 2)(I, I)

    def qkv_w(ws):
        return (C.c_void_p * 3)(ws["q"][0].ptr, ws["k"][0].ptr, ws["v"][0].ptr)

    def qkv_s(ws):
        return (C.c_void_p * 3)(ws["q"][1].ptr, ws["k"][1].ptr, ws["v"][1].ptr)

    groups = [
        ("rmsnorm_qkv_rope_int8", 1, lambda ws: L.ng_rmsnorm_qkv_rope_int8(
            normed.vp, q.vp, kb.vp, vb.vp, x.vp, w_attn.vp, eps, qkv_w(ws), qkv_s(ws), pos.ip, M, H, NQ, NKV, D,
            theta)),
        ("rmsnorm", 1, lambda ws: L.cuda_rmsnorm(normed.vp, x.vp, w_attn.vp, M, H, eps)),
        ("qkv_shared_a", 1, lambda ws: L.ng_gemm_int8_shared_a(3, qkv_c, normed.vp, qkv_w(ws), qkv_s(ws), qkv_n, M,
                                                                H)),
        ("rope_qk", 1, lambda ws: L.ng_rope_qk_with_theta(q.vp, q.vp, kb.vp, kb.vp, pos.ip, 1, M, NQ, NKV, D, 0,
                                                          theta)),
        ("o", 1, lambda ws: L.cuda_gemm_int8(o.vp, attn.vp, ws["o"][0].vp, ws["o"][1].vp, M, H, H, True)),
        ("add_rmsnorm", 1, lambda ws: L.cuda_add_rmsnorm(normed.vp, res2.vp, o.vp, x.vp, w_attn.vp, M, H, eps)),
        ("gate_up_silu_mul", 1, lambda ws: L.ng_gemm_int8_silu_mul(sw.vp, gate.vp, up.vp, normed.vp, ws["gate"][0].vp,
                                                                   ws["gate"][1].vp, ws["up"][0].vp, ws["up"][1].vp,
                                                                   M, H, I)),
        ("gate_up_shared_a", 1, lambda ws: L.ng_gemm_int8_shared_a(
            2, (C.c_void_p * 2)(gate.ptr, up.ptr), normed.vp, (C.c_void_p * 2)(ws["gate"][0].ptr, ws["up"][0].ptr),
            (C.c_void_p * 2)(ws["gate"][1].ptr, ws["up"][1].ptr), gu_n, M, H)),
        ("silu_mul", 1, lambda ws: L.cuda_silu_mul(sw.vp, gate.vp, up.vp, M * I)),
        ("down_add", 1, lambda ws: L.ng_gemm_int8_add(out.vp, o.vp, sw.vp, ws["down"][0].vp, ws["down"][1].vp,
                                                      res.vp, M, I, H)),
        ("down", 1, lambda ws: L.cuda_gemm_int8(o.vp, sw.vp, ws["down"][0].vp, ws["down"][1].vp, M, I, H, True)),
        ("add", 1, lambda ws: L.cuda_add(out.vp, o.vp, res.vp, M * H)),
    ]
    for label, per_call, fn in groups:
        seq = [sets[i % 2] for i in range(PROFILE_WARMUP + PROFILE_LAUNCHES)]
        log_profile(f"mistral7b_int8_decode_M1/{label}", PROFILE_LAUNCHES * per_call, PROFILE_WARMUP * per_call)
        for ws in seq:
            if fn(ws) != 0:
                raise RuntimeError(f"{label} failed")
        hip.sync()
    for ws in sets:
        for wq, sc in ws.values():
            wq.free()
            sc.free()
    for b_ in (x, attn, res, w_attn, pos, normed, q, o, out, res2, kb, vb, gate, up, sw):
        b_.free()


def log_profile(label, dispatches, warmup):
    print(f"[profile] {label} warmup={warmup} dispatches={dispatches}", file=sys.stderr, flush=True)


def engine_unfused_pools_for(L, hip, cfg, d, shared, stream):
    """The kernels of the engine's unfused sequence that the fused layer does
    not launch (engine_bf16_launches, engine_int8_launches), with buffer pools
    as in kernel_pools_for: RMSNorm in place, add in place, SiLU in place, mul
    in place, the device copy of the residual, and for bf16 the dtype
    conversions the bf16 layer runs around attention."""
    T, H, I, e = cfg.T, cfg.H, cfg.I, cfg.e
    eps = C.c_float(cfg.eps)
    th, ti = T * H * e, T * I * e
    bf = cfg.dtype == "bf16"
    rms = L.cuda_bf16_rmsnorm if bf else L.cuda_rmsnorm
    add = L.cuda_bf16_add if bf else L.cuda_add
    silu = L.cuda_bf16_silu if bf else L.cuda_silu
    mul = L.cuda_bf16_mul if bf else L.cuda_mul

    def mk(name, footprint, specs, launch):
        def make():
            n = pool_slots(footprint)
            pools = [Pool(hip, nbytes, n, init) for nbytes, init in specs]
            thunks = [(name, (lambda j=j: launch(*[p.at(j) for p in pools]))) for j in range(n)]
            return thunks, pools
        return name, make

    yield mk("rmsnorm_inplace", 2 * th, [(th, d["x"])],
             lambda x: rms(x, x, shared["w_ffn"].vp, T, H, eps))
    yield mk("add", 3 * th, [(th, d["x"]), (th, d["residual"])], lambda a, r: add(a, a, r, T * H))
    yield mk("silu", 2 * ti, [(ti, d["gate"])], lambda g: silu(g, g, T * I))
    yield mk("mul", 3 * ti, [(ti, d["gate"]), (ti, d["up"])], lambda g, u: mul(g, g, u, T * I))
    yield mk("copy_residual", 2 * th, [(th, d["x"]), (th, None)],
             lambda x, o: hip.h.hipMemcpyAsync(o, x, th, 3, stream))
    if not bf:
        return
    # The conversions around attention, with the element counts the engine
    # passes (layer.cu:1537-1543,1574): Q (num_tokens x hidden_size) and K (V is
    # the same) bf16 -> fp16, and the attention output (num_tokens x
    # hidden_size) fp16 -> bf16.
    nk = T * cfg.nkv * cfg.D
    xh = (d["x"].astype(np.uint32) << 16).view(np.float32).astype(np.float16).view(np.uint16)
    yield mk("cvt_q", 2 * th, [(th, d["x"]), (th, None)], lambda q, o: L.cuda_bf16_to_fp16(o, q, T * H))
    yield mk("cvt_k", 4 * nk, [(2 * nk, d["k"]), (2 * nk, None)], lambda k, o: L.cuda_bf16_to_fp16(o, k, nk))
    yield mk("cvt_attn_out", 2 * th, [(th, xh), (th, None)], lambda x, o: L.cuda_fp16_to_bf16(o, x, T * H))


def engine_unfused_kernel_bytes(cfg):
    """Algorithmic bytes of engine_unfused_pools_for's kernels."""
    T, H, I, e = cfg.T, cfg.H, cfg.I, cfg.e
    return {"rmsnorm_inplace": 2 * T * H * e + H * e, "add": 3 * T * H * e, "silu": 2 * T * I * e,
            "mul": 3 * T * I * e, "copy_residual": 2 * T * H * e, "cvt_q": 4 * T * H,
            "cvt_k": 4 * T * cfg.nkv * cfg.D, "cvt_attn_out": 4 * T * H}


def engine_int8_report(cfg, per, seq):
    """The fp16 INT8 engine layer's memory-bound sequence (cuda_layer_forward,
    layer.cu:458-598): its graph step time and per-kernel averages, unfused as
    the engine calls it and with the fused call-site change."""
    b = engine_bf16_bytes(cfg)
    lb = W.layer_bytes(cfg)
    fb = lb["rmsnorm"] + lb["rope_q"] + lb["rope_k"] + lb["add_rmsnorm"] + lb["silu_mul"] + lb["add"]
    ek = engine_unfused_kernel_bytes(cfg)
    eng = seq["engine_int8_kernels_us"]
    unfused_sum = (2 * eng["copy_residual"] + per["rmsnorm"] + per["rope_q"] + per["rope_k"] + eng["add"]
                   + eng["rmsnorm_inplace"] + eng["silu"] + eng["mul"] + per["add"])
    us, fus = seq["engine_int8_step_ms"] * 1e3, seq["engine_int8_fused_step_ms"] * 1e3
    return {
        "unfused": {"us_per_step": us, "us_per_layer": unfused_sum, "layer_bytes": b, "GBps": b / us / 1e3,
                    "sequence": ["copy residual", "rmsnorm", "rope_q", "rope_k", "add (in place)", "copy residual",
                                 "rmsnorm (in place)", "silu (in place)", "mul (in place)", "add"],
                    "kernels": {k: {"us": u, "bytes": ek[k], "frac": ek[k] / u / 1e3 / PEAK_GBPS}
                                for k, u in eng.items()}},
        "fused": {"us_per_step": fus, "layer_bytes": fb, "GBps": fb / fus / 1e3, "frac": fb / fus / 1e3 / PEAK_GBPS,
                  "sequence": ["rmsnorm", "rope_q", "rope_k", "add_rmsnorm (residual_in = layer input, normed in "
                               "place)", "silu_mul (in place)", "add"]},
        "saved_us": us - fus,
        "note": "the engine's INT8 layer (layer.cu:458-598) around its GEMMs and attention; fused = the call sites "
                "changed to the fused entry points (cuda_add + copy + cuda_rmsnorm -> cuda_add_rmsnorm, "
                "cuda_silu + cuda_mul -> cuda_silu_mul, the first copy dropped)"}


# ----------------------------------------------------------------------------- main

def load_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, calibrated on a copy)."""
    try:
        t = json.loads(TRAFFIC_FILE.read_text())
        return t["mistral7b_prefill/silu_mul"]["hbm_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="mistral7b_prefill")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile-pass", "--pmc-pass", dest="profile_pass", action="store_true",
                    help="eager launches of every kernel for rocprofv3 (kernel trace and --pmc runs)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="time only cuda_gemm_int8 at Mistral-7B's INT8 projections and print that JSON")
    ap.add_argument("--profile-decode", action="store_true",
                    help="eager launches of the INT8 layer's decode steps (fused and unfused) for rocprofv3")
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the fused decode entry points and the INT8 decode layer, print that JSON")
    ap.add_argument("--floors-only", action="store_true",
                    help="time only the access-pattern floor kernels and print that JSON")
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
    if args.profile_pass:
        profile_pass(L, hip, stream)
        return
    if args.profile_decode:
        profile_decode(L, hip, stream)
        return
    if args.decode_only:
        print(json.dumps({"norm_gemm_int8_shared_a": norm_shared_extras(L, hip, stream),
                          "gemm_int8_silu_mul": silu_mul_gemm_extras(L, hip, stream),
                          "gemm_int8_silu_mul_llama2_7b": silu_mul_gemm_extras(L, hip, stream, N=11008),
                          "gemm_int8_add": gemm_add_extras(L, hip, stream),
                          "int8_decode_layer": int8_decode_layer_extras(L, hip, stream)}), flush=True)
        return
    if args.gemm_only:
        print(json.dumps({"gemm_int8": gemm_extras(L, hip, stream),
                          "gemm_int8_shared_a": shared_a_extras(L, hip, stream),
                          "norm_gemm_int8_shared_a": norm_shared_extras(L, hip, stream),
                          "gemm_int8_silu_mul": silu_mul_gemm_extras(L, hip, stream),
                          "gemm_int8_silu_mul_llama2_7b": silu_mul_gemm_extras(L, hip, stream, N=11008),
                          "gemm_int8_add": gemm_add_extras(L, hip, stream),
                          "int8_decode_layer": int8_decode_layer_extras(L, hip, stream)}), flush=True)
        return
    if args.floors_only:
        print(json.dumps({"floors": floor_extras(hip, stream)}), flush=True)
        return

    cfg = W.CONFIGS[args.config]
    log(f"layer {cfg.key}: {args.warmup} warmup + {args.steps} timed graph replays")
    step_ms, wall_ms, per, nsets, slots, seq = run_layer(L, hip, stream, cfg, args.steps, args.warmup)
    lb = W.layer_bytes(cfg)
    layer_bytes = sum(lb[k] for k in W.LAYER_KERNELS)
    copy_us = copy_times(hip, stream, [lb[k] for k in W.LAYER_KERNELS])
    kernels = {}
    for k in W.LAYER_KERNELS:
        us = per[k]
        kernels[k] = {"us": us, "GBps": lb[k] / us / 1e3, "frac": lb[k] / us / 1e3 / PEAK_GBPS, "bytes": lb[k],
                      "buffer_sets": slots[k], "copy_us": copy_us[lb[k]], "vs_copy": copy_us[lb[k]] / us}
    us_layer = sum(kernels[k]["us"] for k in W.LAYER_KERNELS)
    log(f"layer done: {us_layer:.1f} us summed kernel time, {step_ms * 1e3:.1f} us per step")
    qk_bytes = lb["rope_q"] + lb["rope_k"] - 4 * cfg.T
    fused_qk = {"entry_point": "ng_rope_qk_with_theta", "rope_qk_us": per["rope_qk"],
                "rope_qk_GBps": qk_bytes / per["rope_qk"] / 1e3,
                "us_per_layer": us_layer - per["rope_q"] - per["rope_k"] + per["rope_qk"],
                "note": "Q and K rotated in one launch; the engine's own sequence (the headline) calls "
                        "cuda_rope_with_theta twice"}
    # Steady state with this library's fused entry points: the residual add
    # that ends layer L and the RMSNorm that starts layer L+1 are one
    # cuda_add_rmsnorm, and Q and K rotate in one launch. Needs call-site
    # changes in the engine, so it is reported beside the headline.
    fused_layer = fused_layer_report(cfg, per, seq)
    engine_int8 = engine_int8_report(cfg, per, seq) if cfg.dtype != "bf16" else None

    extra = {}
    if not args.no_extra:
        for key in ("mistral7b_decode", "llama2_13b_prefill", "mistral_nemo_bf16"):
            log(f"layer {key}")
            c2 = W.CONFIGS[key]
            s2, _, p2, _, _, seq2 = run_layer(L, hip, stream, c2, 20, 3)
            lb2 = W.layer_bytes(c2)
            b2 = sum(lb2[k] for k in W.LAYER_KERNELS)
            u2 = sum(p2[k] for k in W.LAYER_KERNELS)
            cu2 = copy_times(hip, stream, [lb2[k] for k in W.LAYER_KERNELS])
            extra[key] = {"us_per_layer": u2, "us_per_step": s2 * 1e3, "GBps": b2 / u2 / 1e3,
                          "frac": b2 / u2 / 1e3 / PEAK_GBPS, "layer_bytes": b2, "per_kernel_us": p2,
                          "per_kernel_copy_us": {k: cu2[lb2[k]] for k in W.LAYER_KERNELS},
                          "fused_layer_variant": fused_layer_report(c2, p2, seq2)}
            if c2.dtype == "bf16":
                eb = engine_bf16_bytes(c2)
                eu = seq2["engine_bf16_step_ms"] * 1e3
                ebk = engine_unfused_kernel_bytes(c2)
                extra[key]["engine_bf16_unfused"] = {
                    "us_per_step": eu, "layer_bytes": eb,
                    "kernels": {k: {"us": u, "bytes": ebk[k], "frac": ebk[k] / u / 1e3 / PEAK_GBPS}
                                for k, u in seq2["engine_bf16_kernels_us"].items()},
                    "sequence": ["copy residual", "rmsnorm", "rope_q", "rope_k", "add", "copy residual",
                                 "rmsnorm (in place)", "silu (in place)", "mul (in place)", "add"],
                    "note": "the bf16 engine's own sequence (layer.cu:1497-1615: two device copies, RMSNorm, "
                            "RoPE Q and K, add, RMSNorm, SiLU, mul, add); us_per_step of this layer above uses "
                            "the fused ng_bf16_add_rmsnorm and ng_bf16_silu_mul instead, which need a call-site "
                            "change in the engine (layer.cu:1584-1607)"}
        log("gather / rmsnorm+int8 / dequant")
        extra.update(extra_kernels(L, hip, stream))
        log("access-pattern floors")
        extra["floors"] = floor_extras(hip, stream)
        sized = [v for v in extra.values() if isinstance(v, dict) and "bytes" in v and "us" in v]
        xc = copy_times(hip, stream, [v["bytes"] for v in sized])
        for v in sized:
            v["copy_us"], v["vs_copy"] = xc[v["bytes"]], xc[v["bytes"]] / v["us"]

    dom = "silu_mul"
    roof = {"kernel": "cuda_silu_mul (ng::ew_vec_kernel<_Float16, EW_SILU_MUL, 1>)", "bound": "hbm",
            "achieved": kernels[dom]["GBps"], "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": kernels[dom]["GBps"] / PEAK_GBPS, "traffic": load_traffic(),
            "traffic_source": f"{TRAFFIC_FILE.relative_to(ROOT)}: FETCH_SIZE and WRITE_SIZE per dispatch from "
                              "rocprofv3 --pmc runs of bench.py --profile-pass, scaled by a 256 MiB copy; read "
                              "from the committed profile, not measured by this run",
            "algorithmic_bytes_per_launch": lb[dom], "avg_launch_us": kernels[dom]["us"]}

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(cfg, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": layer_bytes / (step_ms * 1e-3) / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
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
        "fused_qk_variant": fused_qk,
        "fused_layer_variant": fused_layer,
        "engine_int8_layer": engine_int8,
        "pct_of_peak": layer_bytes / us_layer / 1e3 / PEAK_GBPS * 100,
        "host_wall_ms_per_step": wall_ms,
        "layer_bytes": layer_bytes,
        "per_kernel": kernels,
        "copy_note": "copy_us: a plain device-to-device hipMemcpyAsync moving the kernel's algorithmic bytes "
                     "(half read, half written), timed the same way; vs_copy = copy_us / us",
        "extra": extra,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
