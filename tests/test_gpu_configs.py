"""Every benchmark configuration at its full size, on the benchmark's own inputs.

Each layer configuration (Mistral-7B decode and prefill, Llama-2-13B prefill,
Mistral-Nemo bf16, and TinyLlama-1.1B at T = 1 and 128 in fp16) runs its six
kernels through the C ABI exactly as the engine calls them (RoPE,
add+RMSNorm and SwiGLU in place), on the seeded inputs bench.py times
(neurogrid_amd.workloads, PCG64 seed 0). The oracle recomputes every row, in
chunks of rows so that host memory stays bounded; the residual sums and the
final residual add of fp16 configurations are also checked against numpy's
float16 addition (exactly RN(a + b)), independently of the oracle.
Bars: bit-exact for RMSNorm, add+RMSNorm (both outputs), residual add,
gather, int8 codes, scales and dequant; |d| <= 1e-2 or 2 ulp for RoPE and
SwiGLU.

TinyLlama's reference golden path is fp32 on the CPU
(scripts/generate_golden.py); the GPU kernels take 16-bit data, so its shapes
(pkg/types/config.go:93-106: hidden 2048, intermediate 5632, Q [T,32,64],
K [T,4,64], theta 1e4, table [32000,2048]) run here in fp16.

The embedding gathers of the Mistral-7B, Mistral-Nemo and TinyLlama
configurations ([32000,4096] uniform ids; [131072,5120] bf16 with Zipf(1.1)
ids; [32000,2048] uniform ids) and the quantisation configuration (RMSNorm +
per-token int8 on Student-t(3) activations with x20 outlier channels; int8
[14336,4096] per-row dequant) are compared in full.

The last test captures a layer into a HIP graph, replays it three times with
eager work and output clearing in between, and checks every replay bit for bit
against the eager run.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from gpu_util import C, HipRuntime, assert_bits_equal, assert_close16, banner, dev, empty, get, ok
from neurogrid_amd import workloads as W

pytestmark = pytest.mark.gpu

LAYER_CONFIGS = ["mistral7b_decode", "mistral7b_prefill", "llama2_13b_prefill", "mistral_nemo_bf16",
                 "tinyllama_t1", "tinyllama_t128"]


def gpu_config(key):
    """The configuration as the GPU kernels run it: TinyLlama's fp32 CPU-golden
    shapes are taken in fp16, the others as they are."""
    cfg = W.CONFIGS[key]
    if cfg.dtype == "f32":
        cfg = dataclasses.replace(cfg, key=cfg.key + "_f16", dtype="f16")
    return cfg


def chunks(T, elems_per_row, budget=1 << 24):
    """Row ranges of about `budget` elements each."""
    step = max(1, budget // max(1, elems_per_row))
    return [(r0, min(T, r0 + step)) for r0 in range(0, T, step)]


def entry_points(lib, dtype):
    bf = dtype == "bf16"
    return dict(
        rms=lib.cuda_bf16_rmsnorm if bf else lib.cuda_rmsnorm,
        rope=lib.cuda_bf16_rope_with_theta if bf else lib.cuda_rope_with_theta,
        addn=lib.ng_bf16_add_rmsnorm if bf else lib.cuda_add_rmsnorm,
        swig=lib.ng_bf16_silu_mul if bf else lib.cuda_silu_mul,
        add=lib.cuda_bf16_add if bf else lib.cuda_add,
    )


def f16_add(a, b):
    """RN_f16(a + b) for fp16 bit patterns (exact: the fp32 sum of two fp16 values is exact)."""
    return (a.view(np.float16) + b.view(np.float16)).view(np.uint16)


@pytest.mark.parametrize("key", LAYER_CONFIGS)
def test_layer_configuration(lib, ora, key):
    cfg = gpu_config(key)
    banner(f"layer config {cfg.key}")
    d = W.make_layer_inputs(cfg, seed=0, with_table=False)
    T, H, I, D, dt = cfg.T, cfg.H, cfg.I, cfg.D, cfg.dtype
    e = entry_points(lib, dt)
    eps, theta = C.c_float(cfg.eps), C.c_float(cfg.theta)

    # 1. RMSNorm
    xb, wa, wf = dev(d["x"]), dev(d["w_attn"]), dev(d["w_ffn"])
    yb = empty(d["x"].nbytes)
    ok(e["rms"](yb.vp, xb.vp, wa.vp, T, H, eps), "rmsnorm")
    y = get(yb, np.uint16, (T, H))
    for r0, r1 in chunks(T, H):
        assert_bits_equal(y[r0:r1], ora.rmsnorm(d["x"][r0:r1], d["w_attn"], cfg.eps, dt),
                          f"{cfg.key} rmsnorm rows {r0}-{r1}")
    del y
    yb.free()

    # 2-3. RoPE on Q and K, in place
    pb = dev(d["pos"])
    for name, nh in (("q", cfg.nq), ("k", cfg.nkv)):
        tb = dev(d[name])
        ok(e["rope"](tb.vp, tb.vp, pb.ip, 1, T, nh, D, 0, theta), f"rope {name}")
        got = get(tb, np.uint16, d[name].shape)
        same = 0
        for r0, r1 in chunks(T, nh * D):
            want = ora.rope(d[name][r0:r1], d["pos"][r0:r1], 0, cfg.theta, dt)
            same += assert_close16(got[r0:r1], want, dt, f"{cfg.key} rope {name} rows {r0}-{r1}") * (r1 - r0)
        assert same / T > 0.95, f"{cfg.key} rope {name}: only {same / T:.3f} bit-identical"
        tb.free()

    # 4. add + RMSNorm, in place (normed over input, residual_out over residual_in)
    rb = dev(d["residual"])
    ok(e["addn"](xb.vp, rb.vp, xb.vp, rb.vp, wf.vp, T, H, eps), "add_rmsnorm")
    normed, res_out = get(xb, np.uint16, (T, H)), get(rb, np.uint16, (T, H))
    for r0, r1 in chunks(T, H):
        yw, row = ora.add_rmsnorm(d["x"][r0:r1], d["residual"][r0:r1], d["w_ffn"], cfg.eps, dt)
        assert_bits_equal(res_out[r0:r1], row, f"{cfg.key} residual_out rows {r0}-{r1}")
        assert_bits_equal(normed[r0:r1], yw, f"{cfg.key} normed rows {r0}-{r1}")
    if dt == "f16":
        assert_bits_equal(res_out, f16_add(d["x"], d["residual"]), f"{cfg.key} residual_out vs numpy")

    # 5. SwiGLU, in place into gate
    gb, ub = dev(d["gate"]), dev(d["up"])
    ok(e["swig"](gb.vp, gb.vp, ub.vp, T * I), "silu_mul")
    act = get(gb, np.uint16, (T, I))
    for r0, r1 in chunks(T, I):
        want = ora.elementwise("silu_mul", d["gate"][r0:r1], d["up"][r0:r1], dtype=dt)
        assert_close16(act[r0:r1], want, dt, f"{cfg.key} silu_mul rows {r0}-{r1}")
    del act
    gb.free()
    ub.free()

    # 6. residual add: out = down + residual_out
    db, ob = dev(d["x"]), empty(d["x"].nbytes)
    ok(e["add"](ob.vp, db.vp, rb.vp, T * H), "add")
    out = get(ob, np.uint16, (T, H))
    for r0, r1 in chunks(T, H):
        assert_bits_equal(out[r0:r1], ora.elementwise("add", d["x"][r0:r1], res_out[r0:r1], dtype=dt),
                          f"{cfg.key} residual add rows {r0}-{r1}")
    if dt == "f16":
        assert_bits_equal(out, f16_add(d["x"], res_out), f"{cfg.key} residual add vs numpy")


def _pattern_table(V, H, seed):
    """A [V, H] table of 16-bit patterns (a gather copies bits, so any values do)."""
    out = np.empty((V, H), np.uint16)
    step = max(1, (1 << 24) // H)
    for r0 in range(0, V, step):
        r1 = min(V, r0 + step)
        i = np.arange(r0 * H, r1 * H, dtype=np.uint64).reshape(r1 - r0, H)
        out[r0:r1] = ((i * np.uint64(2654435761) + np.uint64(seed)) >> np.uint64(13)).astype(np.uint16)
    return out


@pytest.mark.parametrize("key", ["mistral7b_prefill", "mistral_nemo_bf16", "tinyllama_t1", "tinyllama_t128"])
def test_gather_configuration(lib, key):
    cfg = gpu_config(key)
    banner(f"gather config {key}: table [{cfg.vocab},{cfg.H}], {cfg.ids} ids")
    rng = np.random.Generator(np.random.PCG64(0))
    if cfg.ids.startswith("zipf"):
        ids = W.zipf_ids(rng, cfg.T, cfg.vocab, float(cfg.ids.split(":")[1]))
        assert np.bincount(ids).max() > 1  # Zipf ids repeat
    else:
        ids = rng.integers(0, cfg.vocab, cfg.T).astype(np.int32)
    table = _pattern_table(cfg.vocab, cfg.H, 7)
    tb, ib, ob = dev(table), dev(ids), empty(2 * cfg.T * cfg.H)
    ok(lib.cuda_gather_embeddings(ob.vp, tb.vp, ib.ip, cfg.H, cfg.T), "gather")
    assert_bits_equal(get(ob, np.uint16, (cfg.T, cfg.H)), table[ids], f"{key} gather")


def test_quant_configuration(lib, ora):
    banner("quant config: rmsnorm+int8 [4096,4096] Student-t(3) with outliers; dequant [14336,4096]")
    q = W.make_quant_inputs(seed=0)
    T, H = q["x"].shape
    xb, wb, qb, sb = dev(q["x"]), dev(q["w"]), empty(q["x"].size), empty(4 * T)
    ok(lib.ng_rmsnorm_quant_int8(qb.vp, sb.vp, xb.vp, wb.vp, T, H, C.c_float(1e-5)), "norm+int8")
    qw, sw = ora.rmsnorm_quant(q["x"], q["w"], 1e-5)
    assert_bits_equal(get(sb, np.float32, (T,)).view(np.uint32), sw.view(np.uint32), "scales")
    codes = get(qb, np.int8, (T, H))
    assert_bits_equal(codes, qw, "codes")
    # the outlier channels dominate the row maxima: the largest |code| sits on one of them in most rows
    top = np.abs(codes.astype(np.int32)).argmax(axis=1)
    assert np.isin(top, q["outlier_channels"]).mean() > 0.5
    assert (np.abs(codes.astype(np.int32)).max(axis=1) == 127).all()

    N, K = q["wq"].shape
    wqb, wsb, wob = dev(q["wq"]), dev(q["wscale"]), empty(2 * N * K)
    ok(lib.cuda_dequantize_weights(wob.vp, wqb.vp, wsb.vp, N, K, 1), "dequant")
    assert_bits_equal(get(wob, np.uint16, (N, K)), ora.dequant(q["wq"], q["wscale"], "row"), "dequant")


def test_layer_graph_replay(lib):
    """The decode layer captured into a HIP graph on the library's stream,
    replayed three times: every replay equals the eager run bit for bit."""
    cfg = W.CONFIGS["mistral7b_decode"]
    banner("graph capture of the decode layer")
    d = W.make_layer_inputs(cfg, seed=0, with_table=False)
    T, H, I, D = cfg.T, cfg.H, cfg.I, cfg.D
    eps, theta = C.c_float(cfg.eps), C.c_float(cfg.theta)
    x, res, wa, wf, pos = dev(d["x"]), dev(d["residual"]), dev(d["w_attn"]), dev(d["w_ffn"]), dev(d["pos"])
    q, k, g, u = dev(d["q"]), dev(d["k"]), dev(d["gate"]), dev(d["up"])
    outs = dict(normed=empty(d["x"].nbytes), q=empty(d["q"].nbytes), k=empty(d["k"].nbytes),
                h2=empty(d["x"].nbytes), ro=empty(d["x"].nbytes), act=empty(d["gate"].nbytes),
                out=empty(d["x"].nbytes))
    shapes = dict(normed=(T, H), q=d["q"].shape, k=d["k"].shape, h2=(T, H), ro=(T, H), act=(T, I), out=(T, H))

    def layer():
        # Out of place throughout, so that a replay recomputes the same values.
        ok(lib.cuda_rmsnorm(outs["normed"].vp, x.vp, wa.vp, T, H, eps))
        ok(lib.cuda_rope_with_theta(outs["q"].vp, q.vp, pos.ip, 1, T, cfg.nq, D, 0, theta))
        ok(lib.cuda_rope_with_theta(outs["k"].vp, k.vp, pos.ip, 1, T, cfg.nkv, D, 0, theta))
        ok(lib.cuda_add_rmsnorm(outs["h2"].vp, outs["ro"].vp, x.vp, res.vp, wf.vp, T, H, eps))
        ok(lib.cuda_silu_mul(outs["act"].vp, g.vp, u.vp, T * I))
        ok(lib.cuda_add(outs["out"].vp, x.vp, outs["ro"].vp, T * H))

    def snapshot():
        return {n: get(b, np.uint16, shapes[n]) for n, b in outs.items()}

    def clear():
        for n, b in outs.items():
            b.upload(np.zeros(shapes[n], np.uint16))

    layer()
    eager = snapshot()
    hip = HipRuntime()
    stream = hip.stream()
    lib.ng_set_stream(stream)
    try:
        graph, ex = hip.capture(stream, layer)
        try:
            for rep in range(3):
                clear()
                # unrelated eager work on the same stream between replays
                scratch = empty(d["x"].nbytes)
                ok(lib.cuda_add(scratch.vp, x.vp, res.vp, T * H))
                hip.check(hip.h.hipStreamSynchronize(stream), "hipStreamSynchronize")
                scratch.free()
                hip.launch(ex, stream)
                got = snapshot()
                for n in outs:
                    assert_bits_equal(got[n], eager[n], f"replay {rep}: {n}")
        finally:
            hip.destroy(graph, ex)
    finally:
        lib.ng_set_stream(None)
        hip.h.hipStreamDestroy(stream)
