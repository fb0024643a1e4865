"""The fp16 INT8 engine layer's memory-bound sequence against the fused entry
points that replace it at its call site.

gpu/engine/layer.cu:458-598 (cuda_layer_forward): residual = copy(input);
normed = rmsnorm(input); ... normed = o_proj(attn); normed = add(normed,
residual) in place; residual = copy(normed); normed = rmsnorm(normed) in place;
... gate = silu(gate) in place; gate = mul(gate, up) in place; ...
output = add(down, residual). The replacement drops the first copy (the input
is the residual), makes add + copy + rmsnorm one
cuda_add_rmsnorm(normed, residual, normed, input, w) in place on normed, and
silu + mul one cuda_silu_mul(gate, gate, up); the other calls stay.

- residual: bit-exact (both are fp16(o_proj + input));
- normed: within the fp16 bar. The fused kernel takes the sum of squares over
  the fp32 sums before rounding (kernels.cu:216-233), the two-call sequence
  over the rounded fp16 sums; the row scale differs by far less than an fp16
  ulp, so a few elements land on the other side of a rounding boundary;
- SwiGLU: within the bar (one rounding of silu(g)·u instead of two);
- the whole six-kernel memory-bound sequence, run both ways on the same
  inputs, ends with layer outputs within the bar of each other.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, assert_close16, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(29))


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("T,H", [(1, 4096), (64, 4096), (4096, 4096), (300, 5120), (7, 4100)])
def test_add_rmsnorm_call_site(lib, T, H):
    banner(f"int8 layer call site add+rmsnorm T={T} H={H}")
    eps = C.c_float(1e-5)
    x_in = f16(RNG.standard_normal((T, H)) * 2)         # the layer's input (hidden states)
    attn = f16(RNG.standard_normal((T, H)))             # o_proj output, in `normed`
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    wb = dev(w)

    # The engine's sequence (layer.cu:458-459, 559-570).
    inp, normed, residual = dev(x_in), dev(attn), dev(x_in)          # residual = copy(input)
    ok(lib.cuda_add(normed.vp, normed.vp, residual.vp, T * H), "cuda_add")
    summed = get(normed, np.uint16, (T, H))
    residual.upload(summed)                                          # residual = copy(normed)
    ok(lib.cuda_rmsnorm(normed.vp, normed.vp, wb.vp, T, H, eps), "cuda_rmsnorm")
    want_norm, want_res = get(normed, np.uint16, (T, H)), get(residual, np.uint16, (T, H))

    # The fused replacement: no copies, input read directly.
    normed2, residual2 = dev(attn), empty(2 * T * H)
    ok(lib.cuda_add_rmsnorm(normed2.vp, residual2.vp, normed2.vp, inp.vp, wb.vp, T, H, eps), "cuda_add_rmsnorm")
    assert_bits_equal(get(residual2, np.uint16, (T, H)), want_res, "residual")
    same = assert_close16(get(normed2, np.uint16, (T, H)), want_norm, "f16", "normed")
    assert same > 0.97, f"only {same:.4f} of normed bit-identical"
    assert_bits_equal(get(inp, np.uint16, (T, H)), x_in, "input untouched")


@pytest.mark.parametrize("n", [14336, 4096 * 14336, 1000003])
def test_silu_mul_call_site(lib, n):
    banner(f"int8 layer call site silu*mul n={n}")
    g = f16(RNG.standard_normal(n) * 3)
    u = f16(RNG.standard_normal(n))
    gate, up = dev(g), dev(u)
    ok(lib.cuda_silu(gate.vp, gate.vp, n), "cuda_silu")
    ok(lib.cuda_mul(gate.vp, gate.vp, up.vp, n), "cuda_mul")
    want = get(gate, np.uint16, (n,))
    gate2 = dev(g)
    ok(lib.cuda_silu_mul(gate2.vp, gate2.vp, up.vp, n), "cuda_silu_mul")
    same = assert_close16(get(gate2, np.uint16, (n,)), want, "f16", "silu_mul")
    print(f"silu_mul: {same:.4f} of elements bit-identical to the two-call sequence", flush=True)


@pytest.mark.parametrize("T", [64, 512])
def test_layer_sequence_side_by_side(lib, T):
    """The memory-bound calls of cuda_layer_forward at Mistral-7B shapes, unfused
    as the engine makes them and with the call-site change, on the same inputs;
    the GEMM and attention outputs they consume are given (o_proj, gate, up,
    down). Q and K, rotated by the same calls both ways, match bit for bit; the
    normed FFN input, the SwiGLU output and the layer output within the fp16 bar."""
    banner(f"int8 layer memory-bound sequence side by side T={T}")
    H, I, NQ, NKV, D = 4096, 14336, 32, 8, 128
    eps, theta = C.c_float(1e-5), C.c_float(1e6)
    x_in = f16(RNG.standard_normal((T, H)))
    o_out = f16(RNG.standard_normal((T, H)))
    g, u = f16(RNG.standard_normal((T, I))), f16(RNG.standard_normal((T, I)))
    down = f16(RNG.standard_normal((T, H)))
    q0, k0 = f16(RNG.standard_normal((T, NQ, D))), f16(RNG.standard_normal((T, NKV, D)))
    w_attn, w_ffn = f16(1 + 0.02 * RNG.standard_normal(H)), f16(1 + 0.02 * RNG.standard_normal(H))
    pos = dev(RNG.integers(0, 4096, T).astype(np.int32))
    ip = C.cast(C.c_void_p(pos.ptr), C.POINTER(C.c_int))
    wa, wf, inp, upb = dev(w_attn), dev(w_ffn), dev(x_in), dev(u)

    def run(fused: bool):
        normed, q, k = empty(2 * T * H), dev(q0), dev(k0)
        attn, gate, dn, out = dev(o_out), dev(g), dev(down), empty(2 * T * H)
        residual = empty(2 * T * H)
        if not fused:
            residual.upload(x_in)                                        # copy residual <- input
        ok(lib.cuda_rmsnorm(normed.vp, inp.vp, wa.vp, T, H, eps))
        ok(lib.cuda_rope_with_theta(q.vp, q.vp, ip, 1, T, NQ, D, 0, theta))
        ok(lib.cuda_rope_with_theta(k.vp, k.vp, ip, 1, T, NKV, D, 0, theta))
        if fused:
            ok(lib.cuda_add_rmsnorm(attn.vp, residual.vp, attn.vp, inp.vp, wf.vp, T, H, eps))
            ok(lib.cuda_silu_mul(gate.vp, gate.vp, upb.vp, T * I))
        else:
            ok(lib.cuda_add(attn.vp, attn.vp, residual.vp, T * H))
            residual.upload(get(attn, np.uint16, (T, H)))                # copy residual <- sum
            ok(lib.cuda_rmsnorm(attn.vp, attn.vp, wf.vp, T, H, eps))
            ok(lib.cuda_silu(gate.vp, gate.vp, T * I))
            ok(lib.cuda_mul(gate.vp, gate.vp, upb.vp, T * I))
        ok(lib.cuda_add(out.vp, dn.vp, residual.vp, T * H))
        return {n: get(b, np.uint16, shape) for n, b, shape in
                (("normed", normed, (T, H)), ("q", q, q0.shape), ("k", k, k0.shape), ("ffn_in", attn, (T, H)),
                 ("swiglu", gate, (T, I)), ("residual", residual, (T, H)), ("out", out, (T, H)))}

    a, b = run(False), run(True)
    for n in ("normed", "q", "k", "residual", "out"):
        assert_bits_equal(b[n], a[n], n)
    assert_close16(b["ffn_in"], a["ffn_in"], "f16", "ffn_in")
    assert_close16(b["swiglu"], a["swiglu"], "f16", "swiglu")
