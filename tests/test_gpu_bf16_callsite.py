"""The bf16 engine's residual + FFN sequence against the fused entry points
that replace it at its call site.

gpu/engine/layer.cu:1497-1500,1583-1596,1604-1607: residual = copy(input);
normed = bf16_add(normed, residual); residual = copy(normed);
normed = bf16_rmsnorm(normed) in place; gate = bf16_silu(gate) in place;
gate = bf16_mul(gate, up) in place. The replacement is one
ng_bf16_add_rmsnorm(normed, residual, normed, input, w) in place on normed,
and one ng_bf16_silu_mul(gate, gate, up).

- residual: bit-exact (both are bf16(normed + input));
- normed: within the bf16 bar. The fused kernel takes the sum of squares over
  the fp32 sums before rounding, as cuda_add_rmsnorm does (kernels.cu:216-233),
  the two-call sequence over the rounded bf16 sums; the row scale differs by
  far less than a bf16 ulp, so a few elements land on the other side of a
  rounding boundary;
- SwiGLU: within the bar (one rounding of silu(g)·u instead of two).
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, assert_close16, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(23))


def bf16(x):
    from oracle.oracle import f32_to_bf16_bits

    return f32_to_bf16_bits(np.asarray(x, np.float32))


@pytest.mark.parametrize("T,H", [(1, 5120), (64, 5120), (2048, 5120), (300, 4096), (7, 4100)])
def test_add_rmsnorm_call_site(lib, T, H):
    banner(f"bf16 call site add+rmsnorm T={T} H={H}")
    eps = C.c_float(1e-5)
    x_in = bf16(RNG.standard_normal((T, H)) * 2)        # the layer's input (hidden states)
    attn = bf16(RNG.standard_normal((T, H)))            # o_proj output, in `normed`
    w = bf16(1 + 0.02 * RNG.standard_normal(H))
    wb = dev(w)

    # The engine's sequence.
    inp, normed, residual = dev(x_in), dev(attn), dev(x_in)          # residual = copy(input)
    ok(lib.cuda_bf16_add(normed.vp, normed.vp, residual.vp, T * H), "cuda_bf16_add")
    summed = get(normed, np.uint16, (T, H))
    residual.upload(summed)                                          # residual = copy(normed)
    ok(lib.cuda_bf16_rmsnorm(normed.vp, normed.vp, wb.vp, T, H, eps), "cuda_bf16_rmsnorm")
    want_norm, want_res = get(normed, np.uint16, (T, H)), get(residual, np.uint16, (T, H))

    # The fused replacement: no copies, input read directly.
    normed2, residual2 = dev(attn), empty(2 * T * H)
    ok(lib.ng_bf16_add_rmsnorm(normed2.vp, residual2.vp, normed2.vp, inp.vp, wb.vp, T, H, eps),
       "ng_bf16_add_rmsnorm")
    assert_bits_equal(get(residual2, np.uint16, (T, H)), want_res, "residual")
    same = assert_close16(get(normed2, np.uint16, (T, H)), want_norm, "bf16", "normed")
    assert same > 0.97, f"only {same:.4f} of normed bit-identical"
    assert_bits_equal(get(inp, np.uint16, (T, H)), x_in, "input untouched")


@pytest.mark.parametrize("n", [14336, 2048 * 14336, 1000003])
def test_silu_mul_call_site(lib, n):
    banner(f"bf16 call site silu*mul n={n}")
    g = bf16(RNG.standard_normal(n) * 3)
    u = bf16(RNG.standard_normal(n))
    gate, up = dev(g), dev(u)
    ok(lib.cuda_bf16_silu(gate.vp, gate.vp, n), "cuda_bf16_silu")
    ok(lib.cuda_bf16_mul(gate.vp, gate.vp, up.vp, n), "cuda_bf16_mul")
    want = get(gate, np.uint16, (n,))
    gate2 = dev(g)
    ok(lib.ng_bf16_silu_mul(gate2.vp, gate2.vp, up.vp, n), "ng_bf16_silu_mul")
    same = assert_close16(get(gate2, np.uint16, (n,)), want, "bf16", "silu_mul")
    print(f"silu_mul: {same:.4f} of elements bit-identical to the two-call sequence", flush=True)
